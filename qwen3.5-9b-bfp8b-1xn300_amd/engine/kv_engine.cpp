// kv_engine.cpp -- engine-side mirror of the reference's KV-cache path over
// the libkvc C ABI (see kv_engine.h for what is real and what is synthetic).
#include "kv_engine.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "../../include/kvc.h"

namespace kvengine {
namespace {

constexpr int kQHeads = 16, kHeadDim = 256;
constexpr int kQRow = kQHeads * kHeadDim;
constexpr float kAttnScale = 1.0f / 16.0f;  // src/model_config.h:40
// Gated-DeltaNet shapes (src/model_config.h:25-31)
constexpr int kSsmVHeads = 32, kSsmDv = 128, kSsmDk = 128, kSsmC = 8192;
constexpr int kSsmRow = kSsmC + kSsmVHeads * kSsmDv + 2 * kSsmVHeads;  // conv in | z | alpha | beta
constexpr int kSsmOut = kSsmVHeads * kSsmDv;
constexpr int kSsmW = 4 * kSsmC + 2 * kSsmVHeads + kSsmDv;  // conv_w | dt_bias | a | norm_w (fp32)
constexpr int kBoundary = 256;                               // snapshot interval

// engine globals (src/engine.cpp:70, :97 and the cache arrays at :81-94)
bool g_loaded = false;
EngineConfig g_cfg;
kvc_ctx* g_ctx = nullptr;
int32_t g_seq = -1;
std::vector<int> g_cached_tokens;
double g_last_prefill_ms = 0.0;
int g_last_prefix = 0;
int g_mismatches = 0;
int g_checks = 0;
uint64_t g_out_digest = 0;  // hash of the last processed token's layer outputs
std::vector<StepOutput> g_steps;
// recurrent-state hash at each processed boundary, keyed by a hash of the tokens before it
std::unordered_map<uint64_t, uint64_t> g_boundary_state;
// device weights and staging for one prefill batch (bf16 bits unless noted)
float* d_norm_w = nullptr;  // fp32 [n_attn][2][256]: q_norm, k_norm
float* d_ssm_w = nullptr;   // fp32 [n_ssm][kSsmW]
uint16_t *d_qkv = nullptr, *d_q = nullptr, *d_gate = nullptr, *d_out = nullptr;
uint16_t *d_ssm_in = nullptr, *d_ssm_out = nullptr;

bool kvc_ok(int rc, const char* what) {
    if (rc == KVC_OK) return true;
    fprintf(stderr, "%s: %s\n", what, kvc_last_error());
    return false;
}
bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    return false;
}

uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t hash_bytes(const void* p, size_t n, uint64_t h) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        memcpy(&w, b + i, 8);
        h = mix64(h ^ w);
    }
    for (; i < n; i++) h = mix64(h ^ b[i]);
    return h;
}

uint16_t f32_to_bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// uniform (0, 1] and N(0,1) draws keyed by (key, i): splitmix64 + Box-Muller
double uniform01(uint64_t key, int i) {
    return ((double)(mix64(key + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ULL) >> 40) + 1.0) / 16777217.0;
}
void normal_f64(uint64_t key, double* dst, int n) {
    for (int i = 0; i < n; i += 2) {
        const uint64_t r = mix64(key + (uint64_t)(i / 2 + 1) * 0x9E3779B97F4A7C15ULL);
        const double u1 = ((double)(r >> 40) + 1.0) / 16777217.0;  // (0, 1]
        const double u2 = (double)(r & 0xFFFFFF) / 16777216.0;
        const double rad = std::sqrt(-2.0 * std::log(u1));
        dst[i] = rad * std::cos(6.283185307179586 * u2);
        if (i + 1 < n) dst[i + 1] = rad * std::sin(6.283185307179586 * u2);
    }
}
void normal_bf16(uint64_t key, uint16_t* dst, int n) {
    std::vector<double> t(n);
    normal_f64(key, t.data(), n);
    for (int i = 0; i < n; i++) dst[i] = f32_to_bf16_rne((float)t[i]);
}

uint64_t projection_key(int layer, int token, int pos, int which) {
    return mix64(g_cfg.seed ^ mix64(((uint64_t)(uint32_t)layer << 40) ^ ((uint64_t)(uint32_t)token << 8) ^
                                    ((uint64_t)(uint32_t)pos << 20) ^ (uint64_t)which));
}
uint64_t weight_key(int layer, int which) {
    return mix64(g_cfg.seed * 0x2545F4914F6CDD1DULL ^ mix64((uint64_t)layer * 16 + (uint64_t)which));
}

uint64_t token_prefix_hash(const int* tok, int n) {
    return hash_bytes(tok, (size_t)n * sizeof(int), 0x6B76656E67696E65ULL);
}

// Gated-DeltaNet layer weights (fp32): conv taps 0.5 N(0,1), dt_bias N(0,1),
// a in [-1, -0.05] (decay = exp(softplus(.) a) < 1), norm in [0.5, 1.5]
void synthetic_ssm_weights(int l, std::vector<float>& w) {
    w.resize(kSsmW);
    std::vector<double> t(4 * kSsmC + kSsmVHeads);
    normal_f64(weight_key(1000 + l, 0), t.data(), (int)t.size());
    for (int i = 0; i < 4 * kSsmC; i++) w[i] = (float)(0.5 * t[i]);
    for (int i = 0; i < kSsmVHeads; i++) w[4 * kSsmC + i] = (float)t[4 * kSsmC + i];
    for (int i = 0; i < kSsmVHeads; i++)
        w[4 * kSsmC + kSsmVHeads + i] = (float)(-0.05 - 0.95 * uniform01(weight_key(1000 + l, 1), i));
    for (int i = 0; i < kSsmDv; i++)
        w[4 * kSsmC + 2 * kSsmVHeads + i] = (float)(0.5 + uniform01(weight_key(1000 + l, 2), i));
}

// hash of every recurrent layer's state (rec + conv) of the engine's sequence
bool state_hash(uint64_t* out) {
    std::vector<float> rec((size_t)kSsmVHeads * kSsmDv * kSsmDk), conv((size_t)3 * kSsmC);
    uint64_t h = 0x73746174ULL;
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) {
        void *r = nullptr, *c = nullptr;
        if (!kvc_ok(kvc_state_ptrs(g_ctx, g_seq, l, &r, &c), "kvc_state_ptrs") ||
            !hip_ok(hipMemcpy(rec.data(), r, rec.size() * 4, hipMemcpyDeviceToHost), "state read") ||
            !hip_ok(hipMemcpy(conv.data(), c, conv.size() * 4, hipMemcpyDeviceToHost), "state read"))
            return false;
        h = hash_bytes(rec.data(), rec.size() * 4, h);
        h = hash_bytes(conv.data(), conv.size() * 4, h);
    }
    *out = h;
    return true;
}

// next token from the history and the last token's layer outputs
// (src/engine.cpp:4020-4036 samples from the logits; here the "logits" are
// those outputs)
int sample_token(int last_token, int pos, float temperature) {
    uint64_t h = mix64(g_cfg.seed ^ ((uint64_t)(uint32_t)last_token << 17) ^ (uint64_t)pos ^ g_out_digest);
    if (temperature > 0.f) h = mix64(h ^ 0x7E3Du);
    return (int)(mix64(h) % (uint64_t)kVocab);
}

// Tokens [pos0, pos0 + n) of `tok` (the tokens before pos0 are g_cached_tokens)
// through every layer.  Attention layers: producer + append (kvc_qkv_append),
// then the batched prefill attention for n >= 2 (src/engine.cpp:2843-2929) or
// decode attention for n == 1 (:3478-3564).  Gated-DeltaNet layers: the layer
// step on the live recurrent state.
bool process_tokens(const int* tok, int n, int pos0) {
    if (!kvc_ok(kvc_seq_reserve(g_ctx, &g_seq, 1, n, nullptr), "kvc_seq_reserve")) return false;
    const bool keep = g_cfg.keep_outputs;
    const size_t first_step = g_steps.size();
    if (keep) {
        for (int i = 0; i < n; i++) {
            StepOutput so;
            so.pos = pos0 + i;
            so.from_prefill = n >= 2;
            so.out.resize(g_cfg.n_attn_layers);
            so.ssm_out.resize(g_cfg.n_ssm_layers);
            if (n == 1) {
                so.q.resize(g_cfg.n_attn_layers);
                so.gate.resize(g_cfg.n_attn_layers);
            }
            g_steps.push_back(std::move(so));
        }
    }
    uint64_t digest = 0x6F7574ULL;
    std::vector<uint16_t> rows((size_t)n * std::max(kQkvRow, kSsmRow)), out((size_t)n * kQRow);
    for (int layer = 0; layer < g_cfg.n_attn_layers; layer++) {
        for (int i = 0; i < n; i++)
            normal_bf16(projection_key(layer, tok[i], pos0 + i, 0), &rows[(size_t)i * kQkvRow], kQkvRow);
        if (!hip_ok(hipMemcpy(d_qkv, rows.data(), (size_t)n * kQkvRow * 2, hipMemcpyHostToDevice), "upload qkv"))
            return false;
        const float* nw = d_norm_w + (size_t)layer * 2 * kHeadDim;
        if (!kvc_ok(kvc_qkv_append(g_ctx, layer, &g_seq, 1, n, d_qkv, KVC_DTYPE_BF16, nw, nw + kHeadDim, d_q, d_gate,
                                   nullptr),
                    "kvc_qkv_append"))
            return false;
        const int rc = n >= 2 ? kvc_prefill_attn(g_ctx, layer, &g_seq, 1, n, d_q, d_gate, d_out, KVC_DTYPE_BF16,
                                                 kAttnScale, nullptr)
                              : kvc_decode_attn(g_ctx, layer, &g_seq, 1, d_q, nullptr, nullptr, d_gate, d_out,
                                                KVC_DTYPE_BF16, kAttnScale, nullptr);
        if (!kvc_ok(rc, n >= 2 ? "kvc_prefill_attn" : "kvc_decode_attn")) return false;
        if (!hip_ok(hipMemcpy(out.data(), d_out, out.size() * 2, hipMemcpyDeviceToHost), "download out")) return false;
        digest = hash_bytes(&out[(size_t)(n - 1) * kQRow], kQRow * 2, digest);
        if (keep) {
            for (int i = 0; i < n; i++)
                g_steps[first_step + i].out[layer].assign(out.begin() + (size_t)i * kQRow,
                                                          out.begin() + (size_t)(i + 1) * kQRow);
            if (n == 1) {
                StepOutput& so = g_steps[first_step];
                so.q[layer].resize(kQRow);
                so.gate[layer].resize(kQRow);
                if (!hip_ok(hipMemcpy(so.q[layer].data(), d_q, kQRow * 2, hipMemcpyDeviceToHost), "download q") ||
                    !hip_ok(hipMemcpy(so.gate[layer].data(), d_gate, kQRow * 2, hipMemcpyDeviceToHost),
                            "download gate"))
                    return false;
            }
        }
    }
    std::vector<uint16_t> sout((size_t)n * kSsmOut);
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) {
        for (int i = 0; i < n; i++)
            normal_bf16(projection_key(1000 + l, tok[i], pos0 + i, 4), &rows[(size_t)i * kSsmRow], kSsmRow);
        if (!hip_ok(hipMemcpy(d_ssm_in, rows.data(), (size_t)n * kSsmRow * 2, hipMemcpyHostToDevice), "upload ssm"))
            return false;
        const float* w = d_ssm_w + (size_t)l * kSsmW;
        if (!kvc_ok(kvc_deltanet_step(g_ctx, l, &g_seq, 1, n, d_ssm_in, KVC_DTYPE_BF16, w, w + 4 * kSsmC,
                                      w + 4 * kSsmC + kSsmVHeads, w + 4 * kSsmC + 2 * kSsmVHeads, d_ssm_out,
                                      KVC_DTYPE_BF16, nullptr),
                    "kvc_deltanet_step"))
            return false;
        if (!hip_ok(hipMemcpy(sout.data(), d_ssm_out, sout.size() * 2, hipMemcpyDeviceToHost), "download ssm out"))
            return false;
        digest = hash_bytes(&sout[(size_t)(n - 1) * kSsmOut], kSsmOut * 2, digest);
        if (keep)
            for (int i = 0; i < n; i++)
                g_steps[first_step + i].ssm_out[l].assign(sout.begin() + (size_t)i * kSsmOut,
                                                          sout.begin() + (size_t)(i + 1) * kSsmOut);
    }
    g_out_digest = digest;
    std::vector<int32_t> t32(tok, tok + n);
    if (!kvc_ok(kvc_seq_commit(g_ctx, &g_seq, 1, n, t32.data(), nullptr), "kvc_seq_commit")) return false;
    // remember the recurrent state at a boundary the commit snapshotted
    const int end = pos0 + n;
    if (g_cfg.verify_restore && g_cfg.n_ssm_layers > 0 && end % kBoundary == 0 && (int)g_cached_tokens.size() == pos0) {
        std::vector<int> hist(g_cached_tokens);
        hist.insert(hist.end(), tok, tok + n);
        uint64_t h = 0;
        if (!state_hash(&h)) return false;
        g_boundary_state[token_prefix_hash(hist.data(), end)] = h;
    }
    return true;
}

void free_device() {
    for (uint16_t** p : {&d_qkv, &d_q, &d_gate, &d_out, &d_ssm_in, &d_ssm_out})
        if (*p) {
            (void)hipFree(*p);
            *p = nullptr;
        }
    for (float** p : {&d_norm_w, &d_ssm_w})
        if (*p) {
            (void)hipFree(*p);
            *p = nullptr;
        }
}

}  // namespace

void synthetic_qkv_row(int layer, int token, int pos, std::vector<uint16_t>& row) {
    row.resize(kQkvRow);
    normal_bf16(projection_key(layer, token, pos, 0), row.data(), kQkvRow);
}

// q_norm / k_norm weights in [0.5, 1.5]
void synthetic_norm_weights(int layer, std::vector<float>& q_norm, std::vector<float>& k_norm) {
    q_norm.resize(kHeadDim);
    k_norm.resize(kHeadDim);
    for (int i = 0; i < kHeadDim; i++) {
        q_norm[i] = (float)(0.5 + uniform01(weight_key(layer, 0), i));
        k_norm[i] = (float)(0.5 + uniform01(weight_key(layer, 1), i));
    }
}

bool load_model_and_tokenizer(const EngineConfig& cfg) {
    if (g_loaded) shutdown();
    g_cfg = cfg;
    kvc_config kc;
    kvc_config_default(&kc);
    kc.n_attn_layers = cfg.n_attn_layers;
    kc.n_ssm_layers = cfg.n_ssm_layers;
    kc.max_seqs = 4;
    kc.max_seq_len = cfg.max_ctx;
    kc.pool_blocks = cfg.pool_blocks;
    kc.pool_fraction = cfg.pool_fraction;
    kc.snapshot_interval = kBoundary;
    kc.snapshot_slots = cfg.n_ssm_layers > 0 ? cfg.snapshot_slots : 0;
    if (!kvc_ok(kvc_create(&kc, &g_ctx), "kvc_create")) return false;
    if (!kvc_ok(kvc_seq_create(g_ctx, &g_seq), "kvc_seq_create")) {
        shutdown();
        return false;
    }
    const size_t B = kPrefillBatch;
    bool ok = hip_ok(hipMalloc((void**)&d_qkv, B * kQkvRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_q, B * kQRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_gate, B * kQRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_out, B * kQRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_ssm_in, B * kSsmRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_ssm_out, B * kSsmOut * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_norm_w, (size_t)std::max(1, cfg.n_attn_layers) * 2 * kHeadDim * 4),
                     "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_ssm_w, (size_t)std::max(1, cfg.n_ssm_layers) * kSsmW * 4), "hipMalloc");
    std::vector<float> qn, kn, w;
    for (int l = 0; ok && l < cfg.n_attn_layers; l++) {
        synthetic_norm_weights(l, qn, kn);
        ok = hip_ok(hipMemcpy(d_norm_w + (size_t)l * 2 * kHeadDim, qn.data(), kHeadDim * 4, hipMemcpyHostToDevice),
                    "upload norms") &&
             hip_ok(hipMemcpy(d_norm_w + (size_t)l * 2 * kHeadDim + kHeadDim, kn.data(), kHeadDim * 4,
                              hipMemcpyHostToDevice),
                    "upload norms");
    }
    for (int l = 0; ok && l < cfg.n_ssm_layers; l++) {
        synthetic_ssm_weights(l, w);
        ok = hip_ok(hipMemcpy(d_ssm_w + (size_t)l * kSsmW, w.data(), (size_t)kSsmW * 4, hipMemcpyHostToDevice),
                    "upload ssm weights");
    }
    if (!ok) {
        shutdown();
        return false;
    }
    g_loaded = true;
    g_boundary_state.clear();
    g_mismatches = g_checks = 0;
    reset_state();
    return true;
}

// src/engine.cpp:4164-4176: the reference zero-fills every cache and state
// array; here the sequence drops its block references (its blocks stay in the
// prefix index for later requests), and libkvc zero-fills its recurrent state
// before the next Gated-DeltaNet step unless a snapshot restore replaces it.
void reset_state() {
    if (!g_loaded) return;
    kvc_ok(kvc_seq_reset(g_ctx, g_seq), "kvc_seq_reset");
    g_cached_tokens.clear();
    g_out_digest = 0;
}

void shutdown() {
    free_device();
    if (g_ctx) kvc_destroy(g_ctx);
    g_ctx = nullptr;
    g_seq = -1;
    g_loaded = false;
    g_cached_tokens.clear();
    g_steps.clear();
}

double get_last_prefill_ms() { return g_last_prefill_ms; }

int generate(const std::vector<int>& prompt_tokens, int max_tokens, float temperature, TokenCallback cb,
             StopReason* stop_reason) {
    if (!g_loaded) {
        fprintf(stderr, "Model not loaded\n");
        return 0;
    }
    g_steps.clear();
    int total_generated = 0;

    // truncate the prompt to fit the context window (src/engine.cpp:4048-4056)
    std::vector<int> tokens = prompt_tokens;
    int max_prompt = g_cfg.max_ctx - std::min(max_tokens, g_cfg.max_ctx / 2);
    if (max_prompt < 1) max_prompt = 1;
    if ((int)tokens.size() > max_prompt) {
        if (g_cfg.verbose)
            printf("  [truncating prompt from %zu to %d tokens to fit ctx=%d]\n", tokens.size(), max_prompt,
                   g_cfg.max_ctx);
        tokens.erase(tokens.begin(), tokens.begin() + ((int)tokens.size() - max_prompt));
    }
    if (tokens.empty()) {
        fprintf(stderr, "generate: empty prompt\n");
        return 0;
    }

    // prefix reuse (src/engine.cpp:4058-4080).  The reference keeps one token
    // list and reuses it only when it is a strict prefix of the prompt; the
    // library matches against every block it has cached, at 32-token block
    // granularity and, with recurrent layers, at a state snapshot boundary,
    // and never the whole prompt (one token must run to produce logits).
    reset_state();
    std::vector<int32_t> t32(tokens.begin(), tokens.end());
    int32_t reuse = 0;
    if (!kvc_ok(kvc_prefix_match(g_ctx, g_seq, t32.data(), (int32_t)t32.size(), &reuse, nullptr), "kvc_prefix_match"))
        return 0;
    g_last_prefix = reuse;
    g_cached_tokens.assign(tokens.begin(), tokens.begin() + reuse);
    // the recurrent layers resume from the restored snapshot state; with
    // verify_restore it is checked against the hash taken at that boundary
    if (g_cfg.verify_restore && reuse > 0 && g_cfg.n_ssm_layers > 0) {
        auto it = g_boundary_state.find(token_prefix_hash(tokens.data(), reuse));
        if (it != g_boundary_state.end()) {
            uint64_t h = 0;
            if (!state_hash(&h)) return 0;
            g_checks++;
            if (h != it->second) g_mismatches++;
        }
    }
    const int new_tokens = (int)tokens.size() - reuse;
    if (reuse > 0 && g_cfg.verbose) printf("  [prefix cache: reusing %d tokens, prefilling %d new]\n", reuse, new_tokens);

    auto t_start = std::chrono::high_resolution_clock::now();
    {
        const int n_prompt = (int)tokens.size();
        int offset = reuse;
        while (offset < n_prompt) {
            const int batch = std::min(kPrefillBatch, n_prompt - offset);
            if (!process_tokens(tokens.data() + offset, batch, offset)) return 0;
            g_cached_tokens.insert(g_cached_tokens.end(), tokens.begin() + offset, tokens.begin() + offset + batch);
            offset += batch;
        }
    }
    int next_token = sample_token(tokens.back(), (int)tokens.size(), temperature);
    g_cached_tokens.assign(tokens.begin(), tokens.end());  // :4118
    auto t_prefill = std::chrono::high_resolution_clock::now();
    g_last_prefill_ms = std::chrono::duration<double, std::milli>(t_prefill - t_start).count();
    if (g_cfg.verbose) printf("  [prefill: %.1f ms for %d new tokens]\n", g_last_prefill_ms, new_tokens);

    // decode loop (src/engine.cpp:4128-4154): every emitted token is fed back
    while (total_generated < max_tokens) {
        total_generated++;
        if (cb && !cb(next_token, "<" + std::to_string(next_token) + ">")) {
            if (stop_reason) *stop_reason = STOP_CALLBACK;
            return total_generated;
        }
        const int p = (int)g_cached_tokens.size();
        if (!process_tokens(&next_token, 1, p)) {
            if (stop_reason) *stop_reason = STOP_LENGTH;
            return total_generated;
        }
        g_cached_tokens.push_back(next_token);  // :4151
        next_token = sample_token(next_token, p + 1, temperature);
    }
    if (stop_reason) *stop_reason = STOP_LENGTH;
    return total_generated;
}

int pos() {
    int32_t len = 0;
    if (g_loaded) kvc_seq_len(g_ctx, g_seq, &len);
    return len;
}
const std::vector<int>& cached_tokens() { return g_cached_tokens; }
int last_prefix_len() { return g_last_prefix; }
int state_restore_mismatches() { return g_mismatches; }
int state_restore_checks() { return g_checks; }
kvc_ctx* context() { return g_ctx; }
int32_t sequence() { return g_seq; }
const std::vector<StepOutput>& step_outputs() { return g_steps; }

}  // namespace kvengine
