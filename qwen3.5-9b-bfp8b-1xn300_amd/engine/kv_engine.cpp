// kv_engine.cpp -- engine-side mirror of the reference's KV-cache path over
// the libkvc C ABI (see kv_engine.h for what is real and what is synthetic).
#include "kv_engine.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <atomic>
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

// One conversation: a libkvc sequence (its length is g_pos, src/engine.cpp:70)
// with the token history the reference keeps in g_cached_tokens (:97).
struct Session {
    bool live = false;
    int32_t seq = -1;
    std::vector<int> cached_tokens;
    uint64_t out_digest = 0;  // hash of the last processed token's layer outputs (sampling state)
    int last_prefix = 0;
    std::vector<StepOutput> steps;
};

// engine globals (the reference's cache arrays at src/engine.cpp:81-94 live in
// the libkvc context)
bool g_loaded = false;
EngineConfig g_opts;  // set_engine_config(): applies at the next load
EngineConfig g_cfg;   // the loaded engine's options
int g_max_ctx = 0;
kvc_ctx* g_ctx = nullptr;
std::vector<Session> g_sessions;
double g_last_prefill_ms = 0.0;
int g_mismatches = 0;
int g_checks = 0;
std::atomic<int> g_hang_layer{-1};
std::atomic<int> g_hang_op{0};
// recurrent-state hash at each processed boundary, keyed by a hash of the tokens before it
std::unordered_map<uint64_t, uint64_t> g_boundary_state;
// device weights and staging for one prefill batch (bf16 bits unless noted)
float* d_norm_w = nullptr;  // fp32 [n_attn][2][256]: q_norm, k_norm
float* d_ssm_w = nullptr;   // fp32 [n_ssm][kSsmW]
uint16_t *d_qkv = nullptr, *d_q = nullptr, *d_gate = nullptr, *d_out = nullptr;
uint16_t *d_ssm_in = nullptr, *d_ssm_out = nullptr;
const std::vector<int> kNoTokens;
const std::vector<StepOutput> kNoSteps;

void mark(int layer, int op) {
    g_hang_layer.store(layer, std::memory_order_relaxed);
    g_hang_op.store(op, std::memory_order_relaxed);
}

Session* session_at(int id) {
    if (!g_loaded || id < 0 || id >= (int)g_sessions.size() || !g_sessions[id].live) return nullptr;
    return &g_sessions[id];
}

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

// hash of every recurrent layer's state (rec + conv) of a sequence
bool state_hash(int32_t seq, uint64_t* out) {
    std::vector<float> rec((size_t)kSsmVHeads * kSsmDv * kSsmDk), conv((size_t)3 * kSsmC);
    uint64_t h = 0x73746174ULL;
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) {
        void *r = nullptr, *c = nullptr;
        mark(l, 3);
        if (!kvc_ok(kvc_state_ptrs(g_ctx, seq, l, &r, &c), "kvc_state_ptrs") ||
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
int sample_token(const Session& ss, int last_token, int pos, float temperature) {
    uint64_t h = mix64(g_cfg.seed ^ ((uint64_t)(uint32_t)last_token << 17) ^ (uint64_t)pos ^ ss.out_digest);
    if (temperature > 0.f) h = mix64(h ^ 0x7E3Du);
    return (int)(mix64(h) % (uint64_t)kVocab);
}

// Tokens [pos0, pos0 + n) of `tok` (the tokens before pos0 are the session's
// cached tokens) through every layer.  Attention layers: producer + append
// (kvc_qkv_append), then the batched prefill attention for n >= 2
// (src/engine.cpp:2843-2929) or decode attention for n == 1 (:3478-3564).
// Gated-DeltaNet layers: the layer step on the live recurrent state.
bool process_tokens(Session& ss, const int* tok, int n, int pos0) {
    if (!kvc_ok(kvc_seq_reserve(g_ctx, &ss.seq, 1, n, nullptr), "kvc_seq_reserve")) return false;
    const bool keep = g_cfg.keep_outputs;
    const size_t first_step = ss.steps.size();
    for (int i = 0; i < n; i++) {
        StepOutput so;
        so.pos = pos0 + i;
        so.token = tok[i];
        so.from_prefill = n >= 2;
        so.digest = 0x73746570ULL;
        if (keep) {
            so.out.resize(g_cfg.n_attn_layers);
            so.ssm_out.resize(g_cfg.n_ssm_layers);
            if (n == 1) {
                so.q.resize(g_cfg.n_attn_layers);
                so.gate.resize(g_cfg.n_attn_layers);
            }
        }
        ss.steps.push_back(std::move(so));
    }
    uint64_t digest = 0x6F7574ULL;
    std::vector<uint16_t> rows((size_t)n * std::max(kQkvRow, kSsmRow)), out((size_t)n * kQRow);
    for (int layer = 0; layer < g_cfg.n_attn_layers; layer++) {
        for (int i = 0; i < n; i++)
            normal_bf16(projection_key(layer, tok[i], pos0 + i, 0), &rows[(size_t)i * kQkvRow], kQkvRow);
        mark(layer, 4);
        if (!hip_ok(hipMemcpy(d_qkv, rows.data(), (size_t)n * kQkvRow * 2, hipMemcpyHostToDevice), "upload qkv"))
            return false;
        const float* nw = d_norm_w + (size_t)layer * 2 * kHeadDim;
        if (!kvc_ok(kvc_qkv_append(g_ctx, layer, &ss.seq, 1, n, d_qkv, KVC_DTYPE_BF16, nw, nw + kHeadDim, d_q, d_gate,
                                   nullptr),
                    "kvc_qkv_append"))
            return false;
        const int rc = n >= 2 ? kvc_prefill_attn(g_ctx, layer, &ss.seq, 1, n, d_q, d_gate, d_out, KVC_DTYPE_BF16,
                                                 kAttnScale, nullptr)
                              : kvc_decode_attn(g_ctx, layer, &ss.seq, 1, d_q, nullptr, nullptr, d_gate, d_out,
                                                KVC_DTYPE_BF16, kAttnScale, nullptr);
        if (!kvc_ok(rc, n >= 2 ? "kvc_prefill_attn" : "kvc_decode_attn")) return false;
        mark(layer, 1);
        if (!hip_ok(hipMemcpy(out.data(), d_out, out.size() * 2, hipMemcpyDeviceToHost), "download out")) return false;
        digest = hash_bytes(&out[(size_t)(n - 1) * kQRow], kQRow * 2, digest);
        for (int i = 0; i < n; i++) {
            StepOutput& so = ss.steps[first_step + i];
            so.digest = hash_bytes(&out[(size_t)i * kQRow], kQRow * 2, so.digest);
            if (keep) so.out[layer].assign(out.begin() + (size_t)i * kQRow, out.begin() + (size_t)(i + 1) * kQRow);
        }
        if (keep && n == 1) {
            StepOutput& so = ss.steps[first_step];
            so.q[layer].resize(kQRow);
            so.gate[layer].resize(kQRow);
            if (!hip_ok(hipMemcpy(so.q[layer].data(), d_q, kQRow * 2, hipMemcpyDeviceToHost), "download q") ||
                !hip_ok(hipMemcpy(so.gate[layer].data(), d_gate, kQRow * 2, hipMemcpyDeviceToHost), "download gate"))
                return false;
        }
    }
    std::vector<uint16_t> sout((size_t)n * kSsmOut);
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) {
        for (int i = 0; i < n; i++)
            normal_bf16(projection_key(1000 + l, tok[i], pos0 + i, 4), &rows[(size_t)i * kSsmRow], kSsmRow);
        mark(1000 + l, 4);
        if (!hip_ok(hipMemcpy(d_ssm_in, rows.data(), (size_t)n * kSsmRow * 2, hipMemcpyHostToDevice), "upload ssm"))
            return false;
        const float* w = d_ssm_w + (size_t)l * kSsmW;
        if (!kvc_ok(kvc_deltanet_step(g_ctx, l, &ss.seq, 1, n, d_ssm_in, KVC_DTYPE_BF16, w, w + 4 * kSsmC,
                                      w + 4 * kSsmC + kSsmVHeads, w + 4 * kSsmC + 2 * kSsmVHeads, d_ssm_out,
                                      KVC_DTYPE_BF16, nullptr),
                    "kvc_deltanet_step"))
            return false;
        mark(l, 2);
        if (!hip_ok(hipMemcpy(sout.data(), d_ssm_out, sout.size() * 2, hipMemcpyDeviceToHost), "download ssm out"))
            return false;
        digest = hash_bytes(&sout[(size_t)(n - 1) * kSsmOut], kSsmOut * 2, digest);
        for (int i = 0; i < n; i++) {
            StepOutput& so = ss.steps[first_step + i];
            so.digest = hash_bytes(&sout[(size_t)i * kSsmOut], kSsmOut * 2, so.digest);
            if (keep) so.ssm_out[l].assign(sout.begin() + (size_t)i * kSsmOut, sout.begin() + (size_t)(i + 1) * kSsmOut);
        }
    }
    ss.out_digest = digest;
    std::vector<int32_t> t32(tok, tok + n);
    if (!kvc_ok(kvc_seq_commit(g_ctx, &ss.seq, 1, n, t32.data(), nullptr), "kvc_seq_commit")) return false;
    // remember the recurrent state at a boundary the commit snapshotted
    const int end = pos0 + n;
    if (g_cfg.verify_restore && g_cfg.n_ssm_layers > 0 && end % kBoundary == 0 &&
        (int)ss.cached_tokens.size() == pos0) {
        std::vector<int> hist(ss.cached_tokens);
        hist.insert(hist.end(), tok, tok + n);
        uint64_t h = 0;
        if (!state_hash(ss.seq, &h)) return false;
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

// Context budget of a prompt (src/engine.cpp:4048-4056): it keeps its last
// max(1, ctx - min(max_tokens, ctx / 2)) tokens, so that generation has room.
int prompt_budget(int max_tokens) { return std::max(1, g_max_ctx - std::min(max_tokens, g_max_ctx / 2)); }

// The seed of a synthetic model: the config's, else a hash of its path.
uint64_t model_seed(const char* model_path) {
    if (g_opts.seed) return g_opts.seed;
    const char* p = model_path ? model_path : "";
    return hash_bytes(p, strlen(p), 0x716D6F64656CULL) | 1;
}

bool reset_one(Session& ss) {
    ss.cached_tokens.clear();
    ss.out_digest = 0;
    return kvc_ok(kvc_seq_reset(g_ctx, ss.seq), "kvc_seq_reset");
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

void set_engine_config(const EngineConfig& cfg) { g_opts = cfg; }
const EngineConfig& engine_config() { return g_loaded ? g_cfg : g_opts; }

bool load_model_and_tokenizer(const char* model_path, int max_ctx) {
    if (g_loaded) shutdown();
    if (max_ctx < 1) {
        fprintf(stderr, "load_model_and_tokenizer: context of %d tokens\n", max_ctx);
        return false;
    }
    g_cfg = g_opts;
    g_cfg.seed = model_seed(model_path);
    g_max_ctx = max_ctx;
    const int n_sessions = std::max(1, g_cfg.max_sessions);
    kvc_config kc;
    kvc_config_default(&kc);
    kc.n_attn_layers = g_cfg.n_attn_layers;
    kc.n_ssm_layers = g_cfg.n_ssm_layers;
    kc.max_seqs = n_sessions;
    kc.max_seq_len = max_ctx;
    kc.pool_blocks = g_cfg.pool_blocks;
    kc.pool_fraction = g_cfg.pool_fraction;
    kc.snapshot_interval = kBoundary;
    kc.snapshot_slots = g_cfg.n_ssm_layers > 0 ? g_cfg.snapshot_slots : 0;
    if (!kvc_ok(kvc_create(&kc, &g_ctx), "kvc_create")) return false;
    const size_t B = kPrefillBatch;
    bool ok = hip_ok(hipMalloc((void**)&d_qkv, B * kQkvRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_q, B * kQRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_gate, B * kQRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_out, B * kQRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_ssm_in, B * kSsmRow * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_ssm_out, B * kSsmOut * 2), "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_norm_w, (size_t)std::max(1, g_cfg.n_attn_layers) * 2 * kHeadDim * 4),
                     "hipMalloc") &&
              hip_ok(hipMalloc((void**)&d_ssm_w, (size_t)std::max(1, g_cfg.n_ssm_layers) * kSsmW * 4), "hipMalloc");
    std::vector<float> qn, kn, w;
    for (int l = 0; ok && l < g_cfg.n_attn_layers; l++) {
        synthetic_norm_weights(l, qn, kn);
        ok = hip_ok(hipMemcpy(d_norm_w + (size_t)l * 2 * kHeadDim, qn.data(), kHeadDim * 4, hipMemcpyHostToDevice),
                    "upload norms") &&
             hip_ok(hipMemcpy(d_norm_w + (size_t)l * 2 * kHeadDim + kHeadDim, kn.data(), kHeadDim * 4,
                              hipMemcpyHostToDevice),
                    "upload norms");
    }
    for (int l = 0; ok && l < g_cfg.n_ssm_layers; l++) {
        synthetic_ssm_weights(l, w);
        ok = hip_ok(hipMemcpy(d_ssm_w + (size_t)l * kSsmW, w.data(), (size_t)kSsmW * 4, hipMemcpyHostToDevice),
                    "upload ssm weights");
    }
    g_sessions.assign((size_t)n_sessions, Session());
    g_loaded = ok;
    // session 0 serves the reference-signature generate()
    if (!ok || create_session() != 0) {
        shutdown();
        return false;
    }
    g_boundary_state.clear();
    g_mismatches = g_checks = 0;
    mark(-1, 0);
    return true;
}

int create_session() {
    if (!g_loaded) return -1;
    for (int id = 0; id < (int)g_sessions.size(); id++) {
        Session& ss = g_sessions[id];
        if (ss.live) continue;
        ss = Session();
        if (!kvc_ok(kvc_seq_create(g_ctx, &ss.seq), "kvc_seq_create")) return -1;
        ss.live = true;
        return id;
    }
    fprintf(stderr, "create_session: all %zu sessions in use\n", g_sessions.size());
    return -1;
}

bool release_session(int session) {
    Session* ss = session_at(session);
    if (!ss) return false;
    const bool ok = kvc_ok(kvc_seq_release(g_ctx, ss->seq), "kvc_seq_release");
    *ss = Session();
    return ok;
}

bool reset_session(int session) {
    Session* ss = session_at(session);
    return ss && reset_one(*ss);
}

// src/engine.cpp:4164-4176: the reference zero-fills every cache and state
// array; here the session drops its block references (its blocks stay in the
// prefix index for later requests), and libkvc zero-fills its recurrent state
// before the next Gated-DeltaNet step unless a snapshot restore replaces it.
void reset_state() { reset_session(0); }

void shutdown() {
    free_device();
    if (g_ctx) kvc_destroy(g_ctx);
    g_ctx = nullptr;
    g_loaded = false;
    g_sessions.clear();
}

void get_hang_info(int& layer, int& op) {
    layer = g_hang_layer.load(std::memory_order_relaxed);
    op = g_hang_op.load(std::memory_order_relaxed);
}

double get_last_prefill_ms() { return g_last_prefill_ms; }

int generate(const std::vector<int>& prompt_tokens, int max_tokens, float temperature, TokenCallback cb,
             StopReason* stop_reason) {
    return generate_session(0, prompt_tokens, max_tokens, temperature, std::move(cb), stop_reason);
}

int generate_session(int session, const std::vector<int>& prompt_tokens, int max_tokens, float temperature,
                     TokenCallback cb, StopReason* stop_reason) {
    if (!g_loaded) {
        fprintf(stderr, "generate: no model loaded\n");
        return 0;
    }
    Session* sp = session_at(session);
    if (!sp) {
        fprintf(stderr, "generate: session %d is not open\n", session);
        return 0;
    }
    Session& ss = *sp;
    ss.steps.clear();

    const int budget = prompt_budget(max_tokens);
    const size_t cut = prompt_tokens.size() > (size_t)budget ? prompt_tokens.size() - (size_t)budget : 0;
    if (cut && g_cfg.verbose)
        printf("  [prompt of %zu tokens: the first %zu dropped, context %d]\n", prompt_tokens.size(), cut, g_max_ctx);
    const std::vector<int> tokens(prompt_tokens.begin() + (std::ptrdiff_t)cut, prompt_tokens.end());
    if (tokens.empty()) {
        fprintf(stderr, "generate: empty prompt\n");
        return 0;
    }

    // Prefix reuse (src/engine.cpp:4058-4080).  The reference keeps one token
    // list and reuses it only when it is a strict prefix of the prompt; the
    // library matches against every block any session has committed, at
    // 32-token block granularity and, with recurrent layers, at a state
    // snapshot boundary, and never the whole prompt (one token must run to
    // produce logits).
    if (!reset_one(ss)) return 0;
    std::vector<int32_t> t32(tokens.begin(), tokens.end());
    int32_t reuse = 0;
    if (!kvc_ok(kvc_prefix_match(g_ctx, ss.seq, t32.data(), (int32_t)t32.size(), &reuse, nullptr),
                "kvc_prefix_match"))
        return 0;
    ss.last_prefix = reuse;
    ss.cached_tokens.assign(tokens.begin(), tokens.begin() + reuse);
    // the recurrent layers resume from the restored snapshot state; with
    // verify_restore it is checked against the hash taken at that boundary
    if (g_cfg.verify_restore && reuse > 0 && g_cfg.n_ssm_layers > 0) {
        auto it = g_boundary_state.find(token_prefix_hash(tokens.data(), reuse));
        if (it != g_boundary_state.end()) {
            uint64_t h = 0;
            if (!state_hash(ss.seq, &h)) return 0;
            g_checks++;
            if (h != it->second) g_mismatches++;
        }
    }
    const int n_prompt = (int)tokens.size();
    if (reuse > 0 && g_cfg.verbose)
        printf("  [session %d: %d cached tokens reused, %d to prefill]\n", session, reuse, n_prompt - reuse);

    const auto t0 = std::chrono::high_resolution_clock::now();
    for (int at = reuse; at < n_prompt;) {
        const int batch = std::min(kPrefillBatch, n_prompt - at);
        if (!process_tokens(ss, tokens.data() + at, batch, at)) return 0;
        ss.cached_tokens.insert(ss.cached_tokens.end(), tokens.begin() + at, tokens.begin() + at + batch);
        at += batch;
    }
    int next_token = sample_token(ss, tokens.back(), n_prompt, temperature);
    g_last_prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::high_resolution_clock::now() - t0).count();
    if (g_cfg.verbose) printf("  [prefill: %.1f ms for %d tokens]\n", g_last_prefill_ms, n_prompt - reuse);

    // decode loop (src/engine.cpp:4128-4154): every emitted token is fed back
    int emitted = 0;
    StopReason why = STOP_LENGTH;
    while (emitted < max_tokens) {
        emitted++;
        if (cb && !cb(next_token, "<" + std::to_string(next_token) + ">")) {
            why = STOP_CALLBACK;
            break;
        }
        const int p = (int)ss.cached_tokens.size();
        if (p >= g_max_ctx || !process_tokens(ss, &next_token, 1, p)) break;
        ss.cached_tokens.push_back(next_token);
        next_token = sample_token(ss, next_token, p + 1, temperature);
    }
    if (stop_reason) *stop_reason = why;
    return emitted;
}

int pos(int session) {
    const Session* ss = session_at(session);
    int32_t len = 0;
    if (ss) kvc_seq_len(g_ctx, ss->seq, &len);
    return len;
}
const std::vector<int>& cached_tokens(int session) {
    const Session* ss = session_at(session);
    return ss ? ss->cached_tokens : kNoTokens;
}
int last_prefix_len(int session) {
    const Session* ss = session_at(session);
    return ss ? ss->last_prefix : 0;
}
int state_restore_mismatches() { return g_mismatches; }
int state_restore_checks() { return g_checks; }
kvc_ctx* context() { return g_ctx; }
int32_t sequence(int session) {
    const Session* ss = session_at(session);
    return ss ? ss->seq : -1;
}
const std::vector<StepOutput>& step_outputs(int session) {
    const Session* ss = session_at(session);
    return ss ? ss->steps : kNoSteps;
}

}  // namespace kvengine
