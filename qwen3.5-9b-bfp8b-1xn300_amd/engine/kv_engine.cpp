// kv_engine.cpp -- engine-side mirror of the reference's KV-cache path over
// the libkvc C ABI (see kv_engine.h for what is real and what is synthetic).
#include "kv_engine.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "../../include/kvc.h"

namespace kvengine {
namespace {

constexpr int kQHeads = 16, kKvHeads = 4, kHeadDim = 256;
constexpr int kQRow = kQHeads * kHeadDim, kKvRow = kKvHeads * kHeadDim;
constexpr float kAttnScale = 1.0f / 16.0f;  // src/model_config.h:40

// engine globals (src/engine.cpp:70, :97 and the cache arrays at :81-94)
bool g_loaded = false;
EngineConfig g_cfg;
kvc_ctx* g_ctx = nullptr;
int32_t g_seq = -1;
std::vector<int> g_cached_tokens;
double g_last_prefill_ms = 0.0;
int g_last_prefix = 0;
int g_mismatches = 0;
std::vector<uint64_t> g_digest;  // per Gated-DeltaNet layer
std::vector<StepOutput> g_steps;
// device staging for one prefill batch (bf16 bits)
uint16_t *d_q = nullptr, *d_gate = nullptr, *d_k = nullptr, *d_v = nullptr, *d_out = nullptr;

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

uint16_t f32_to_bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// n values ~ N(0,1) (Box-Muller over splitmix64 draws keyed by `key`), bf16 RNE
void normal_bf16(uint64_t key, uint16_t* dst, int n) {
    for (int i = 0; i < n; i += 2) {
        const uint64_t r = mix64(key + (uint64_t)(i / 2 + 1) * 0x9E3779B97F4A7C15ULL);
        const double u1 = ((double)(r >> 40) + 1.0) / 16777217.0;  // (0, 1]
        const double u2 = (double)(r & 0xFFFFFF) / 16777216.0;
        const double rad = std::sqrt(-2.0 * std::log(u1));
        dst[i] = f32_to_bf16_rne((float)(rad * std::cos(6.283185307179586 * u2)));
        if (i + 1 < n) dst[i + 1] = f32_to_bf16_rne((float)(rad * std::sin(6.283185307179586 * u2)));
    }
}

uint64_t projection_key(int layer, int token, int pos, int which) {
    return mix64(g_cfg.seed ^ mix64(((uint64_t)(uint32_t)layer << 40) ^ ((uint64_t)(uint32_t)token << 8) ^
                                    ((uint64_t)(uint32_t)pos << 20) ^ (uint64_t)which));
}

uint64_t digest_init(int l) { return mix64(g_cfg.seed * 0x2545F4914F6CDD1DULL + (uint64_t)l + 1); }
uint64_t digest_step(uint64_t d, int l, int token, int pos) {
    return mix64(d ^ ((uint64_t)(uint32_t)token * 0x9E3779B97F4A7C15ULL) ^ ((uint64_t)(uint32_t)pos << 32) ^
                 (uint64_t)l);
}

// write the host digests into word 0-1 of each layer's recurrent state
bool push_digests() {
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) {
        void *rec = nullptr, *conv = nullptr;
        if (!kvc_ok(kvc_state_ptrs(g_ctx, g_seq, l, &rec, &conv), "kvc_state_ptrs")) return false;
        if (!hip_ok(hipMemcpy(rec, &g_digest[l], 8, hipMemcpyHostToDevice), "state write")) return false;
    }
    return true;
}

// next token from the history and the recurrent digest (src/engine.cpp:4020-4036
// samples from the logits; here the "logits" are this digest)
int sample_token(int last_token, int pos, float temperature) {
    uint64_t h = g_cfg.seed ^ ((uint64_t)(uint32_t)last_token << 17) ^ (uint64_t)pos;
    for (uint64_t d : g_digest) h = mix64(h ^ d);
    if (temperature > 0.f) h = mix64(h ^ 0x7E3Du);
    return (int)(mix64(h) % (uint64_t)kVocab);
}

void keep_outputs(int pos0, int n, bool prefill) {
    if (!g_cfg.keep_outputs) return;
    for (int i = 0; i < n; i++) {
        StepOutput so;
        so.pos = pos0 + i;
        so.from_prefill = prefill;
        so.out.resize(g_cfg.n_attn_layers);
        g_steps.push_back(std::move(so));
    }
}

// Tokens [pos0, pos0 + n) of `tok`: append K/V and attend, every layer.  n >= 2
// takes the batched prefill path (src/engine.cpp:2843-2929), n == 1 the decode
// path with the append fused into the attention launch (:3521-3564).
bool process_tokens(const int* tok, int n, int pos0) {
    if (!kvc_ok(kvc_seq_reserve(g_ctx, &g_seq, 1, n, nullptr), "kvc_seq_reserve")) return false;
    const size_t first_step = g_steps.size();
    keep_outputs(pos0, n, n >= 2);
    std::vector<uint16_t> q((size_t)n * kQRow), gate((size_t)n * kQRow), k((size_t)n * kKvRow), v((size_t)n * kKvRow);
    std::vector<uint16_t> qi, gi, ki, vi, out((size_t)n * kQRow);
    for (int layer = 0; layer < g_cfg.n_attn_layers; layer++) {
        for (int i = 0; i < n; i++) {
            synthetic_projection(layer, tok[i], pos0 + i, qi, gi, ki, vi);
            std::copy(qi.begin(), qi.end(), q.begin() + (size_t)i * kQRow);
            std::copy(gi.begin(), gi.end(), gate.begin() + (size_t)i * kQRow);
            std::copy(ki.begin(), ki.end(), k.begin() + (size_t)i * kKvRow);
            std::copy(vi.begin(), vi.end(), v.begin() + (size_t)i * kKvRow);
        }
        if (!hip_ok(hipMemcpy(d_q, q.data(), q.size() * 2, hipMemcpyHostToDevice), "upload q") ||
            !hip_ok(hipMemcpy(d_gate, gate.data(), gate.size() * 2, hipMemcpyHostToDevice), "upload gate") ||
            !hip_ok(hipMemcpy(d_k, k.data(), k.size() * 2, hipMemcpyHostToDevice), "upload k") ||
            !hip_ok(hipMemcpy(d_v, v.data(), v.size() * 2, hipMemcpyHostToDevice), "upload v"))
            return false;
        if (n >= 2) {
            if (!kvc_ok(kvc_append(g_ctx, layer, &g_seq, 1, n, d_k, d_v, nullptr), "kvc_append") ||
                !kvc_ok(kvc_prefill_attn(g_ctx, layer, &g_seq, 1, n, d_q, d_gate, d_out, KVC_DTYPE_BF16, kAttnScale,
                                         nullptr),
                        "kvc_prefill_attn"))
                return false;
        } else if (!kvc_ok(kvc_decode_attn(g_ctx, layer, &g_seq, 1, d_q, d_k, d_v, d_gate, d_out, KVC_DTYPE_BF16,
                                           kAttnScale, nullptr),
                           "kvc_decode_attn")) {
            return false;
        }
        if (g_cfg.keep_outputs) {
            if (!hip_ok(hipMemcpy(out.data(), d_out, out.size() * 2, hipMemcpyDeviceToHost), "download out"))
                return false;
            for (int i = 0; i < n; i++)
                g_steps[first_step + i].out[layer].assign(out.begin() + (size_t)i * kQRow,
                                                          out.begin() + (size_t)(i + 1) * kQRow);
        }
    }
    // the recurrent layers advance over the same tokens; the commit below may
    // snapshot their state at a 256-token boundary
    for (int i = 0; i < n; i++)
        for (int l = 0; l < g_cfg.n_ssm_layers; l++) g_digest[l] = digest_step(g_digest[l], l, tok[i], pos0 + i);
    if (g_cfg.n_ssm_layers > 0 && !push_digests()) return false;
    std::vector<int32_t> t32(tok, tok + n);
    return kvc_ok(kvc_seq_commit(g_ctx, &g_seq, 1, n, t32.data(), nullptr), "kvc_seq_commit");
}

}  // namespace

void synthetic_projection(int layer, int token, int pos, std::vector<uint16_t>& q, std::vector<uint16_t>& gate,
                          std::vector<uint16_t>& k, std::vector<uint16_t>& v) {
    q.resize(kQRow);
    gate.resize(kQRow);
    k.resize(kKvRow);
    v.resize(kKvRow);
    normal_bf16(projection_key(layer, token, pos, 0), q.data(), kQRow);
    normal_bf16(projection_key(layer, token, pos, 1), gate.data(), kQRow);
    normal_bf16(projection_key(layer, token, pos, 2), k.data(), kKvRow);
    normal_bf16(projection_key(layer, token, pos, 3), v.data(), kKvRow);
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
    kc.snapshot_slots = cfg.n_ssm_layers > 0 ? cfg.snapshot_slots : 0;
    if (!kvc_ok(kvc_create(&kc, &g_ctx), "kvc_create")) return false;
    if (!kvc_ok(kvc_seq_create(g_ctx, &g_seq), "kvc_seq_create")) {
        shutdown();
        return false;
    }
    const size_t qbytes = (size_t)kPrefillBatch * kQRow * 2, kvbytes = (size_t)kPrefillBatch * kKvRow * 2;
    if (!hip_ok(hipMalloc((void**)&d_q, qbytes), "hipMalloc") || !hip_ok(hipMalloc((void**)&d_gate, qbytes), "hipMalloc") ||
        !hip_ok(hipMalloc((void**)&d_out, qbytes), "hipMalloc") || !hip_ok(hipMalloc((void**)&d_k, kvbytes), "hipMalloc") ||
        !hip_ok(hipMalloc((void**)&d_v, kvbytes), "hipMalloc")) {
        shutdown();
        return false;
    }
    g_loaded = true;
    reset_state();
    return true;
}

// src/engine.cpp:4164-4176: the reference zero-fills every cache and state
// array; here the sequence drops its block references (its blocks stay in the
// prefix index for later requests) and the recurrent layers restart.
void reset_state() {
    if (!g_loaded) return;
    kvc_ok(kvc_seq_reset(g_ctx, g_seq), "kvc_seq_reset");
    g_cached_tokens.clear();
    g_digest.assign(g_cfg.n_ssm_layers, 0);
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) g_digest[l] = digest_init(l);
    if (g_cfg.n_ssm_layers > 0) push_digests();
}

void shutdown() {
    for (uint16_t** p : {&d_q, &d_gate, &d_k, &d_v, &d_out})
        if (*p) {
            (void)hipFree(*p);
            *p = nullptr;
        }
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
    if (!kvc_ok(kvc_seq_reset(g_ctx, g_seq), "kvc_seq_reset")) return 0;
    std::vector<int32_t> t32(tokens.begin(), tokens.end());
    int32_t reuse = 0;
    if (!kvc_ok(kvc_prefix_match(g_ctx, g_seq, t32.data(), (int32_t)t32.size(), &reuse, nullptr), "kvc_prefix_match"))
        return 0;
    g_last_prefix = reuse;
    g_cached_tokens.assign(tokens.begin(), tokens.begin() + reuse);
    // recurrent layers resume from the restored state; check it against a
    // recomputation over the reused tokens
    for (int l = 0; l < g_cfg.n_ssm_layers; l++) {
        uint64_t want = digest_init(l);
        for (int i = 0; i < reuse; i++) want = digest_step(want, l, tokens[i], i);
        uint64_t got = want;
        if (reuse > 0) {
            void *rec = nullptr, *conv = nullptr;
            if (!kvc_ok(kvc_state_ptrs(g_ctx, g_seq, l, &rec, &conv), "kvc_state_ptrs") ||
                !hip_ok(hipMemcpy(&got, rec, 8, hipMemcpyDeviceToHost), "state read"))
                return 0;
            if (got != want) g_mismatches++;
        }
        g_digest[l] = got;
    }
    if (reuse == 0 && g_cfg.n_ssm_layers > 0 && !push_digests()) return 0;
    const int new_tokens = (int)tokens.size() - reuse;
    if (reuse > 0 && g_cfg.verbose) printf("  [prefix cache: reusing %d tokens, prefilling %d new]\n", reuse, new_tokens);

    auto t_start = std::chrono::high_resolution_clock::now();
    {
        const int n_prompt = (int)tokens.size();
        int offset = reuse;
        while (offset < n_prompt) {
            const int batch = std::min(kPrefillBatch, n_prompt - offset);
            if (!process_tokens(tokens.data() + offset, batch, offset)) return 0;
            offset += batch;
        }
    }
    int next_token = sample_token(tokens.back(), (int)tokens.size(), temperature);
    g_cached_tokens.assign(tokens.begin(), tokens.end());  // :4118
    auto t_prefill = std::chrono::high_resolution_clock::now();
    g_last_prefill_ms = std::chrono::duration<double, std::milli>(t_prefill - t_start).count();
    if (g_cfg.verbose)
        printf("  [prefill: %.1f ms for %d new tokens]\n", g_last_prefill_ms, new_tokens);

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
kvc_ctx* context() { return g_ctx; }
int32_t sequence() { return g_seq; }
const std::vector<StepOutput>& step_outputs() { return g_steps; }

}  // namespace kvengine
