// Integration tests of the KV-cache path through the engine-side mirror
// (kvengine::generate / reset_state / ...), in the style of the reference's
// src/tests/test_inference.cpp: EXPECT_* macros, one function per behaviour.
// Needs a HIP device.  The parity checks load the CPU oracle
// (oracle/libkvc_oracle.so, test infrastructure) next to this binary's repo.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/kvc.h"
#include "../../qwen3.5-9b-bfp8b-1xn300_amd/engine/kv_engine.h"

static int g_failures = 0;
static int g_tests = 0;

#define EXPECT_EQ(a, b)                                                                      \
    do {                                                                                     \
        g_tests++;                                                                           \
        auto _a = (a);                                                                       \
        auto _b = (b);                                                                       \
        if (!(_a == _b)) {                                                                   \
            fprintf(stderr, "FAIL %s:%d: %s != %s\n", __FILE__, __LINE__, #a, #b);         \
            g_failures++;                                                                    \
        }                                                                                    \
    } while (0)

#define EXPECT_TRUE(x)                                                           \
    do {                                                                         \
        g_tests++;                                                               \
        if (!(x)) {                                                              \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #x);        \
            g_failures++;                                                        \
        }                                                                        \
    } while (0)

#define EXPECT_LE(a, b)                                                                          \
    do {                                                                                         \
        g_tests++;                                                                               \
        auto _a = (a);                                                                           \
        auto _b = (b);                                                                           \
        if (!(_a <= _b)) {                                                                       \
            fprintf(stderr, "FAIL %s:%d: %s = %g, expected <= %g\n", __FILE__, __LINE__, #a,   \
                    (double)_a, (double)_b);                                                     \
            g_failures++;                                                                        \
        }                                                                                        \
    } while (0)

using kvengine::EngineConfig;

// ---- CPU oracle (test infrastructure only) ---------------------------------
typedef void (*decode_fn)(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int, int, float,
                          const uint16_t*, int, float*);
static decode_fn g_orc_decode = nullptr;

static bool load_oracle() {
    char exe[PATH_MAX];
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    if (n <= 0) return false;
    exe[n] = 0;
    std::string dir(exe);
    dir = dir.substr(0, dir.rfind('/'));
    const std::string path = dir + "/../../oracle/libkvc_oracle.so";
    void* h = dlopen(path.c_str(), RTLD_NOW);
    if (!h) {
        fprintf(stderr, "cannot load the oracle %s: %s\n", path.c_str(), dlerror());
        return false;
    }
    g_orc_decode = (decode_fn)dlsym(h, "orc_decode_attn");
    return g_orc_decode != nullptr;
}

static float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static std::vector<int> random_tokens(int n, uint64_t seed) {
    std::vector<int> t(n);
    uint64_t s = seed;
    for (int i = 0; i < n; i++) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        t[i] = (int)((s >> 33) % kvengine::kVocab);
    }
    return t;
}

struct Run {
    std::vector<int> tokens;
    int n = 0;
    int reuse = 0;
    std::vector<kvengine::StepOutput> steps;
};

static Run run_generate(const std::vector<int>& prompt, int max_tokens) {
    Run r;
    kvengine::StopReason reason = kvengine::STOP_CALLBACK;
    r.n = kvengine::generate(prompt, max_tokens, 0.0f,
                             [&](int id, const std::string&) {
                                 r.tokens.push_back(id);
                                 return true;
                             },
                             &reason);
    r.reuse = kvengine::last_prefix_len();
    r.steps = kvengine::step_outputs();
    return r;
}

static bool load(int max_ctx, int n_ssm) {
    EngineConfig cfg;
    cfg.max_ctx = max_ctx;
    cfg.n_ssm_layers = n_ssm;
    cfg.pool_blocks = 2048;
    return kvengine::load_model_and_tokenizer(cfg);
}

// outputs of positions >= from agree bit for bit (same kernels, same keys)
static bool same_outputs(const Run& a, const Run& b, int from) {
    for (const auto& sa : a.steps) {
        if (sa.pos < from) continue;
        bool found = false;
        for (const auto& sb : b.steps) {
            if (sb.pos != sa.pos) continue;
            found = true;
            if (sa.out != sb.out) return false;
        }
        if (!found) return false;
    }
    return true;
}

static void test_not_loaded() {
    printf("  test_not_loaded...\n");
    kvengine::shutdown();
    EXPECT_EQ(kvengine::generate({1, 2, 3}, 4, 0.0f, nullptr), 0);
}

static void test_basic_generation() {
    printf("  test_basic_generation...\n");
    EXPECT_TRUE(load(4096, 0));
    kvengine::reset_state();
    auto prompt = random_tokens(40, 1);
    auto r = run_generate(prompt, 16);
    EXPECT_EQ(r.n, 16);
    EXPECT_EQ((int)r.tokens.size(), 16);
    // g_cached_tokens.size() == g_pos after every generate step (src/engine.cpp:4118, :4151)
    EXPECT_EQ((int)kvengine::cached_tokens().size(), 56);
    EXPECT_EQ(kvengine::pos(), 56);
    EXPECT_EQ((int)r.steps.size(), 56);
    bool finite = true;
    for (const auto& st : r.steps)
        for (const auto& o : st.out)
            for (uint16_t b : o) finite = finite && std::isfinite(bf16f(b));
    EXPECT_TRUE(finite);
}

static void test_prompt_caching() {
    printf("  test_prompt_caching...\n");
    // first request, then the conversation extended with new tokens
    EXPECT_TRUE(load(4096, 0));
    auto prompt = random_tokens(100, 2);
    auto r1 = run_generate(prompt, 8);
    std::vector<int> all_ids = prompt;
    all_ids.insert(all_ids.end(), r1.tokens.begin(), r1.tokens.end());
    auto suffix = random_tokens(5, 3);
    all_ids.insert(all_ids.end(), suffix.begin(), suffix.end());
    auto r2 = run_generate(all_ids, 8);
    // 108 cached tokens are a prefix of the 113-token prompt: 96 reused (3 blocks)
    EXPECT_EQ(r2.reuse, 96);
    EXPECT_EQ(r2.n, 8);
    // the same request on a fresh engine (nothing cached) generates the same
    // tokens and the same attention outputs for every position it recomputes
    EXPECT_TRUE(load(4096, 0));
    auto r3 = run_generate(all_ids, 8);
    EXPECT_EQ(r3.reuse, 0);
    EXPECT_TRUE(r2.tokens == r3.tokens);
    EXPECT_TRUE(same_outputs(r2, r3, 96));
}

static void test_greedy_determinism() {
    printf("  test_greedy_determinism...\n");
    EXPECT_TRUE(load(4096, 0));
    auto prompt = random_tokens(70, 4);
    kvengine::reset_state();
    auto r1 = run_generate(prompt, 16);
    kvengine::reset_state();
    auto r2 = run_generate(prompt, 16);
    EXPECT_EQ(kvengine::pos(), 86);
    // the second run reuses the cached blocks (never the whole prompt)
    EXPECT_EQ(r2.reuse, 64);
    EXPECT_TRUE(r1.tokens == r2.tokens);
    EXPECT_TRUE(same_outputs(r2, r1, 64));
}

static void test_divergent_prompt() {
    printf("  test_divergent_prompt...\n");
    // the reference resets on a divergent prompt (src/engine.cpp:4067-4071);
    // the block index still reuses the shared whole blocks
    EXPECT_TRUE(load(4096, 0));
    auto a = random_tokens(200, 5);
    run_generate(a, 4);
    std::vector<int> b(a.begin(), a.begin() + 150);
    b.push_back((a[150] + 1) % kvengine::kVocab);
    auto extra = random_tokens(20, 6);
    b.insert(b.end(), extra.begin(), extra.end());
    auto rb = run_generate(b, 8);
    EXPECT_EQ(rb.reuse, 128);
    EXPECT_TRUE(load(4096, 0));
    auto rs = run_generate(b, 8);
    EXPECT_TRUE(rb.tokens == rs.tokens);
    EXPECT_TRUE(same_outputs(rb, rs, 128));
}

static void test_context_truncation() {
    printf("  test_context_truncation...\n");
    // an over-long prompt keeps its last max_ctx - max_tokens tokens (:4048-4056)
    EXPECT_TRUE(load(512, 0));
    auto prompt = random_tokens(700, 7);
    auto r = run_generate(prompt, 64);
    EXPECT_EQ(r.n, 64);
    EXPECT_EQ(kvengine::pos(), 512);
    const auto& cached = kvengine::cached_tokens();
    EXPECT_TRUE(std::vector<int>(cached.begin(), cached.begin() + 448) ==
                std::vector<int>(prompt.end() - 448, prompt.end()));
}

static void test_attention_parity() {
    printf("  test_attention_parity...\n");
    EXPECT_TRUE(load(4096, 0));
    auto prompt = random_tokens(300, 8);
    auto r = run_generate(prompt, 4);
    const int L = kvengine::pos();  // 304 keys; the last decode step saw all of them
    const int layer = 3;
    std::vector<uint16_t> kc((size_t)L * 1024), vc((size_t)L * 1024);
    void *dk = nullptr, *dv = nullptr;
    EXPECT_EQ(hipMalloc(&dk, kc.size() * 2), hipSuccess);
    EXPECT_EQ(hipMalloc(&dv, vc.size() * 2), hipSuccess);
    int32_t seq = kvengine::sequence(), n = L;
    EXPECT_EQ(kvc_gather(kvengine::context(), layer, &seq, 1, 0, &n, dk, dv, nullptr), KVC_OK);
    EXPECT_EQ(hipMemcpy(kc.data(), dk, kc.size() * 2, hipMemcpyDeviceToHost), hipSuccess);
    EXPECT_EQ(hipMemcpy(vc.data(), dv, vc.size() * 2, hipMemcpyDeviceToHost), hipSuccess);
    EXPECT_EQ(hipFree(dk), hipSuccess);
    EXPECT_EQ(hipFree(dv), hipSuccess);
    // the cache holds exactly the appended projections (bit-exact)
    const auto& cached = kvengine::cached_tokens();
    bool exact = true;
    std::vector<uint16_t> q, g, k, v;
    for (int p = 0; p < L; p++) {
        kvengine::synthetic_projection(layer, cached[p], p, q, g, k, v);
        exact = exact && !memcmp(&kc[(size_t)p * 1024], k.data(), 2048) && !memcmp(&vc[(size_t)p * 1024], v.data(), 2048);
    }
    EXPECT_TRUE(exact);
    // the last decode step's output vs the oracle over the same cache
    if (!g_orc_decode) {
        EXPECT_TRUE(g_orc_decode != nullptr);
        return;
    }
    kvengine::synthetic_projection(layer, cached[L - 1], L - 1, q, g, k, v);
    std::vector<float> ref(16 * 256);
    g_orc_decode(q.data(), kc.data(), vc.data(), L, 16, 4, 256, 1.0f / 16.0f, g.data(), 0, ref.data());
    const auto& got = r.steps.back();
    EXPECT_EQ(got.pos, L - 1);
    double maxd = 0, se = 0, sr = 0;
    for (int i = 0; i < 16 * 256; i++) {
        const double d = bf16f(got.out[layer][i]) - ref[i];
        maxd = std::fmax(maxd, std::fabs(d));
        se += d * d;
        sr += (double)ref[i] * ref[i];
    }
    EXPECT_LE(maxd, 2e-2);
    EXPECT_LE(std::sqrt(se / sr), 1e-2);
    printf("    decode vs oracle: max|diff| %.2e, rel rms %.2e\n", maxd, std::sqrt(se / sr));
}

static void test_hybrid_resume() {
    printf("  test_hybrid_resume...\n");
    // 24 Gated-DeltaNet + 8 attention layers: reuse stops at the last state
    // snapshot (every 256 tokens) inside the shared prefix, and the restored
    // state decides what is generated next
    EXPECT_TRUE(load(4096, 24));
    auto prompt = random_tokens(600, 9);
    auto r1 = run_generate(prompt, 8);
    std::vector<int> all_ids = prompt;
    all_ids.insert(all_ids.end(), r1.tokens.begin(), r1.tokens.end());
    auto suffix = random_tokens(30, 10);
    all_ids.insert(all_ids.end(), suffix.begin(), suffix.end());
    auto r2 = run_generate(all_ids, 12);
    EXPECT_EQ(r2.reuse, 512);
    EXPECT_EQ(kvengine::state_restore_mismatches(), 0);
    EXPECT_TRUE(load(4096, 24));
    auto r3 = run_generate(all_ids, 12);
    EXPECT_EQ(r3.reuse, 0);
    EXPECT_TRUE(r2.tokens == r3.tokens);
    EXPECT_TRUE(same_outputs(r2, r3, 512));
}

static void test_reset_state() {
    printf("  test_reset_state...\n");
    EXPECT_TRUE(load(4096, 0));
    run_generate(random_tokens(64, 11), 4);
    kvengine::reset_state();
    EXPECT_EQ(kvengine::pos(), 0);
    EXPECT_TRUE(kvengine::cached_tokens().empty());
}

int main() {
    setvbuf(stdout, nullptr, _IOLBF, 0);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
        fprintf(stderr, "no HIP device\n");
        return 2;
    }
    const bool oracle = load_oracle();
    printf("Running KV engine tests (oracle %s)\n", oracle ? "loaded" : "missing");
    test_not_loaded();
    test_basic_generation();
    test_prompt_caching();
    test_greedy_determinism();
    test_divergent_prompt();
    test_context_truncation();
    test_attention_parity();
    test_hybrid_resume();
    test_reset_state();
    kvengine::shutdown();
    printf("%d/%d checks passed\n", g_tests - g_failures, g_tests);
    return g_failures ? 1 : 0;
}
