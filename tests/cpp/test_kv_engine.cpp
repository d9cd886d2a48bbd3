// Integration tests of the KV-cache path through the engine-side mirror
// (kvengine::generate / reset_state / ...), one function per behaviour, after
// the behaviours the reference's src/tests/test_inference.cpp covers (basic
// generation, prompt caching, determinism, reset) plus those this path adds
// (hybrid resume, multi-session serving, parity with the CPU oracle).
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

// The stop reasons carry the reference's numeric values (src/engine.h:23:
// enum StopReason { STOP_EOS, STOP_LENGTH, STOP_CALLBACK }).
static_assert(kvengine::STOP_EOS == 0 && kvengine::STOP_LENGTH == 1 && kvengine::STOP_CALLBACK == 2,
              "StopReason values differ from the reference's engine.h");

// ---- checks ----------------------------------------------------------------
// Each check is counted; a failed one prints where and what was compared, and
// the run continues so that one report lists every failure.
struct Tally {
    int checks = 0;
    int failed = 0;
};
static Tally g_tally;

static void check_at(bool ok, const char* expr, const char* file, int line) {
    g_tally.checks++;
    if (ok) return;
    g_tally.failed++;
    fprintf(stderr, "    check failed (%s:%d): %s\n", file, line, expr);
}

template <class A, class B>
static void check_cmp_at(bool ok, const A& got, const B& want, const char* expr, const char* file, int line) {
    g_tally.checks++;
    if (ok) return;
    g_tally.failed++;
    fprintf(stderr, "    check failed (%s:%d): %s -- got %.6g, want %.6g\n", file, line, expr, (double)got,
            (double)want);
}

#define CHECK(cond) check_at((cond), #cond, __FILE__, __LINE__)
#define CHECK_EQ(got, want)                                                     \
    do {                                                                        \
        const auto g_ = (got);                                                  \
        const auto w_ = (want);                                                 \
        check_cmp_at(g_ == w_, g_, w_, #got " == " #want, __FILE__, __LINE__); \
    } while (0)
#define CHECK_LE(got, bound)                                                      \
    do {                                                                          \
        const auto g_ = (got);                                                    \
        const auto b_ = (bound);                                                  \
        check_cmp_at(g_ <= b_, g_, b_, #got " <= " #bound, __FILE__, __LINE__);  \
    } while (0)

using kvengine::EngineConfig;

// ---- CPU oracle (test infrastructure only) ---------------------------------
typedef void (*decode_fn)(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int, int, float,
                          const uint16_t*, int, float*);
typedef void (*rope_tables_fn)(int, int, float, float*, float*);
typedef void (*produce_fn)(const float*, int, int, int, int, const float*, const float*, float, const float*,
                           const float*, float*, float*, float*, float*);
static decode_fn g_orc_decode = nullptr;
static rope_tables_fn g_orc_rope_tables = nullptr;
static produce_fn g_orc_produce = nullptr;

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
    g_orc_rope_tables = (rope_tables_fn)dlsym(h, "orc_rope_tables");
    g_orc_produce = (produce_fn)dlsym(h, "orc_qkv_produce");
    return g_orc_decode && g_orc_rope_tables && g_orc_produce;
}

static float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// bf16 patterns -> integers ordered like their values
static int ord16(uint16_t b) { return (b & 0x8000) ? 0x8000 - (int)b : (int)b; }

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

static bool load(int max_ctx, int n_ssm, bool verify_restore = false, int sessions = 4, bool keep = true,
                 const char* model = "synthetic/qwen3.5-9b") {
    EngineConfig cfg;
    cfg.n_ssm_layers = n_ssm;
    cfg.verify_restore = verify_restore;
    cfg.pool_blocks = 2048;
    cfg.max_sessions = sessions;
    cfg.keep_outputs = keep;
    kvengine::set_engine_config(cfg);
    return kvengine::load_model_and_tokenizer(model, max_ctx);
}

// outputs of positions >= from agree bit for bit (same kernels, same keys)
static bool same_outputs(const Run& a, const Run& b, int from) {
    for (const auto& sa : a.steps) {
        if (sa.pos < from) continue;
        bool found = false;
        for (const auto& sb : b.steps) {
            if (sb.pos != sa.pos) continue;
            found = true;
            if (sa.out != sb.out || sa.ssm_out != sb.ssm_out) return false;
        }
        if (!found) return false;
    }
    return true;
}

static void test_not_loaded() {
    printf("  test_not_loaded...\n");
    kvengine::shutdown();
    CHECK_EQ(kvengine::generate({1, 2, 3}, 4, 0.0f, nullptr), 0);
}

static void test_basic_generation() {
    printf("  test_basic_generation...\n");
    CHECK(load(4096, 0));
    kvengine::reset_state();
    auto prompt = random_tokens(40, 1);
    auto r = run_generate(prompt, 16);
    CHECK_EQ(r.n, 16);
    CHECK_EQ((int)r.tokens.size(), 16);
    // g_cached_tokens.size() == g_pos after every generate step (src/engine.cpp:4118, :4151)
    CHECK_EQ((int)kvengine::cached_tokens().size(), 56);
    CHECK_EQ(kvengine::pos(), 56);
    CHECK_EQ((int)r.steps.size(), 56);
    bool finite = true;
    for (const auto& st : r.steps)
        for (const auto& o : st.out)
            for (uint16_t b : o) finite = finite && std::isfinite(bf16f(b));
    CHECK(finite);
}

static void test_prompt_caching() {
    printf("  test_prompt_caching...\n");
    // first request, then the conversation extended with new tokens
    CHECK(load(4096, 0));
    auto prompt = random_tokens(100, 2);
    auto r1 = run_generate(prompt, 8);
    std::vector<int> all_ids = prompt;
    all_ids.insert(all_ids.end(), r1.tokens.begin(), r1.tokens.end());
    auto suffix = random_tokens(5, 3);
    all_ids.insert(all_ids.end(), suffix.begin(), suffix.end());
    auto r2 = run_generate(all_ids, 8);
    // 108 cached tokens are a prefix of the 113-token prompt: 96 reused (3 blocks)
    CHECK_EQ(r2.reuse, 96);
    CHECK_EQ(r2.n, 8);
    // the same request on a fresh engine (nothing cached) generates the same
    // tokens and the same attention outputs for every position it recomputes
    CHECK(load(4096, 0));
    auto r3 = run_generate(all_ids, 8);
    CHECK_EQ(r3.reuse, 0);
    CHECK(r2.tokens == r3.tokens);
    CHECK(same_outputs(r2, r3, 96));
}

static void test_greedy_determinism() {
    printf("  test_greedy_determinism...\n");
    CHECK(load(4096, 0));
    auto prompt = random_tokens(70, 4);
    kvengine::reset_state();
    auto r1 = run_generate(prompt, 16);
    kvengine::reset_state();
    auto r2 = run_generate(prompt, 16);
    CHECK_EQ(kvengine::pos(), 86);
    // the second run reuses the cached blocks (never the whole prompt)
    CHECK_EQ(r2.reuse, 64);
    CHECK(r1.tokens == r2.tokens);
    CHECK(same_outputs(r2, r1, 64));
}

static void test_divergent_prompt() {
    printf("  test_divergent_prompt...\n");
    // the reference resets on a divergent prompt (src/engine.cpp:4067-4071);
    // the block index still reuses the shared whole blocks
    CHECK(load(4096, 0));
    auto a = random_tokens(200, 5);
    run_generate(a, 4);
    std::vector<int> b(a.begin(), a.begin() + 150);
    b.push_back((a[150] + 1) % kvengine::kVocab);
    auto extra = random_tokens(20, 6);
    b.insert(b.end(), extra.begin(), extra.end());
    auto rb = run_generate(b, 8);
    CHECK_EQ(rb.reuse, 128);
    CHECK(load(4096, 0));
    auto rs = run_generate(b, 8);
    CHECK(rb.tokens == rs.tokens);
    CHECK(same_outputs(rb, rs, 128));
}

static void test_context_truncation() {
    printf("  test_context_truncation...\n");
    // an over-long prompt keeps its last max_ctx - max_tokens tokens (:4048-4056)
    CHECK(load(512, 0));
    auto prompt = random_tokens(700, 7);
    auto r = run_generate(prompt, 64);
    CHECK_EQ(r.n, 64);
    CHECK_EQ(kvengine::pos(), 512);
    const auto& cached = kvengine::cached_tokens();
    CHECK(std::vector<int>(cached.begin(), cached.begin() + 448) ==
                std::vector<int>(prompt.end() - 448, prompt.end()));
}

static void test_attention_parity() {
    printf("  test_attention_parity...\n");
    if (!g_orc_decode) {
        CHECK(g_orc_decode != nullptr);
        return;
    }
    CHECK(load(4096, 0));
    auto prompt = random_tokens(300, 8);
    auto r = run_generate(prompt, 4);
    const int L = kvengine::pos();  // 304 keys; the last decode step saw all of them
    const int layer = 3;
    std::vector<uint16_t> kc((size_t)L * 1024), vc((size_t)L * 1024);
    void *dk = nullptr, *dv = nullptr;
    CHECK_EQ(hipMalloc(&dk, kc.size() * 2), hipSuccess);
    CHECK_EQ(hipMalloc(&dv, vc.size() * 2), hipSuccess);
    int32_t seq = kvengine::sequence(), n = L;
    CHECK_EQ(kvc_gather(kvengine::context(), layer, &seq, 1, 0, &n, dk, dv, nullptr), KVC_OK);
    CHECK_EQ(hipMemcpy(kc.data(), dk, kc.size() * 2, hipMemcpyDeviceToHost), hipSuccess);
    CHECK_EQ(hipMemcpy(vc.data(), dv, vc.size() * 2, hipMemcpyDeviceToHost), hipSuccess);
    CHECK_EQ(hipFree(dk), hipSuccess);
    CHECK_EQ(hipFree(dv), hipSuccess);
    // the cache holds the producer's output for every position: V bit-exact,
    // K (RMSNorm + RoPE) within one bf16 ulp of the oracle and >= 99% exact
    const auto& cached = kvengine::cached_tokens();
    std::vector<float> cos_t((size_t)L * 32), sin_t((size_t)L * 32), qn, kn, rowf(kvengine::kQkvRow);
    g_orc_rope_tables(L, 64, 1.0e7f, cos_t.data(), sin_t.data());
    kvengine::synthetic_norm_weights(layer, qn, kn);
    std::vector<uint16_t> row;
    std::vector<float> q(16 * 256), g(16 * 256), k(1024), v(1024);
    bool v_exact = true;
    int k_far = 0;
    long k_same = 0;
    for (int p = 0; p < L; p++) {
        kvengine::synthetic_qkv_row(layer, cached[p], p, row);
        for (int i = 0; i < kvengine::kQkvRow; i++) rowf[i] = bf16f(row[i]);
        g_orc_produce(rowf.data(), 16, 4, 256, 64, qn.data(), kn.data(), 1e-6f, &cos_t[(size_t)p * 32],
                      &sin_t[(size_t)p * 32], q.data(), g.data(), k.data(), v.data());
        for (int i = 0; i < 1024; i++) {
            v_exact = v_exact && vc[(size_t)p * 1024 + i] == bf16_rne(v[i]);
            const int d = std::abs(ord16(kc[(size_t)p * 1024 + i]) - ord16(bf16_rne(k[i])));
            k_far += d > 1;
            k_same += d == 0;
        }
    }
    CHECK(v_exact);
    CHECK_EQ(k_far, 0);
    CHECK(k_same >= (long)(0.99 * L * 1024));
    // the last decode step (its produced q and gate) vs the oracle over the same cache
    const auto& got = r.steps.back();
    CHECK_EQ(got.pos, L - 1);
    CHECK(!got.q.empty() && got.q[layer].size() == 16 * 256);
    if (got.q.empty()) return;
    std::vector<float> ref(16 * 256);
    g_orc_decode(got.q[layer].data(), kc.data(), vc.data(), L, 16, 4, 256, 1.0f / 16.0f, got.gate[layer].data(), 1,
                 ref.data());
    double maxd = 0, se = 0, sr = 0;
    for (int i = 0; i < 16 * 256; i++) {
        const double d = bf16f(got.out[layer][i]) - ref[i];
        maxd = std::fmax(maxd, std::fabs(d));
        se += d * d;
        sr += (double)ref[i] * ref[i];
    }
    CHECK_LE(maxd, 2e-2);
    CHECK_LE(std::sqrt(se / sr), 1e-2);
    printf("    decode vs oracle: max|diff| %.2e, rel rms %.2e; K exact %.4f\n", maxd, std::sqrt(se / sr),
           (double)k_same / ((double)L * 1024));
}

static void test_hybrid_resume() {
    printf("  test_hybrid_resume...\n");
    // 24 Gated-DeltaNet + 8 attention layers: reuse stops at the last state
    // snapshot (every 256 tokens) inside the shared prefix, and the restored
    // state decides what is generated next
    CHECK(load(4096, 24, true));
    auto prompt = random_tokens(600, 9);
    auto r1 = run_generate(prompt, 8);
    std::vector<int> all_ids = prompt;
    all_ids.insert(all_ids.end(), r1.tokens.begin(), r1.tokens.end());
    auto suffix = random_tokens(30, 10);
    all_ids.insert(all_ids.end(), suffix.begin(), suffix.end());
    auto r2 = run_generate(all_ids, 12);
    CHECK_EQ(r2.reuse, 512);
    CHECK_EQ(kvengine::state_restore_checks(), 1);
    CHECK_EQ(kvengine::state_restore_mismatches(), 0);
    CHECK(load(4096, 24));
    auto r3 = run_generate(all_ids, 12);
    CHECK_EQ(r3.reuse, 0);
    CHECK(r2.tokens == r3.tokens);
    CHECK(same_outputs(r2, r3, 512));  // attention and Gated-DeltaNet outputs, bit for bit
}

static void test_reset_state() {
    printf("  test_reset_state...\n");
    CHECK(load(4096, 0));
    run_generate(random_tokens(64, 11), 4);
    kvengine::reset_state();
    CHECK_EQ(kvengine::pos(), 0);
    CHECK(kvengine::cached_tokens().empty());
}


static void test_hang_info() {
    printf("  test_hang_info...\n");
    // the last blocking device call before control returned: the read of the
    // last recurrent layer's output on a hybrid model, of the last attention
    // layer's output on a pure-attention one (src/engine.cpp:100-101)
    int layer = 0, op = 0;
    CHECK(load(1024, 0));
    kvengine::get_hang_info(layer, op);
    CHECK_EQ(layer, -1);
    CHECK_EQ(op, 0);
    run_generate(random_tokens(40, 12), 2);
    kvengine::get_hang_info(layer, op);
    CHECK_EQ(layer, 7);
    CHECK_EQ(op, 1);
    CHECK(load(1024, 24, true));
    run_generate(random_tokens(40, 13), 2);
    kvengine::get_hang_info(layer, op);
    CHECK_EQ(layer, 23);
    CHECK_EQ(op, 2);
}

static void test_model_path_names_the_model() {
    printf("  test_model_path_names_the_model...\n");
    // load_model_and_tokenizer(model_path, max_ctx) keeps the reference's
    // signature; the path names the synthetic model (its seed)
    auto prompt = random_tokens(50, 14);
    CHECK(load(1024, 0, false, 4, true, "synthetic/a"));
    auto a1 = run_generate(prompt, 6);
    CHECK(load(1024, 0, false, 4, true, "synthetic/a"));
    auto a2 = run_generate(prompt, 6);
    CHECK(load(1024, 0, false, 4, true, "synthetic/b"));
    auto b = run_generate(prompt, 6);
    CHECK(a1.tokens == a2.tokens);
    CHECK(same_outputs(a1, a2, 0));
    CHECK(a1.tokens != b.tokens);
    CHECK(!kvengine::load_model_and_tokenizer("synthetic/a", 0));  // no context: refused
    CHECK_EQ(kvengine::generate(prompt, 4, 0.0f, nullptr), 0);    // and nothing is loaded
}

// One turn of a conversation on a session: the prompt grows by the turn's
// suffix, generation appends its tokens (src/chat.cpp:117-184).
struct Turn {
    int reuse = 0;
    std::vector<int> generated;
    std::vector<std::pair<int, uint64_t>> digests;  // (position, digest of every layer output)
};

static Turn chat_turn(int session, std::vector<int>& ids, int max_gen) {
    Turn t;
    kvengine::StopReason why = kvengine::STOP_CALLBACK;
    const int n = kvengine::generate_session(session, ids, max_gen, 0.0f,
                                             [&](int id, const std::string&) {
                                                 t.generated.push_back(id);
                                                 return true;
                                             },
                                             &why);
    CHECK_EQ(n, max_gen);
    ids.insert(ids.end(), t.generated.begin(), t.generated.end());
    t.reuse = kvengine::last_prefix_len(session);
    for (const auto& st : kvengine::step_outputs(session)) t.digests.push_back({st.pos, st.digest});
    // g_cached_tokens == the conversation, g_pos == its length (src/engine.cpp:4118, :4151)
    CHECK(kvengine::cached_tokens(session) == ids);
    CHECK_EQ(kvengine::pos(session), (int)ids.size());
    return t;
}

static std::vector<int> turn_suffix(int conv, int turn) {
    return random_tokens(30 + 11 * conv + 7 * turn, 1000 + 10 * conv + turn);
}

// positions both runs processed hold the same outputs, bit for bit
static bool same_digests(const Turn& a, const Turn& b) {
    int common = 0;
    for (const auto& da : a.digests)
        for (const auto& db : b.digests)
            if (da.first == db.first) {
                if (da.second != db.second) return false;
                common++;
            }
    return common > 0;
}

static void test_interleaved_sessions() {
    printf("  test_interleaved_sessions...\n");
    // Four multi-turn conversations on one hybrid engine (24 Gated-DeltaNet +
    // 8 attention layers), sharing a 300-token system prefix, their turns
    // interleaved round-robin.  Every turn must reuse exactly the longest
    // snapshot boundary (multiple of 256) that some session has committed
    // and that leaves one prompt token to run, and must generate the same
    // tokens with the same attention and Gated-DeltaNet outputs, bit for bit,
    // as the same conversation run alone on a fresh engine.
    constexpr int kConv = 4, kTurns = 3, kGen = 6;
    CHECK(load(4096, 24, false, kConv, false));
    const std::vector<int> sys = random_tokens(300, 900);
    std::vector<int> ids[kConv];
    int session[kConv];
    Turn rec[kConv][kTurns];
    std::vector<std::vector<int>> committed;  // every history a session has processed
    for (int c = 0; c < kConv; c++) {
        session[c] = c == 0 ? 0 : kvengine::create_session();
        CHECK_EQ(session[c], c);
    }
    for (int turn = 0; turn < kTurns; turn++)
        for (int c = 0; c < kConv; c++) {
            if (turn == 0) ids[c] = sys;
            const auto sfx = turn_suffix(c, turn);
            ids[c].insert(ids[c].end(), sfx.begin(), sfx.end());
            int want = 0;
            for (int b = 256; b <= (int)ids[c].size() - 1; b += 256)
                for (const auto& h : committed)
                    if ((int)h.size() >= b && std::equal(h.begin(), h.begin() + b, ids[c].begin())) want = b;
            rec[c][turn] = chat_turn(session[c], ids[c], kGen);
            CHECK_EQ(rec[c][turn].reuse, want);
            committed.push_back(ids[c]);
        }
    CHECK_EQ(rec[1][0].reuse, 256);  // the shared system prefix, from conversation 0
    CHECK_EQ(rec[0][1].reuse, 256);  // its own history
    CHECK_EQ(kvengine::create_session(), -1);  // all sessions in use
    CHECK(kvengine::release_session(3));
    CHECK_EQ(kvengine::create_session(), 3);
    // each conversation alone on a fresh engine
    for (int c = 0; c < kConv; c++) {
        CHECK(load(4096, 24, false, 1, false));
        std::vector<int> solo;
        for (int turn = 0; turn < kTurns; turn++) {
            if (turn == 0) solo = sys;
            const auto sfx = turn_suffix(c, turn);
            solo.insert(solo.end(), sfx.begin(), sfx.end());
            const Turn t = chat_turn(0, solo, kGen);
            CHECK(t.generated == rec[c][turn].generated);
            CHECK(same_digests(t, rec[c][turn]));
        }
        CHECK(solo == ids[c]);
    }
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
    test_hang_info();
    test_model_path_names_the_model();
    test_interleaved_sessions();
    kvengine::shutdown();
    printf("%d of %d checks passed\n", g_tally.checks - g_tally.failed, g_tally.checks);
    return g_tally.failed ? 1 : 0;
}
