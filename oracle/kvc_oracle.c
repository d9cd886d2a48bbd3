/*
 * kvc_oracle.c -- CPU restatement of the reference KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the CPU
 * baseline timed by bench.py.  The product never links or calls it.
 *
 * Built with -O3 -march=native and WITHOUT -ffast-math (the reference builds
 * with -ffast-math, Makefile:47; the oracle must be deterministic).
 *
 * What pins each function (tests/test_oracle_*.py):
 *   splitmix64           published test vector (seed 1234567)
 *   box_muller           closed form at chosen uniforms; moments of 1e6 draws
 *   f32_to_bf16_rne      exhaustive: nearest-even by exact comparison in fp64
 *                        over every bf16 neighbourhood; NaN/Inf cases
 *   f32_to_bf16_trunc    bit identity (top 16 bits)
 *   fast_expf(_rne)      every finite bf16 input and 20000 random fp32
 *                        inputs against an exact rational model: the fused
 *                        multiply-add rounded once to fp32, then truncated
 *                        (rounded to nearest even); an unfused multiply-add
 *                        fails it; constants at x = 0, ln2 multiples, clamps
 *   sigmoid/silu mode 1  every finite bf16 input against the same model with
 *                        each fp32 step (add, divide, multiply) exactly rounded
 *   cache_append/gather  byte equality + canary (untouched slots unchanged)
 *   decode_attn          fp64 two-pass softmax brute force; L=1 -> v0;
 *                        identical keys -> mean(V); one dominant key -> V_j;
 *                        GQA head map via per-head constant V; gate identity
 *   prefill_attn         row i equals decode at L=pos0+i+1 computed by the
 *                        fp64 brute force; perturbing keys j > pos0+i leaves
 *                        row i unchanged (causality)
 *   truncate/reference_prefix  known-answer cases derived from
 *                        src/engine.cpp:4048-4080 by hand; brute-force LCP
 *   block_hash/chain     determinism, prefix property, weak-hash collisions
 *   reuse_len            brute-force enumeration of the rule on small inputs
 *   conv_push            explicit three-step shift by hand
 *   deltanet_head_step   fp64 restatement of the delta rule (S <- S*a; S +=
 *                        k (beta (v - S k))^T) on random small heads
 *   rope_tables          theta of pair p at pos 1 is base^(-2p/rope_dim)
 *                        (p = 0, 16, 31 checked against the closed form in
 *                        fp64); cos^2 + sin^2 = 1; pos 0 is the identity
 *   rms_norm_head        constant input -> w; scale invariance (x and 3x);
 *                        output RMS = 1 with unit weights; eps dominates a
 *                        zero head (output 0)
 *   rope_head            unit vector on pair p -> (cos, sin) of the table
 *                        (sign and pairing); pair norms preserved; dims >=
 *                        rope_dim untouched; rotating by positions a then b
 *                        equals a + b to fp32 accuracy
 *   deltanet_layer_step  composition of the pinned conv_push and
 *                        deltanet_head_step; delta-rule invariant S'k = v
 *                        for beta -> 1, a = 0 (decay 1); decay = e^(softplus
 *                        * a) at chosen alpha; a zero projection row leaves
 *                        the state scaled by the decay and gives zero output;
 *                        gated norm: output RMS = |norm_w| for silu(z) = z
 *   qkv_produce          deinterleave: gate rows and v rows are copies of
 *                        the input rows; q/k equal norm-then-rope of their
 *                        rows (composition of the two pinned steps)
 * No function is "parity unpinned".
 */
#include "kvc_oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* splitmix64 (Steele, Lea, Flood 2014) -- the BASELINE input generator.   */
static const uint64_t kGolden = 0x9E3779B97F4A7C15ULL;

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t orc_splitmix64_next(uint64_t* state) {
    *state += kGolden;
    return mix64(*state);
}

uint64_t orc_splitmix64_at(uint64_t seed, uint64_t index) {
    return mix64(seed + (index + 1) * kGolden);
}

/* Box-Muller on one 64-bit draw: u1 from the top 24 bits (in (0,1]), u2 from
 * the next 24 bits (in [0,1)).  Evaluated in double, rounded once to float. */
void orc_box_muller(uint64_t draw, float* z0, float* z1) {
    const double inv24 = 1.0 / 16777216.0;
    double u1 = (double)((draw >> 40) + 1) * inv24;
    double u2 = (double)((draw >> 16) & 0xFFFFFFULL) * inv24;
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925286766559 * u2;
    *z0 = (float)(r * cos(t));
    *z1 = (float)(r * sin(t));
}

void orc_fill_normal_f32(float* dst, size_t n, uint64_t seed, float scale) {
    for (size_t i = 0; i < n; i += 2) {
        float z0, z1;
        orc_box_muller(orc_splitmix64_at(seed, i / 2), &z0, &z1);
        dst[i] = z0 * scale;
        if (i + 1 < n) dst[i + 1] = z1 * scale;
    }
}

void orc_fill_normal_bf16(uint16_t* dst, size_t n, uint64_t seed, float scale) {
    for (size_t i = 0; i < n; i += 2) {
        float z0, z1;
        orc_box_muller(orc_splitmix64_at(seed, i / 2), &z0, &z1);
        dst[i] = orc_f32_to_bf16_rne(z0 * scale);
        if (i + 1 < n) dst[i + 1] = orc_f32_to_bf16_rne(z1 * scale);
    }
}

/* ---------------------------------------------------------------------- */
/* bf16 conversions.  The reference converts by truncation
 * (src/engine.cpp:248-252); this build rounds to nearest even and keeps
 * truncation only for reference-compatible checks. */
uint16_t orc_f32_to_bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN, keep sign */
    }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

uint16_t orc_f32_to_bf16_trunc(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_f32_to_bf16_rne_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_bf16_rne(src[i]);
}

void orc_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_bf16_to_f32(src[i]);
}

/* Schraudolph (1999) exp as the compiled reference computes it
 * (src/engine.cpp:2349-2356): clamp to [-88, 88], then the fp32 bit pattern
 * (int32)(12102203 x + 1065353216), slope 2^23/ln2 and bias 127*2^23.  The
 * reference is built with -ffast-math for an FMA-capable host (Makefile:47,
 * -march=native on an EPYC 9254 whose flags list fma,
 * reference_system_info/lscpu.txt), so clang fuses the multiply-add (probe:
 * clang -O3 -ffast-math -march=znver4 emits vfmadd213ss + vcvttss2si for this
 * expression).  The oracle is built with contraction off and writes the
 * fused operation out.  The scalar int conversion truncates toward zero. */
float orc_fast_expf(float x) {
    if (x < -88.0f) x = -88.0f;
    if (x > 88.0f) x = 88.0f;
    int32_t i = (int32_t)fmaf(12102203.0f, x, 1065353216.0f);
    float f;
    memcpy(&f, &i, 4);
    return f;
}

/* The AVX-512 SiLU's exp (src/engine.cpp:2367-2373): the same fused
 * multiply-add of the clamped -x, converted with _mm512_cvtps_epi32, which
 * rounds to nearest even under the default MXCSR. */
float orc_fast_expf_rne(float x) {
    if (x < -88.0f) x = -88.0f;
    if (x > 88.0f) x = 88.0f;
    int32_t i = (int32_t)rintf(fmaf(12102203.0f, x, 1065353216.0f));
    float f;
    memcpy(&f, &i, 4);
    return f;
}

/* mode 1 is fast_sigmoidf's source expression with an IEEE division
 * (:2358-2360).  The reference's fast-math build may compile the division as
 * an approximate reciprocal and a Newton step: over every finite bf16 input
 * its Zen 4 build differs from this model by at most 1 ulp (subnormal
 * quotients aside), as tests/test_fastmath_forms.py measures. */
float orc_sigmoid(float x, int mode) {
    if (mode == 1) return 1.0f / (1.0f + orc_fast_expf(-x)); /* :2358-2360 */
    return 1.0f / (1.0f + expf(-x));
}

/* SiLU x * sigmoid(x).  mode 1 is the AVX-512 form used on the conv output
 * and the z gate (:2366-2376, called at :2626, :2714, :3227, :3321). */
float orc_silu(float x, int mode) {
    if (mode == 1) return x * (1.0f / (1.0f + orc_fast_expf_rne(0.0f - x)));
    return x * orc_sigmoid(x, 0);
}

/* ---------------------------------------------------------------------- */
void orc_cache_append(uint16_t* kc, uint16_t* vc, int n_kv, int d, int pos,
                      int n_tok, const uint16_t* k, const uint16_t* v) {
    size_t row = (size_t)n_kv * d;
    memcpy(kc + (size_t)pos * row, k, (size_t)n_tok * row * sizeof(uint16_t));
    memcpy(vc + (size_t)pos * row, v, (size_t)n_tok * row * sizeof(uint16_t));
}

void orc_cache_gather(const uint16_t* kc, const uint16_t* vc, int n_kv, int d,
                      int tok0, int n_tok, uint16_t* k_out, uint16_t* v_out) {
    size_t row = (size_t)n_kv * d;
    memcpy(k_out, kc + (size_t)tok0 * row, (size_t)n_tok * row * sizeof(uint16_t));
    memcpy(v_out, vc + (size_t)tok0 * row, (size_t)n_tok * row * sizeof(uint16_t));
}

/* ---------------------------------------------------------------------- */
/* Dot product in the reference's accumulation shape: 16 fused lanes over d,
 * then a halving reduction (src/engine.cpp:3541-3544). Requires d % 16 == 0. */
static float dot16(const float* a, const float* b, int d) {
    float lane[16];
    for (int j = 0; j < 16; j++) lane[j] = 0.0f;
    for (int i = 0; i < d; i += 16)
        for (int j = 0; j < 16; j++) lane[j] = fmaf(a[i + j], b[i + j], lane[j]);
    for (int w = 8; w >= 1; w >>= 1)
        for (int j = 0; j < w; j++) lane[j] += lane[j + w];
    return lane[0];
}

/* One query head against L keys of one KV head: src/engine.cpp:3532-3563.
 * kbase/vbase point at head kv_h of position 0; stride is n_kv*d elements. */
static void attend_head(const float* qh, const uint16_t* kbase,
                        const uint16_t* vbase, size_t stride, int L, int d,
                        float scale, const uint16_t* gh, int gate_mode,
                        float* out, float* kbuf, float* acc) {
    float max_score = -FLT_MAX, sum_exp = 0.0f;
    for (int i = 0; i < d; i++) acc[i] = 0.0f;
    for (int kp = 0; kp < L; kp++) {
        const uint16_t* kh = kbase + (size_t)kp * stride;
        for (int i = 0; i < d; i++) kbuf[i] = orc_bf16_to_f32(kh[i]);
        float score = dot16(qh, kbuf, d) * scale;
        float new_max = score > max_score ? score : max_score;
        float exp_s = expf(score - new_max);
        float corr = expf(max_score - new_max);
        sum_exp = sum_exp * corr + exp_s;
        const uint16_t* vh = vbase + (size_t)kp * stride;
        for (int i = 0; i < d; i++)
            acc[i] = fmaf(exp_s, orc_bf16_to_f32(vh[i]), acc[i] * corr);
        max_score = new_max;
    }
    for (int i = 0; i < d; i++) {
        float o = acc[i] / sum_exp;
        if (gh) o *= orc_sigmoid(orc_bf16_to_f32(gh[i]), gate_mode);
        out[i] = o;
    }
}

#define ORC_MAX_D 1024

void orc_decode_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                     int L, int n_q, int n_kv, int d, float scale,
                     const uint16_t* gate, int gate_mode, float* out) {
    float qh[ORC_MAX_D], kbuf[ORC_MAX_D], acc[ORC_MAX_D];
    size_t stride = (size_t)n_kv * d;
    int group = n_q / n_kv; /* kv_h = h / (n_head / n_head_kv), :3532 */
    for (int h = 0; h < n_q; h++) {
        int kv_h = h / group;
        for (int i = 0; i < d; i++) qh[i] = orc_bf16_to_f32(q[(size_t)h * d + i]);
        attend_head(qh, kc + (size_t)kv_h * d, vc + (size_t)kv_h * d, stride, L,
                    d, scale, gate ? gate + (size_t)h * d : 0, gate_mode,
                    out + (size_t)h * d, kbuf, acc);
    }
}

void orc_prefill_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                      int pos0, int n, int n_q, int n_kv, int d, float scale,
                      const uint16_t* gate, int gate_mode, float* out) {
    size_t row = (size_t)n_q * d;
    for (int i = 0; i < n; i++) {
        /* token ti sits at pos = g_pos + ti and sees kv_len = pos + 1 keys
         * (src/engine.cpp:2844, :2889) */
        orc_decode_attn(q + i * row, kc, vc, pos0 + i + 1, n_q, n_kv, d, scale,
                        gate ? gate + i * row : 0, gate_mode, out + i * row);
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_decode_attn_batch(int n_seqs, const uint16_t* q,
                           const uint16_t* const* kcs,
                           const uint16_t* const* vcs, const int* Ls, int n_q,
                           int n_kv, int d, float scale, float* out, int threads) {
    int total = n_seqs * n_q;
    int group = n_q / n_kv;
    size_t stride = (size_t)n_kv * d;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
    for (int w = 0; w < total; w++) {
        float qh[ORC_MAX_D], kbuf[ORC_MAX_D], acc[ORC_MAX_D];
        int s = w / n_q, h = w % n_q, kv_h = h / group;
        const uint16_t* qs = q + ((size_t)s * n_q + h) * d;
        for (int i = 0; i < d; i++) qh[i] = orc_bf16_to_f32(qs[i]);
        attend_head(qh, kcs[s] + (size_t)kv_h * d, vcs[s] + (size_t)kv_h * d,
                    stride, Ls[s], d, scale, 0, 0,
                    out + ((size_t)s * n_q + h) * d, kbuf, acc);
    }
    (void)threads;
}

/* ---------------------------------------------------------------------- */
int orc_truncate_count(int n_prompt, int max_ctx, int max_tokens) {
    int half = max_ctx / 2;
    int max_prompt = max_ctx - (max_tokens < half ? max_tokens : half);
    if (max_prompt < 1) max_prompt = 1;
    return n_prompt > max_prompt ? n_prompt - max_prompt : 0;
}

int orc_lcp(const int32_t* a, int na, const int32_t* b, int nb) {
    int n = na < nb ? na : nb, i = 0;
    while (i < n && a[i] == b[i]) i++;
    return i;
}

int orc_reference_prefix(const int32_t* cached, int n_cached,
                         const int32_t* prompt, int n_prompt, int* reset) {
    int prefix_len = orc_lcp(prompt, n_prompt, cached, n_cached);
    *reset = 0;
    if (prefix_len < n_cached) { /* divergence -> full reset, :4067-4071 */
        *reset = 1;
        prefix_len = 0;
    }
    if (prefix_len >= n_prompt) { /* whole prompt cached -> reset, :4072-4076 */
        *reset = 1;
        prefix_len = 0;
    }
    return prefix_len;
}

/* The chained block hash of this build (the reference has none).  Each block
 * hash absorbs its parent, its length and every token through the splitmix64
 * finaliser; the root is a fixed constant.  Identical in the HIP library. */
uint64_t orc_hash_root(void) { return 0x6B76635F726F6F74ULL; }

uint64_t orc_block_hash(uint64_t parent, const int32_t* tok, int n, int weak) {
    uint64_t h = mix64(parent ^ (kGolden * (uint64_t)(n + 1)));
    for (int i = 0; i < n; i++)
        h = mix64(h + (uint64_t)(uint32_t)tok[i] + kGolden * (uint64_t)(i + 1));
    return weak ? (h & 0xFULL) : h;
}

void orc_hash_chain(const int32_t* tok, int n_blocks, int block, int weak,
                    uint64_t* out) {
    uint64_t h = orc_hash_root();
    for (int b = 0; b < n_blocks; b++) {
        h = orc_block_hash(h, tok + (size_t)b * block, block, weak);
        out[b] = h;
    }
}

int orc_reuse_len(int lcp, int n_prompt, int block, int interval,
                  const uint8_t* snap, int n_snap, int has_ssm) {
    int limit = n_prompt - 1; /* never reuse the whole prompt, :4072-4076 */
    int m = lcp < limit ? lcp : limit;
    if (m <= 0) return 0;
    m = (m / block) * block;
    if (!has_ssm) return m;
    if (interval <= 0) return 0;
    for (int k = m / interval; k >= 1; k--)
        if (k - 1 < n_snap && snap[k - 1]) return k * interval;
    return 0;
}

/* ---------------------------------------------------------------------- */
void orc_conv_push(float* state, int rows, int channels, const float* x) {
    for (int r = 0; r + 1 < rows; r++)
        memcpy(state + (size_t)r * channels, state + (size_t)(r + 1) * channels,
               (size_t)channels * sizeof(float));
    memcpy(state + (size_t)(rows - 1) * channels, x, (size_t)channels * sizeof(float));
}

void orc_deltanet_head_step(float* state, int dv, int dk, const float* q,
                            const float* k, const float* v, float decay,
                            float beta, float out_scale, float* out) {
    for (int i = 0; i < dv; i++) {
        float* row = state + (size_t)i * dk;
        float sk = 0.0f;
        for (int j = 0; j < dk; j++) {
            row[j] *= decay;
            sk = fmaf(row[j], k[j], sk);
        }
        float dd = beta * (v[i] - sk);
        float o = 0.0f;
        for (int j = 0; j < dk; j++) {
            row[j] = fmaf(k[j], dd, row[j]);
            o = fmaf(row[j], q[j], o);
        }
        out[i] = o * out_scale;
    }
}

/* ---------------------------------------------------------------------- */
/* K producer: per-head RMSNorm + partial NeoX RoPE                         */

void orc_rope_tables(int max_ctx, int rope_dim, float base, float* cos_t, float* sin_t) {
    const int half = rope_dim / 2;
    for (int pos = 0; pos < max_ctx; pos++) {
        for (int p = 0; p < half; p++) {
            const float freq = 1.0f / powf(base, 2.0f * p / rope_dim);
            const float theta = pos * freq;
            cos_t[(size_t)pos * half + p] = cosf(theta);
            sin_t[(size_t)pos * half + p] = sinf(theta);
        }
    }
}

void orc_rms_norm_head(float* x, int d, const float* w, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < d; i++) ss += x[i] * x[i];
    const float r = 1.0f / sqrtf(ss / d + eps);
    for (int i = 0; i < d; i++) x[i] = x[i] * r * w[i];
}

void orc_rope_head(float* x, int rope_dim, const float* cos_row, const float* sin_row) {
    const int half = rope_dim / 2;
    for (int p = 0; p < half; p++) {
        const float x0 = x[p], x1 = x[p + half];
        x[p] = x0 * cos_row[p] - x1 * sin_row[p];
        x[p + half] = x1 * cos_row[p] + x0 * sin_row[p];
    }
}

void orc_qkv_produce(const float* qkv, int n_q, int n_kv, int d, int rope_dim,
                     const float* q_norm, const float* k_norm, float eps,
                     const float* cos_row, const float* sin_row, float* q,
                     float* gate, float* k, float* v) {
    const float* krow = qkv + (size_t)n_q * 2 * d;
    const float* vrow = krow + (size_t)n_kv * d;
    for (int h = 0; h < n_q; h++) {
        if (q) {
            float* qh = q + (size_t)h * d;
            memcpy(qh, qkv + (size_t)h * 2 * d, sizeof(float) * d);
            orc_rms_norm_head(qh, d, q_norm, eps);
            if (rope_dim > 0) orc_rope_head(qh, rope_dim, cos_row, sin_row);
        }
        if (gate) memcpy(gate + (size_t)h * d, qkv + (size_t)h * 2 * d + d, sizeof(float) * d);
    }
    for (int h = 0; h < n_kv; h++) {
        if (k) {
            float* kh = k + (size_t)h * d;
            memcpy(kh, krow + (size_t)h * d, sizeof(float) * d);
            orc_rms_norm_head(kh, d, k_norm, eps);
            if (rope_dim > 0) orc_rope_head(kh, rope_dim, cos_row, sin_row);
        }
        if (v) memcpy(v + (size_t)h * d, vrow + (size_t)h * d, sizeof(float) * d);
    }
}

/* ---------------------------------------------------------------------- */
/* Gated-DeltaNet layer step                                                */

void orc_deltanet_layer_step(float* conv_state, float* ssm_state, const float* proj,
                             const float* conv_w, const float* dt_bias, const float* a,
                             const float* norm_w, int n_v, int n_k, int dk, int dv,
                             float eps, float out_scale, int fast, float* out) {
    const int C = 2 * n_k * dk + n_v * dv;
    const float* x = proj;
    const float* z = proj + C;
    const float* alpha = z + (size_t)n_v * dv;
    const float* beta_raw = alpha + n_v;
    float conv[16384];
    if (C > 16384 || dk > 512 || dv > 512) return;
    const float* s0 = conv_state;
    const float* s1 = conv_state + C;
    const float* s2 = conv_state + 2 * (size_t)C;
    for (int ch = 0; ch < C; ch++) { /* :3209-3226 */
        float sum = s0[ch] * conv_w[ch];
        sum = fmaf(s1[ch], conv_w[C + ch], sum);
        sum = fmaf(s2[ch], conv_w[2 * (size_t)C + ch], sum);
        sum = fmaf(x[ch], conv_w[3 * (size_t)C + ch], sum);
        conv[ch] = orc_silu(sum, fast);
    }
    orc_conv_push(conv_state, 3, C, x); /* :3228-3230 */
    const float* cq = conv;
    const float* ck = conv + (size_t)n_k * dk;
    const float* cv = conv + 2 * (size_t)n_k * dk;
    for (int vh = 0; vh < n_v; vh++) {
        const int kh = vh % n_k;
        float q[512], k[512], o[512];
        float qn = 0.0f, kn = 0.0f;
        for (int j = 0; j < dk; j++) {
            q[j] = cq[(size_t)kh * dk + j];
            k[j] = ck[(size_t)kh * dk + j];
            qn = fmaf(q[j], q[j], qn);
            kn = fmaf(k[j], k[j], kn);
        }
        const float qs = 1.0f / sqrtf(qn + eps), ks = 1.0f / sqrtf(kn + eps);
        for (int j = 0; j < dk; j++) {
            q[j] *= qs;
            k[j] *= ks;
        }
        const float biased = alpha[vh] + dt_bias[vh];
        const float ex = fast ? orc_fast_expf(biased) : expf(biased);
        const float sp = biased > 20.0f ? biased : logf(1.0f + ex);
        const float decay = expf(sp * a[vh]);
        const float beta = orc_sigmoid(beta_raw[vh], fast);
        orc_deltanet_head_step(ssm_state + (size_t)vh * dv * dk, dv, dk, q, k, cv + (size_t)vh * dv, decay,
                               beta, out_scale, o);
        float ss = 0.0f;
        for (int i = 0; i < dv; i++) ss = fmaf(o[i], o[i], ss);
        const float rms = 1.0f / sqrtf(ss / dv + eps);
        for (int i = 0; i < dv; i++)
            out[(size_t)vh * dv + i] = o[i] * rms * norm_w[i] * orc_silu(z[(size_t)vh * dv + i], fast);
    }
}
