/* The reference's sigmoid-bearing expressions, restated so that their
 * fast-math compilation can be measured against the oracle's model of them
 * (test infrastructure only; test_fastmath_forms.py compiles this file
 * with the reference's engine flags, -O3 -ffast-math -march=<its host>,
 * Makefile:14,47, and runs it over every finite bf16 input).
 *
 *   fexp       fast_expf, src/engine.cpp:2349-2356
 *   sig_loop   the gate's fast_sigmoidf applied over a row, :2358-2360
 *   gate_loop  the gated attention output out = (acc / sum) * sigma(gate),
 *              :2922-2923 (prefill) and :3562-3563 (decode)
 *   silu512    the AVX-512 SiLU, :2366-2376 (conv output and z gate)
 */
#include <immintrin.h>
#include <stdint.h>

static inline float fexp(float x) {
    x = x < -88.0f ? -88.0f : (x > 88.0f ? 88.0f : x);
    union {
        float f;
        int32_t i;
    } u;
    u.i = (int32_t)(12102203.0f * x + 1065353216.0f);
    return u.f;
}

static inline float fsig(float x) { return 1.0f / (1.0f + fexp(-x)); }

void sig_loop(const float* g, float* out, int n) {
    for (int d = 0; d < n; d++) out[d] = fsig(g[d]);
}

void gate_loop(const float* acc, float sum, const float* g, float* out, int n) {
    for (int d = 0; d < n; d++) out[d] = (acc[d] / sum) * fsig(g[d]);
}

void silu512(const float* x, float* out, int n) {
    for (int i = 0; i + 16 <= n; i += 16) {
        const __m512 xv = _mm512_loadu_ps(x + i);
        __m512 nx = _mm512_sub_ps(_mm512_setzero_ps(), xv);
        nx = _mm512_max_ps(_mm512_set1_ps(-88.0f), _mm512_min_ps(_mm512_set1_ps(88.0f), nx));
        const __m512i e = _mm512_cvtps_epi32(
            _mm512_fmadd_ps(nx, _mm512_set1_ps(12102203.0f), _mm512_set1_ps(1065353216.0f)));
        const __m512 s = _mm512_div_ps(_mm512_set1_ps(1.0f), _mm512_add_ps(_mm512_set1_ps(1.0f), _mm512_castsi512_ps(e)));
        _mm512_storeu_ps(out + i, _mm512_mul_ps(xv, s));
    }
}
