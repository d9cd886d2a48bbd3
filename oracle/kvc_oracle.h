/*
 * kvc_oracle.h -- CPU restatement of the reference engine's KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline in bench.py.  Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg may load it; nothing in the product links it.
 *
 * Every function cites the reference file:line it restates.  Reference paths
 * are relative to the reference repository root (src/engine.cpp, ...).
 *
 * Layouts (all little-endian, bf16 stored as uint16_t bit patterns):
 *   contiguous cache  [pos][n_kv][d]   -- the reference layout of g_k_cache /
 *                                         g_v_cache (src/engine.cpp:81-84,
 *                                         index pos*kv_dim + kv_h*D + d at :3539)
 *   q, gate, out      [n_q][d] per token
 *   recurrent state   [v_heads][d_v][d_k] fp32 (src/engine.cpp:3282-3286)
 *   conv state        [3][channels] fp32, rows oldest -> newest (:3209-3232)
 *
 * Parity status of each function is listed in the header comment of
 * kvc_oracle.c.
 */
#ifndef KVC_ORACLE_H
#define KVC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numerics helpers ------------------------------------------------- */
uint64_t orc_splitmix64_next(uint64_t* state);
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t index); /* index-th output */
void orc_box_muller(uint64_t draw, float* z0, float* z1);
/* n values ~ N(0,1)*scale, RNE-rounded to bf16; element i uses draw i/2. */
void orc_fill_normal_bf16(uint16_t* dst, size_t n, uint64_t seed, float scale);
void orc_fill_normal_f32(float* dst, size_t n, uint64_t seed, float scale);
uint16_t orc_f32_to_bf16_rne(float x);
uint16_t orc_f32_to_bf16_trunc(float x); /* src/engine.cpp:248-252 */
float orc_bf16_to_f32(uint16_t b);       /* src/engine.cpp:253-258 */
void orc_f32_to_bf16_rne_n(const float* src, uint16_t* dst, size_t n);
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n);
float orc_fast_expf(float x);            /* src/engine.cpp:2349-2356 (fused, truncating) */
float orc_fast_expf_rne(float x);        /* the AVX-512 SiLU's exp, :2367-2373 (fused, RNE) */
float orc_sigmoid(float x, int mode);    /* mode 0 exact, 1 = :2358-2360 */
float orc_silu(float x, int mode);       /* mode 0 exact, 1 = :2366-2376 */

/* ---- cache append / gather (byte copies) ------------------------------ */
/* src/engine.cpp:3521-3525 (decode) and :2885-2889 (prefill, pos = g_pos+ti) */
void orc_cache_append(uint16_t* kc, uint16_t* vc, int n_kv, int d, int pos,
                      int n_tok, const uint16_t* k, const uint16_t* v);
void orc_cache_gather(const uint16_t* kc, const uint16_t* vc, int n_kv, int d,
                      int tok0, int n_tok, uint16_t* k_out, uint16_t* v_out);

/* ---- attention --------------------------------------------------------- */
/* GQA decode with online softmax and sigmoid gate, src/engine.cpp:3528-3564.
 * q [n_q][d] bf16; kc/vc [L][n_kv][d] bf16; gate [n_q][d] bf16 or NULL;
 * out [n_q][d] fp32.  gate_mode: 0 exact sigmoid, 1 Schraudolph (reference). */
void orc_decode_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                     int L, int n_q, int n_kv, int d, float scale,
                     const uint16_t* gate, int gate_mode, float* out);
/* Chunked prefill: row i attends to [0, pos0+i], src/engine.cpp:2843-2924.
 * q/gate [n][n_q][d]; out [n][n_q][d] fp32. */
void orc_prefill_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                      int pos0, int n, int n_q, int n_kv, int d, float scale,
                      const uint16_t* gate, int gate_mode, float* out);
/* Multi-threaded batch of decodes (CPU baseline, all-cores mode): seq s uses
 * kcs[s]/vcs[s] with length Ls[s]; q/out are [n_seqs][n_q][d]. Parallel over
 * (seq, q head).  threads <= 0 means the OpenMP default. */
void orc_decode_attn_batch(int n_seqs, const uint16_t* q,
                           const uint16_t* const* kcs,
                           const uint16_t* const* vcs, const int* Ls, int n_q,
                           int n_kv, int d, float scale, float* out, int threads);
int orc_max_threads(void);

/* ---- prefix cache rules ------------------------------------------------ */
/* Tokens erased from the head of an over-long prompt, src/engine.cpp:4048-4056. */
int orc_truncate_count(int n_prompt, int max_ctx, int max_tokens);
/* Reference reuse decision, src/engine.cpp:4058-4080: returns prefix_len and
 * sets *reset to 1 when reset_state() is called. */
int orc_reference_prefix(const int32_t* cached, int n_cached,
                         const int32_t* prompt, int n_prompt, int* reset);
int orc_lcp(const int32_t* a, int na, const int32_t* b, int nb);
/* Chained 64-bit block hash.  weak != 0 keeps only 4 bits (collision tests). */
uint64_t orc_block_hash(uint64_t parent, const int32_t* tok, int n, int weak);
uint64_t orc_hash_root(void);
void orc_hash_chain(const int32_t* tok, int n_blocks, int block, int weak,
                    uint64_t* out);
/* Build reuse rule: min(block-floor(LCP), snapshot boundary, n_prompt-1).
 * snap[k] != 0 when a state snapshot exists at boundary (k+1)*interval.
 * has_ssm == 0 (pure attention model) ignores snapshots. */
int orc_reuse_len(int lcp, int n_prompt, int block, int interval,
                  const uint8_t* snap, int n_snap, int has_ssm);

/* ---- K producer: per-head RMSNorm + partial RoPE ------------------------ */
/* RoPE tables, src/engine.cpp:2408-2419: for pos < max_ctx, p < rope_dim/2,
 * freq = 1/powf(base, 2p/rope_dim), theta = pos*freq (fp32), cos_t/sin_t
 * [max_ctx][rope_dim/2] = cosf/sinf(theta). */
void orc_rope_tables(int max_ctx, int rope_dim, float base, float* cos_t, float* sin_t);
/* Per-head RMSNorm in place, src/engine.cpp:3497-3512: ss = sum x^2 in index
 * order (fp32), r = 1/sqrtf(ss/d + eps), x[i] = x[i]*r*w[i]. */
void orc_rms_norm_head(float* x, int d, const float* w, float eps);
/* Partial NeoX RoPE in place on dims [0, rope_dim), pairs (p, p+rope_dim/2),
 * src/engine.cpp:2422-2432: x0' = x0 c - x1 s, x1' = x1 c + x0 s with the
 * table row of the token's position. */
void orc_rope_head(float* x, int rope_dim, const float* cos_row, const float* sin_row);
/* The attention producer of one token, src/engine.cpp:3485-3519 (decode) and
 * :2846-2883 (prefill): qkv row = [n_q][2][d] (q then gate of each head),
 * then k [n_kv][d], then v [n_kv][d].  Outputs (fp32): q [n_q][d] normed with
 * q_norm and roped, gate [n_q][d], k [n_kv][d] normed with k_norm and roped,
 * v [n_kv][d]; any output may be NULL. */
void orc_qkv_produce(const float* qkv, int n_q, int n_kv, int d, int rope_dim,
                     const float* q_norm, const float* k_norm, float eps,
                     const float* cos_row, const float* sin_row, float* q,
                     float* gate, float* k, float* v);

/* ---- recurrent state (snapshot semantics only) -------------------------- */
/* Conv window push: rows shift toward oldest, x becomes newest,
 * src/engine.cpp:3228-3230. state [3][channels]. */
void orc_conv_push(float* state, int rows, int channels, const float* x);
/* One Gated-DeltaNet head update, src/engine.cpp:3285-3305:
 *   S <- S*decay; sk_i = S_i.k; S_i += k * beta*(v_i - sk_i); o_i = S_i.q*s.
 * state [dv][dk]. */
void orc_deltanet_head_step(float* state, int dv, int dk, const float* q,
                            const float* k, const float* v, float decay,
                            float beta, float out_scale, float* out);

/* One Gated-DeltaNet layer for one token, in place on conv_state [3][C] and
 * ssm_state [n_v][dv][dk], src/engine.cpp:3197-3327 (decode) and :2600-2716
 * (prefill, per token).  proj = [C conv inputs (q n_k*dk | k n_k*dk | v
 * n_v*dv)][n_v*dv z][n_v alpha][n_v beta], C = 2*n_k*dk + n_v*dv.
 *   conv:  c = silu(s0 w0 + s1 w1 + s2 w2 + x w3) with w [4][C] tap-major,
 *          then the window push (:3204-3232)
 *   q, k of k-head vh % n_k: x / sqrtf(sum x^2 + eps) (:3261-3275)
 *   decay = exp(softplus(alpha + dt_bias) * a), beta = sigmoid(beta_raw)
 *          with softplus(b) = b for b > 20 (:3277-3281)
 *   delta rule per v-head row i: S_i *= decay; S_i += k beta (v_i - S_i.k);
 *          o_i = (S_i.q) * out_scale (:3283-3305)
 *   gated RMSNorm: out = o / sqrtf(mean(o^2) + eps) * norm_w * silu(z)
 *          (:3308-3320)
 * fast = 1 uses the reference's Schraudolph exp in softplus, sigmoid and SiLU
 * (:2349-2374); fast = 0 uses libm expf (the HIP path's semantics). */
void orc_deltanet_layer_step(float* conv_state, float* ssm_state, const float* proj,
                             const float* conv_w, const float* dt_bias, const float* a,
                             const float* norm_w, int n_v, int n_k, int dk, int dv,
                             float eps, float out_scale, int fast, float* out);

#ifdef __cplusplus
}
#endif
#endif
