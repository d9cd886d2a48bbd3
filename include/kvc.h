/*
 * kvc.h -- C ABI of the MI355X-native KV-cache path (libkvc.so, gfx950).
 *
 * The reference engine reaches its KV cache through static globals inside
 * src/engine.cpp; it has no FFI.  This header is the thin C layer its cache
 * sites call instead, one entry point per site:
 *
 *   kvc_create / kvc_destroy    cache + state allocation, src/engine.cpp:3835-3843
 *   kvc_seq_reset               reset_state(), src/engine.cpp:4164-4176
 *   kvc_seq_len                 g_pos, src/engine.cpp:70
 *   kvc_seq_reserve / _commit   g_pos += N / g_pos++ and g_cached_tokens
 *                               commit, src/engine.cpp:3039, :4106, :4118, :4150-4151
 *   kvc_prefix_match            prefix reuse in generate(), src/engine.cpp:4058-4080
 *   kvc_append                  K/V append, src/engine.cpp:3521-3525 and :2885-2889
 *   kvc_qkv_append              the attention producer feeding that append:
 *                               q/k per-head RMSNorm + partial RoPE, then the
 *                               append, src/engine.cpp:3485-3525 and :2846-2889
 *   kvc_decode_attn             GQA decode attention (+ fused append),
 *                               src/engine.cpp:3528-3564
 *   kvc_decode_step             the producer and the decode attention of one
 *                               decode token in one launch,
 *                               src/engine.cpp:3485-3564
 *   kvc_prefill_attn            per-token causal attention of a prefill batch,
 *                               src/engine.cpp:2892-2924
 *   kvc_prefill_step            the producer and the prefill attention of a
 *                               chunk, q and gate built inside the attention,
 *                               src/engine.cpp:2846-2924
 *   kvc_gather                  reads the cache in the reference layout
 *                               [pos][kv_head][d], src/engine.cpp:3539
 *   kvc_state_ptrs              g_ssm_state / g_conv_state, src/engine.cpp:86-94
 *   kvc_deltanet_step           the Gated-DeltaNet layer step that mutates that
 *                               state (conv1d + delta rule + gated RMSNorm),
 *                               src/engine.cpp:3197-3327 and :2600-2716
 *   kvc_snapshot_save/_restore  prefix-boundary copies of that state (new: the
 *                               reference can only extend one live sequence)
 *
 * Conventions (mirroring the reference's error style, src/engine.cpp:4040-4043):
 *   - every call returns int: KVC_OK (0) or a negative KVC_ERR_*; the message
 *     of the last error on the calling thread is kvc_last_error().  No C++
 *     exception crosses this ABI.  A null context is KVC_ERR_INVALID for every
 *     call but kvc_destroy, for which it is a no-op (KVC_OK), like free(NULL).
 *     A rejected device call launches nothing: every argument is checked
 *     before the first launch.
 *   - a context is single-threaded (the reference serialises generate() with a
 *     mutex, src/server.cpp:20).  Device work of one context must be ordered on
 *     one stream: the split-K workspace and its arrival counters are shared.
 *   - streams are hipStream_t passed as void* (NULL = the null stream); every
 *     device op is asynchronous and stream-ordered.
 *   - device pools, block tables and recurrent state belong to the library;
 *     q/k/v/gate/out buffers are caller-owned device memory; host arrays are
 *     borrowed for the duration of the call.
 *   - bf16 tensors are raw 16-bit patterns.  Shapes below use Hq = n_q_heads,
 *     Hkv = n_kv_heads, D = head_dim.
 */
#ifndef KVC_H
#define KVC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVC_ABI_VERSION 2

enum {
    KVC_OK = 0,
    KVC_ERR_INVALID = -1,     /* bad argument or shape */
    KVC_ERR_NO_DEVICE = -2,   /* device op on a host-only context / no GPU */
    KVC_ERR_NOMEM = -3,       /* block pool, snapshot pool or HBM exhausted */
    KVC_ERR_HIP = -4,         /* HIP runtime error (message has the detail) */
    KVC_ERR_RANGE = -5,       /* position or length out of range */
    KVC_ERR_UNSUPPORTED = -6, /* shape the compiled kernels do not cover */
    KVC_ERR_STATE = -7        /* call order violated (e.g. append unreserved) */
};

enum { KVC_DTYPE_F32 = 0, KVC_DTYPE_BF16 = 1 };

/* Test hook: keep 4 bits of the block hash so collisions are frequent; token
 * verification must still reject every false match. */
#define KVC_FLAG_WEAK_HASH 0x1u
/* Decode work split (tuning and test hooks).  By default a decode launch with
 * fewer than 256 (kv head, chunk) items splits each chunk's 256 output dims
 * over two workgroups; these force the split always or never.  They exclude
 * each other. */
#define KVC_FLAG_DECODE_SPLIT_D 0x2u
#define KVC_FLAG_DECODE_NO_SPLIT_D 0x4u
/* Transcendentals.  By default the library computes the reference's
 * Schraudolph (1999) approximations (src/engine.cpp:2349-2376): the output
 * gate sigma(gate) of decode and prefill attention (:3563, :2923), bit-exact
 * for every bf16 gate value with fast_sigmoidf's source expression evaluated
 * with an IEEE division; and in the Gated-DeltaNet step the SiLU of the conv
 * output and of z, the beta sigmoid and the exp in softplus (:2626, :2671,
 * :2674, :2714).  The reference's own -O3 -ffast-math -march=znver4 build
 * (Makefile:47; clang) departs from its source expressions: over every
 * finite bf16 gate, 17 of its sigma values differ from the IEEE quotient by
 * 1 ulp, its gated outputs round to the same bf16 values except for gates at
 * or below -85.5, where it yields NaN, and its AVX-512 SiLU differs by 1 ulp
 * on a fifth of the inputs (tests/test_fastmath_forms.py).  Parity with the
 * compiled reference is therefore within those bounds, not bit for bit.
 * This flag selects exact functions instead (hardware exp/log/rcp, within
 * 2 ulp). */
#define KVC_FLAG_EXACT_MATH 0x8u

typedef struct kvc_config {
    int32_t n_attn_layers;     /* full-attention layers (8, model_config.h:8,34) */
    int32_t n_ssm_layers;      /* Gated-DeltaNet layers (24); 0 = pure attention */
    int32_t n_q_heads;         /* 16 (model_config.h:15) */
    int32_t n_kv_heads;        /* 4  (model_config.h:16) */
    int32_t head_dim;          /* 256 (model_config.h:17) */
    int32_t block_tokens;      /* tokens per cache block: 32 */
    int32_t snapshot_interval; /* state snapshot every N tokens (256); 0 = off */
    int32_t max_seqs;          /* live sequence slots */
    int32_t max_seq_len;       /* tokens per sequence (block-table width) */
    int32_t ssm_v_heads;       /* 32  (model_config.h:28, dt_rank) */
    int32_t ssm_k_dim;         /* 128 (model_config.h:26, d_state) */
    int32_t ssm_v_dim;         /* 128 (model_config.h:29) */
    int32_t conv_rows;         /* 3 = conv_kernel - 1 (engine.cpp:93) */
    int32_t conv_channels;     /* 8192 (model_config.h:31) */
    int64_t pool_blocks;       /* blocks per layer; 0 = from pool_fraction */
    double pool_fraction;      /* share of free HBM for the K/V pools */
    int32_t snapshot_slots;    /* snapshot pool capacity (entries) */
    int32_t decode_chunk_blocks; /* split-K chunk in blocks; 0 = automatic */
    int32_t device;            /* HIP device; -1 = host-only bookkeeping */
    uint32_t flags;            /* KVC_FLAG_* */
    uint64_t alloc_seed;       /* 0: blocks handed out in order; else a seeded
                                  permutation of the free list */
    float rms_norm_eps;        /* q/k per-head RMSNorm eps (1e-6, model_config.h:18) */
    float rope_freq_base;      /* RoPE base (1e7, model_config.h:21) */
    int32_t rope_dim;          /* rotated dims per head, pairs (p, p + rope_dim/2)
                                  (64, model_config.h:22); 0 or a power of two
                                  in [8, head_dim] */
    int32_t reserved;          /* 0 */
} kvc_config;

typedef struct kvc_stats {
    int64_t pool_blocks;      /* blocks per layer */
    int64_t free_blocks;      /* on the free list */
    int64_t cached_blocks;    /* held only by the prefix index (evictable) */
    int64_t indexed_blocks;   /* registered in the prefix index */
    int64_t snapshots;        /* live snapshot entries */
    int64_t snapshot_slots;   /* capacity */
    int64_t hbm_bytes;        /* device bytes owned by the context */
    int64_t block_bytes;      /* bytes of one block of one layer (K or V) */
    int64_t prefix_hits;      /* tokens reused by kvc_prefix_match so far */
    int64_t evictions;        /* index blocks reclaimed under pressure */
} kvc_stats;

typedef struct kvc_ctx kvc_ctx;

/* ---- lifecycle ---------------------------------------------------------- */
void kvc_config_default(kvc_config* cfg); /* Qwen3.5-9B shapes */
int kvc_create(const kvc_config* cfg, kvc_ctx** out);
int kvc_destroy(kvc_ctx* ctx);
const char* kvc_last_error(void);
int kvc_get_stats(kvc_ctx* ctx, kvc_stats* out);
int kvc_abi_version(void);

/* ---- sequences ------------------------------------------------------------ */
int kvc_seq_create(kvc_ctx* ctx, int32_t* seq);
int kvc_seq_release(kvc_ctx* ctx, int32_t seq);
/* reset_state(): length 0, blocks released (src/engine.cpp:4164).  No memset
 * here: the recurrent/conv state of a created or reset sequence reads as zero
 * from its next use on (the Gated-DeltaNet step, a snapshot save or
 * kvc_state_ptrs zero-fill it first, on their stream), unless a snapshot
 * restore writes it.  A graph captured around such a first use would replay
 * the fill: capture after it. */
int kvc_seq_reset(kvc_ctx* ctx, int32_t seq);
int kvc_seq_len(kvc_ctx* ctx, int32_t seq, int32_t* len);
/* Drop tokens beyond len (rollback); len <= current length. */
int kvc_seq_truncate(kvc_ctx* ctx, int32_t seq, int32_t len);
/* Make positions [len, len+n_tok) writable for every seq (allocates blocks and
 * publishes new block-table entries on `stream`).  Until commit, appends and
 * attention address these pending positions. */
int kvc_seq_reserve(kvc_ctx* ctx, const int32_t* seqs, int32_t n_seqs,
                    int32_t n_tok, void* stream);
/* Advance every seq by its n_tok pending tokens (g_pos += N).  tokens
 * [n_seqs][n_tok] (host) extends the token history so full blocks enter the
 * prefix index; NULL commits without indexing (synthetic fills).  When a seq
 * lands on a multiple of snapshot_interval and tokens != NULL, a snapshot of
 * its recurrent state and last segment of K/V is taken on `stream`. */
int kvc_seq_commit(kvc_ctx* ctx, const int32_t* seqs, int32_t n_seqs,
                   int32_t n_tok, const int32_t* tokens, void* stream);

/* ---- prefix cache (host bookkeeping + device restore) ------------------- */
/* seq must be empty.  Finds the longest verified block-chain prefix of
 * tokens[0..n) in the index, caps it at n-1 and, with recurrent layers, at the
 * last snapshot boundary; maps those blocks into seq (zero copy), restores the
 * snapshot's recurrent/conv state and any K/V segment whose blocks were
 * evicted, and sets the seq length to *reuse_len. */
int kvc_prefix_match(kvc_ctx* ctx, int32_t seq, const int32_t* tokens,
                     int32_t n, int32_t* reuse_len, void* stream);

/* ---- device ops ----------------------------------------------------------- */
/* k, v: bf16 [n_seqs][n_tok][Hkv][D] written at pending positions
 * [len, len+n_tok) of layer `layer` (positions must be reserved). */
int kvc_append(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
               int32_t n_seqs, int32_t n_tok, const void* k, const void* v,
               void* stream);
/* Attention producer + append (src/engine.cpp:3485-3525 decode, :2846-2889
 * prefill).  qkv holds the attention projection row of n_tok tokens per seq,
 * [n_seqs][n_tok][row] with row = Hq*2*D + 2*Hkv*D laid out as the
 * reference's: [Hq][q | gate][D], then k [Hkv][D], then v [Hkv][D]; fp32 or
 * bf16 by in_dtype.  For each token at its pending position (as kvc_append):
 * q and k get per-head RMSNorm (x * 1/sqrt(mean(x^2) + eps) * w, weights
 * q_norm / k_norm: device fp32 [D]) and partial NeoX RoPE over dims
 * [0, rope_dim) with the pairs (p, p + rope_dim/2) at the token's position
 * (cos/sin tables built at kvc_create the way src/engine.cpp:2408-2419 builds
 * them); k and v are appended to layer's cache as bf16 (RNE); q and gate are
 * written as bf16 [n_seqs][n_tok][Hq][D] to q_out / gate_out (either may be
 * NULL), ready for kvc_prefill_attn / kvc_decode_attn.  With both NULL only
 * the k / v part of each row is read (the K/V side of kvc_prefill_step). */
int kvc_qkv_append(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                   int32_t n_seqs, int32_t n_tok, const void* qkv,
                   int32_t in_dtype, const void* q_norm, const void* k_norm,
                   void* q_out, void* gate_out, void* stream);
/* One query token per seq.  q: bf16 [n_seqs][Hq][D].  Attends over
 * [0, len + pending).  If k_new/v_new (bf16 [n_seqs][Hkv][D]) are given, they
 * are first written at position len + pending - 1 (fused append; reserve 1
 * token).  gate: NULL or bf16 [n_seqs][Hq][D], out *= sigmoid(gate)
 * (src/engine.cpp:3561-3563).  out: [n_seqs][Hq][D] in out_dtype.
 * score = (q.k) * scale (attn_scale = 1/16, model_config.h:40). */
int kvc_decode_attn(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                    int32_t n_seqs, const void* q, const void* k_new,
                    const void* v_new, const void* gate, void* out,
                    int32_t out_dtype, float scale, void* stream);
/* No counterpart in the reference.  kvc_decode_attn for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments, semantics and results
 * (bit for bit: same work split and kernels), but the split-K partials and
 * arrival counters live in the library's static per-GPU workspace -- a
 * file-scope __device__ array of 4096 split-K items plus counters, 17.6 MB,
 * held by each GPU the library runs on until the process ends -- instead of
 * the context's.  The call allocates nothing.  A launch needing more than
 * 4096 items (chunks x kv heads x output-dim parts) is refused with
 * KVC_ERR_RANGE before anything runs; the automatic split (decode_chunk_blocks
 * = 0) never needs more, for 64 sequences of any length, with or without a
 * forced output-dim split (KVC_FLAG_DECODE_SPLIT_D).  Every call on one GPU shares
 * that workspace: calls that overlap on one GPU (other streams, other
 * contexts, other host threads) race and must be serialised by the caller. */
int kvc_decode_attn_static(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                           int32_t n_seqs, const void* q, const void* k_new,
                           const void* v_new, const void* gate, void* out,
                           int32_t out_dtype, float scale, void* stream);
/* One decode step of an attention layer in one launch: kvc_qkv_append's
 * producer for one token per seq (src/engine.cpp:3485-3525: q/k per-head
 * RMSNorm + partial RoPE at position len + pending - 1, k and v appended
 * there; reserve 1 token) fused into kvc_decode_attn's gated attention
 * (src/engine.cpp:3528-3564, out *= sigmoid(gate)).  qkv: projection rows
 * [n_seqs][Hq*2*D + 2*Hkv*D] in kvc_qkv_append's layout, fp32 or bf16 by
 * in_dtype; q_norm, k_norm: device fp32 [D]; out: [n_seqs][Hq][D] in
 * out_dtype.  Same bits as kvc_qkv_append (same rows, one token) followed by
 * kvc_decode_attn with the produced q and gate and with the appended k / v
 * rows passed as k_new / v_new.  Uses the context's split-K workspace. */
int kvc_decode_step(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                    int32_t n_seqs, const void* qkv, int32_t in_dtype,
                    const void* q_norm, const void* k_norm, void* out,
                    int32_t out_dtype, float scale, void* stream);
/* Causal chunked prefill.  The n_q query tokens of seq s sit at positions
 * [len_s + pending_s - n_q, len_s + pending_s) (their K/V appended already);
 * row i attends to keys [0, pos_i].  q/gate: bf16 [n_seqs][n_q][Hq][D];
 * out: [n_seqs][n_q][Hq][D]. */
int kvc_prefill_attn(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                     int32_t n_seqs, int32_t n_q, const void* q,
                     const void* gate, void* out, int32_t out_dtype,
                     float scale, void* stream);
/* A prefill chunk's attention step from its projection rows: kvc_qkv_append's
 * producer (src/engine.cpp:2846-2889: k and v normalized / rotated and
 * appended at the chunk's pending positions) and kvc_prefill_attn's gated
 * causal attention (src/engine.cpp:2892-2924), with q and the gate built from
 * the rows inside the attention launch instead of going through memory.
 * qkv: [n_seqs][n_q][Hq*2*D + 2*Hkv*D] in kvc_qkv_append's layout, fp32 or
 * bf16 by in_dtype; q_norm, k_norm: device fp32 [D]; out: [n_seqs][n_q][Hq][D]
 * in out_dtype.  Same bits (output and cache) as kvc_qkv_append with q_out and
 * gate_out followed by kvc_prefill_attn on them.  Two launches. */
int kvc_prefill_step(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                     int32_t n_seqs, int32_t n_q, const void* qkv,
                     int32_t in_dtype, const void* q_norm, const void* k_norm,
                     void* out, int32_t out_dtype, float scale, void* stream);
/* Copy positions [tok0, tok0 + n_tok[s]) of each seq into contiguous bf16
 * [n_tok][Hkv][D] (the reference cache layout); outputs are packed back to
 * back in seq order.  Bit-exact. */
int kvc_gather(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
               int32_t n_seqs, int32_t tok0, const int32_t* n_tok,
               void* k_out, void* v_out, void* stream);

/* Integrity checksums of each seq's cached K/V in one layer, one per 16-KiB
 * (block, K|V, kv head) unit (no counterpart in the reference; a cheap check
 * that a reused, restored or copied prefix holds the bytes it should, and
 * which block does not).  out (device memory, uint64) receives, for each seq
 * in order, ceil((len + pending) / 32) x 2 x Hkv entries ordered [block][K, V]
 * [kv head]; entry = sum(w_j) in the low 32 bits and sum(w_j ^ j) in the
 * high 32 bits, both mod 2^32, over the 32-bit words w_j of the unit's
 * [token][d] rows (j = token * D/2 + word) for tokens below len + pending.
 * Reads whole blocks and writes 8 B per unit: the bench's single-launch read
 * floor and a counter calibration of known size. */
int kvc_kv_checksum(kvc_ctx* ctx, int32_t layer, const int32_t* seqs,
                    int32_t n_seqs, uint64_t* out, void* stream);

/* ---- recurrent state + snapshots ---------------------------------------- */
/* Live state of seq for Gated-DeltaNet layer ssm_layer: rec = fp32
 * [v_heads][v_dim][k_dim], conv = fp32 [conv_rows][conv_channels]. */
int kvc_state_ptrs(kvc_ctx* ctx, int32_t seq, int32_t ssm_layer, void** rec,
                   void** conv);
/* Gated-DeltaNet step of n_tok tokens per seq, in place on the state above
 * (src/engine.cpp:3197-3327 decode, :2600-2716 prefill, token by token).
 * proj: [n_seqs][n_tok][row], row = conv_channels raw inputs (q | k | v) +
 * v_heads*v_dim z + v_heads alpha + v_heads beta (12352 at the Qwen3.5
 * shapes), fp32 or bf16 by in_dtype.  Device fp32 weights: conv_w
 * [conv_rows + 1][conv_channels] tap-major (taps 0..2 on the window, oldest
 * first, tap 3 on the input), dt_bias [v_heads], a [v_heads] (decay =
 * exp(softplus(alpha + dt_bias) * a)), norm_w [v_dim].  out: [n_seqs][n_tok]
 * [v_heads * v_dim], fp32 or bf16 (RNE) by out_dtype: the gated-RMSNorm
 * output (o / rms(o) * norm_w * silu(z), o = S q / 11.3137).  By default the
 * SiLU of the conv output and of z, the beta sigmoid and the exp inside
 * softplus are the reference's Schraudolph forms (:2349-2374, :2626, :2671,
 * :2674, :2714); beta's division is correctly rounded, as the reference's
 * scalar fast_sigmoidf divides, and the SiLU's reciprocal is v_rcp_f32
 * (1 ulp), as the reference's fast-math AVX-512 SiLU takes an approximate
 * reciprocal.  The decay's exp and the softplus log are the hardware
 * exp2/log2 (within 2 ulp of libm's expf / logf).  With KVC_FLAG_EXACT_MATH
 * the SiLU, sigmoid and softplus use the hardware exp2/log2/reciprocal
 * (each within 2 ulp of the exact function) instead.  Built for
 * 32 v-heads, 16 k-heads, 128 x 128 heads, a 3-row window and 8192 channels
 * (KVC_ERR_UNSUPPORTED otherwise); one seq's n_tok rows of proj must span
 * less than 2 GiB (KVC_ERR_RANGE otherwise). */
int kvc_deltanet_step(kvc_ctx* ctx, int32_t ssm_layer, const int32_t* seqs,
                      int32_t n_seqs, int32_t n_tok, const void* proj,
                      int32_t in_dtype, const void* conv_w, const void* dt_bias,
                      const void* a, const void* norm_w, void* out,
                      int32_t out_dtype, void* stream);
/* Save each seq's state and the K/V of its last snapshot_interval tokens (all
 * attention layers).  Each seq length must be a positive multiple of
 * snapshot_interval.  snap_ids receives one id per seq.  Bit-exact copies. */
int kvc_snapshot_save(kvc_ctx* ctx, const int32_t* seqs, int32_t n_seqs,
                      int32_t* snap_ids, void* stream);
/* Restore snapshot snap_ids[i] (taken at boundary B) into seqs[i]: the seq must
 * hold at least B - snapshot_interval tokens; it is cut to that length, the
 * segment's K/V is written into fresh blocks, the state is copied in, and the
 * length becomes B. */
int kvc_snapshot_restore(kvc_ctx* ctx, const int32_t* seqs,
                         const int32_t* snap_ids, int32_t n_seqs, void* stream);
int kvc_snapshot_release(kvc_ctx* ctx, int32_t snap_id);

/* ---- synthetic data + sync ---------------------------------------------- */
/* Fill every block of every layer's K and V pool with N(0,1) bf16 (splitmix64
 * + Box-Muller keyed by element index, RNE rounding). */
int kvc_pool_fill_normal(kvc_ctx* ctx, uint64_t seed, void* stream);
/* Fill n bf16 values at dst (device) with N(0,1)*scale, same generator. */
int kvc_fill_normal_bf16(kvc_ctx* ctx, void* dst, int64_t n, uint64_t seed,
                         float scale, void* stream);
int kvc_sync(kvc_ctx* ctx, void* stream);

#ifdef __cplusplus
}
#endif
#endif
