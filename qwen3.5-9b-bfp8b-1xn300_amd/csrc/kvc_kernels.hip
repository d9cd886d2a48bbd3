// kvc_kernels.hip -- gfx950 kernels of the KV-cache path: block-table update,
// append, split-K GQA decode attention (with fused append), causal prefill
// attention, gather, snapshot copy, synthetic fill.
//
// All K/V traffic is bf16; arithmetic is fp32 (v_dot2_f32_bf16 for q.k).
// Softmax runs in the log2 domain: s2 = (q.k) * scale * log2(e), p = 2^(s2-m).
#include <atomic>
#include <mutex>
#include "kvc_device.h"
#include "kvc_internal.h"

namespace kvc {

constexpr int kWaves = 4;           // waves per decode workgroup (each takes 8 tokens of a block)
constexpr int kTokPerWave = kBlockTok / kWaves;  // 8 tokens of a block per wave
constexpr float kNegBig = -1.0e30f;
constexpr float kRescaleSlack = 8.0f;  // lazy rescale: p may reach 2^8

// ---------------------------------------------------------------------------
// Block-table update: entries ride in the argument block.
__global__ void table_update_kernel(TableUpdateArgs a) {
    for (int i = threadIdx.x; i < a.n; i += blockDim.x) a.table[a.index[i]] = a.block[i];
}

// ---------------------------------------------------------------------------
// Per-wave online-softmax state.  m[g] is wave-uniform (log2 domain); l_lane
// is this lane's share of the softmax denominator for its own head; acc[g][j]
// holds output dims d = lane*4 + j of q head g of the group.
struct WaveState {
    float m[kGroup];
    float l[kGroup];  // filled by finalize_l
    float l_lane;
    float acc[kGroup][4];
};

// One block's K/V as held by one wave (the wave owns 8 of the block's 32
// tokens) of a workgroup that produces output dims part dpart of NP (NP = 1:
// all 256 dims; NP = 2: 128).  Lane = 16*ts + c (ts = 0..3, c = 0..15):
//   k[2r + j]: token 4r + ts of the wave's 8, dims (c + 16j)*8 .. +7 (16 B)
//   v[i]:      token tsub*(8/NP) + i of the wave's 8, dims
//              dpart*256/NP + dl*4 .. +3 (8 B), with dl = lane % (64/NP) and
//              tsub = lane / (64/NP); NP = 1 gives token i, dims lane*4 ..
template <int NP>
struct BlockRegs {
    uint4 k[4];
    uint2 v[kTokPerWave / NP];
};

__device__ __forceinline__ void init_state(WaveState& st) {
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        st.m[g] = kNegBig;
        st.l[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) st.acc[g][j] = 0.f;
    }
    st.l_lane = 0.f;
}

// Load the wave's share of one (block, kv_head) unit with unconditional
// 16-B / 8-B loads (every slot of an allocated unit is addressable; slots past
// the sequence end are masked in compute_block).  With NP > 1 the sibling
// workgroups of a chunk (same XCD, dispatched together) all read its K, so K
// is loaded to stay in L2; V, read once, streams past it.
template <int NP>
__device__ __forceinline__ void load_block(BlockRegs<NP>& r, const uint16_t* __restrict__ ku,
                                           const uint16_t* __restrict__ vu, int wave, int lane, int dpart) {
    const int ts = lane >> 4, c = lane & 15;
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int t = wave * kTokPerWave + rr * 4 + ts;
            const uint16_t* src = ku + t * kHeadDim + (c + 16 * j) * 8;
            if constexpr (NP == 1) {
                const u32x4 y = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                r.k[rr * 2 + j] = make_uint4(y[0], y[1], y[2], y[3]);
            } else {
                r.k[rr * 2 + j] = *reinterpret_cast<const uint4*>(src);
            }
        }
    }
    constexpr int kLanesD = 64 / NP, kTokL = kTokPerWave / NP;
    const int dl = lane % kLanesD, tsub = lane / kLanesD;
#pragma unroll
    for (int i = 0; i < kTokL; i++) {
        const u32x2 y = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(
            vu + (wave * kTokPerWave + tsub * kTokL + i) * kHeadDim + dpart * (kHeadDim / NP) + dl * 4));
        r.v[i] = make_uint2(y[0], y[1]);
    }
}

// DPP lane moves inside rows of 16 (no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowRor8 = 0x128;    // lane ^ 8 inside a row of 16
constexpr int kDppRowMirror = 0x140;  // lane -> 15 - lane inside a row
constexpr int kDppHalfMirror = 0x141; // lane -> 7 - lane inside 8 lanes

// x(lane) op x(lane ^ 16) / x(lane ^ 32) through v_permlane*_swap.
__device__ __forceinline__ float sum_xor16(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// x rounded to bf16 (RNE) and widened back; x finite.
__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(cvt_pk_bf16(x, 0.f) << 16); }

// Scores, online softmax update and P.V for one block held in registers.
// qv[g][j][i]: packed bf16 pairs of q head g, dims (c + 16j)*8 + 2i, +1.
// lds_p16: per-wave 32 bf16 p values laid out [g][token].
template <int NP>
__device__ __forceinline__ void compute_block(BlockRegs<NP>& r, const uint32_t (&qv)[kGroup][2][4],
                                              int n_valid, float scale_log2, uint16_t* lds_p16,
                                              WaveState& st, int wave, int lane) {
    const int ts = lane >> 4, c = lane & 15;
    // partial q.k over this lane's 16 dims: a[4*rr + g] for tokens 4rr + ts
    float a[8];
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
#pragma unroll
        for (int g = 0; g < kGroup; g++) {
            float x = 0.f;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint4 k = r.k[rr * 2 + j];
                x = dot2_bf16(qv[g][j][0], k.x, x);
                x = dot2_bf16(qv[g][j][1], k.y, x);
                x = dot2_bf16(qv[g][j][2], k.z, x);
                x = dot2_bf16(qv[g][j][3], k.w, x);
            }
            a[rr * 4 + g] = x;
        }
    }
    // transpose-reduce over the 16 lanes of a token (c bits 3, 2, 1, then 0).
    // Each step pairs lanes that differ in the step's bit and agree on the
    // bits already decided; the mirror moves also flip lower, still
    // undecided bits, which is harmless.
#define KVC_TR(BIT, N, CTRL)                                             \
    {                                                                    \
        const bool sel = (c >> BIT) & 1;                                 \
        _Pragma("unroll") for (int j = 0; j < N / 2; j++) {              \
            const float send = sel ? a[j] : a[j + N / 2];                \
            const float keep = sel ? a[j + N / 2] : a[j];                \
            a[j] = keep + dpp<CTRL>(send);                               \
        }                                                                \
    }
    KVC_TR(3, 8, kDppRowMirror)
    KVC_TR(2, 4, kDppHalfMirror)
    KVC_TR(1, 2, kDppXor2)
#undef KVC_TR
    float sc = a[0] + dpp<kDppXor1>(a[0]);
    const int vi = (c >> 1) & 7;
    const int my_g = vi & 3;
    const int t_loc = (vi >> 2) * 4 + ts;  // token within the wave's 8
    const bool valid = wave * kTokPerWave + t_loc < n_valid;
    sc = valid ? sc * scale_log2 : kNegBig;

    // lazy running max: rescale only when a score passes its head's max by
    // more than the slack (p stays <= 2^slack)
    float m_own = st.m[0];
#pragma unroll
    for (int g = 1; g < kGroup; g++) m_own = (my_g == g) ? st.m[g] : m_own;
    if (__builtin_amdgcn_ballot_w64(sc > m_own + kRescaleSlack) != 0) {
        float mx = sc;
        mx = fmaxf(mx, dpp<kDppRowRor8>(mx));
        mx = max_xor16(mx);
        mx = max_xor32(mx);
        float c_own = 1.f;
#pragma unroll
        for (int g = 0; g < kGroup; g++) {
            const float mb = readlane(mx, g << 1);
            if (mb > st.m[g] + kRescaleSlack) {
                const float cg = fast_exp2(st.m[g] - mb);
#pragma unroll
                for (int j = 0; j < 4; j++) st.acc[g][j] *= cg;
                c_own = (my_g == g) ? cg : c_own;
                st.m[g] = mb;
            }
        }
        st.l_lane *= c_own;
        m_own = st.m[0];
#pragma unroll
        for (int g = 1; g < kGroup; g++) m_own = (my_g == g) ? st.m[g] : m_own;
    }
    // p rounded to bf16 once; the same value feeds l and P.V
    const float p = valid ? bf16_round(fast_exp2(sc - m_own)) : 0.f;
    st.l_lane += p;

    // broadcast p as bf16 [g][token] through LDS
    wave_lds_sync();
    if ((c & 1) == 0) lds_p16[my_g * kTokPerWave + t_loc] = (uint16_t)(__float_as_uint(p) >> 16);
    wave_lds_sync();
    // this lane's tokens t0 .. t0 + 8/NP - 1 of the wave's 8; pw[g][k] =
    // (p[g][t0 + 2k], p[g][t0 + 2k + 1])
    constexpr int kTokL = kTokPerWave / NP;
    const int t0 = (lane / (64 / NP)) * kTokL;
    uint32_t pw[kGroup][kTokL / 2];
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        if constexpr (NP == 1) {
            const uint4 x = *reinterpret_cast<const uint4*>(lds_p16 + g * kTokPerWave);
            pw[g][0] = x.x;
            pw[g][1] = x.y;
            pw[g][2] = x.z;
            pw[g][3] = x.w;
        } else {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(lds_p16 + g * kTokPerWave + t0);
#pragma unroll
            for (int k = 0; k < kTokL / 2; k++) pw[g][k] = src[k];
        }
    }

    if (n_valid < (wave + 1) * kTokPerWave) {  // partial block: stale slots may hold NaN bits
#pragma unroll
        for (int i = 0; i < kTokL; i++)
            if (wave * kTokPerWave + t0 + i >= n_valid) r.v[i] = make_uint2(0, 0);
    }
    // P.V on token pairs with v_dot2_f32_bf16: (v[2k][d], v[2k+1][d]) packed
#pragma unroll
    for (int k = 0; k < kTokL / 2; k++) {
        const uint2 v0 = r.v[2 * k], v1 = r.v[2 * k + 1];
        uint32_t vp[4];
        vp[0] = __builtin_amdgcn_perm(v1.x, v0.x, 0x05040100u);
        vp[1] = __builtin_amdgcn_perm(v1.x, v0.x, 0x07060302u);
        vp[2] = __builtin_amdgcn_perm(v1.y, v0.y, 0x05040100u);
        vp[3] = __builtin_amdgcn_perm(v1.y, v0.y, 0x07060302u);
#pragma unroll
        for (int g = 0; g < kGroup; g++) {
#pragma unroll
            for (int j = 0; j < 4; j++) st.acc[g][j] = dot2_bf16(pw[g][k], vp[j], st.acc[g][j]);
        }
    }
}

// Reduce the per-lane denominators to st.l[g] (wave-uniform).
__device__ __forceinline__ void finalize_l(WaveState& st) {
    float x = st.l_lane;
    x += dpp<kDppRowRor8>(x);
    x = sum_xor16(x);
    x = sum_xor32(x);
#pragma unroll
    for (int g = 0; g < kGroup; g++) st.l[g] = readlane(x, g << 1);
}

__device__ __forceinline__ void load_q(uint32_t (&qv)[kGroup][2][4], const uint16_t* qhead0, int lane) {
    const int c = lane & 15;
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint4 x = *reinterpret_cast<const uint4*>(qhead0 + g * kHeadDim + (c + 16 * j) * 8);
            qv[g][j][0] = x.x;
            qv[g][j][1] = x.y;
            qv[g][j][2] = x.z;
            qv[g][j][3] = x.w;
        }
    }
}

// LDS for one workgroup: per-wave p broadcast + cross-wave merge area.
struct DecodeSmem {
    uint16_t p16[kWaves][32];
    float acc[kWaves][kGroup][kHeadDim];
    float ml[kWaves][kGroup][2];
    int last;
};

// Merge the 4 waves' states; thread t ends with (M, L, A[4]) of head
// g = t >> 6, dims (t & 63) * 4 .. +3.
__device__ __forceinline__ void merge_waves(const WaveState& st, DecodeSmem& sm, int wave, int lane,
                                            float& M, float& L, float (&A)[4]) {
#pragma unroll
    for (int g = 0; g < kGroup; g++)
        *reinterpret_cast<float4*>(&sm.acc[wave][g][lane * 4]) =
            make_float4(st.acc[g][0], st.acc[g][1], st.acc[g][2], st.acc[g][3]);
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < kGroup; g++) {
            sm.ml[wave][g][0] = st.m[g];
            sm.ml[wave][g][1] = st.l[g];
        }
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int g = t >> 6, d0 = (t & 63) * 4;
    M = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, sm.ml[w][g][0]);
    L = 0.f;
    A[0] = A[1] = A[2] = A[3] = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        const float wt = fast_exp2(sm.ml[w][g][0] - M);
        L = fmaf(wt, sm.ml[w][g][1], L);
        const float4 x = *reinterpret_cast<const float4*>(&sm.acc[w][g][d0]);
        A[0] = fmaf(wt, x.x, A[0]);
        A[1] = fmaf(wt, x.y, A[1]);
        A[2] = fmaf(wt, x.z, A[2]);
        A[3] = fmaf(wt, x.w, A[3]);
    }
}

// sigmoid to within a few ulp: v_exp_f32 and v_rcp_f32 (KVC_FLAG_EXACT_MATH)
__device__ __forceinline__ float sigmoidf_exact(float x) {
    return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-x * 1.4426950408889634f));
}
// The output gate sigma(gate) (src/engine.cpp:3563 decode, :2923 prefill):
// the reference's Schraudolph sigmoid by default, the exact one on request.
// ref is a kernel argument, uniform over the launch.
__device__ __forceinline__ float gate_sigmoid(float x, int ref) {
    return ref ? sigmoid_ref(x) : sigmoidf_exact(x);
}

// sigmoid(gate) of dims d0 .. d0 + 3 from their bf16 values gw
__device__ __forceinline__ void gate_factors(uint2 gw, int gate_ref, float (&gs)[4]) {
    gs[0] = gate_sigmoid(bf16lo(gw.x), gate_ref);
    gs[1] = gate_sigmoid(bf16hi(gw.x), gate_ref);
    gs[2] = gate_sigmoid(bf16lo(gw.y), gate_ref);
    gs[3] = gate_sigmoid(bf16hi(gw.y), gate_ref);
}

// out row = A / L (* gs, the gate factors of dims d0 .. d0 + 3, when
// has_gate), written as bf16 (RNE) or fp32.
__device__ __forceinline__ void write_out(void* out, int out_bf16, size_t row_off, int d0, bool has_gate,
                                          const float (&gs)[4], float L, const float (&A)[4]) {
    const float inv = __builtin_amdgcn_rcpf(L);
    float o[4] = {A[0] * inv, A[1] * inv, A[2] * inv, A[3] * inv};
    if (has_gate) {
        o[0] *= gs[0];
        o[1] *= gs[1];
        o[2] *= gs[2];
        o[3] *= gs[3];
    }
    if (out_bf16) {
        uint2 w;
        w.x = pack_bf16x2(o[0], o[1]);
        w.y = pack_bf16x2(o[2], o[3]);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + row_off + d0) = w;
    } else {
        *reinterpret_cast<float4*>(static_cast<float*>(out) + row_off + d0) =
            make_float4(o[0], o[1], o[2], o[3]);
    }
}

// Fused append: copy the new token's K and V rows of kv head h (512 B each)
// into its pool slot.  Run by the one workgroup whose chunk holds the slot,
// after its block walk (which never reads that slot), so no store sits inside
// the load pipeline.
// piece = the 16 B of thread t < 64: K piece t (t < 32) or V piece t - 32;
// blk = the pool block that holds position pos.
__device__ __forceinline__ void append_new_token(uint16_t* kpool, uint16_t* vpool, int blk, int h, int pos,
                                                 const u32x4& piece) {
    const int t = threadIdx.x;
    if (t >= 64) return;
    const size_t off = (((size_t)blk * kKvHeads + h) * kBlockTok + pos % kBlockTok) * kHeadDim;
    const int kv = t >> 5, part = t & 31;
    uint16_t* dst = (kv ? vpool : kpool) + off + part * 8;
    *reinterpret_cast<u32x4*>(dst) = piece;
}

// ---------------------------------------------------------------------------
// Walk blocks [blk0, blk0 + n_blk) of one (sequence, kv head); keys at
// positions >= L are masked.  Block ids are fetched once per
// 64 blocks into a VGPR and read back per block with v_readlane, so no table
// load sits in the pipeline; the first window's ids (first_ids: lane i holds
// block blk0 + i, at least for i < min(64, n_blk)) come from the caller,
// which requests them before its other loads.  Blocks go in straight-line groups of 4 over 2
// register buffers (the wait before each compute covers exactly the buffer it
// reads while the other stays in flight); a window's last 1-3 blocks take a
// straight-line tail of their own, so no load is ever issued for a block that
// is not computed.  With PREP, prep() runs once, after the first blocks' loads
// are issued and before anything uses qv (alone when there is no block): the
// producing decode step builds qv there, so its arithmetic overlaps the first
// loads.  That first group is peeled off the loop, so whatever prep() reads
// is dead for the rest of the walk.
template <int NP, bool PREP, typename Prep>
__device__ __forceinline__ void walk_blocks(const uint16_t* __restrict__ kpool,
                                            const uint16_t* __restrict__ vpool,
                                            const int32_t* __restrict__ trow, int h, int blk0,
                                            int n_blk, int L, const uint32_t (&qv)[kGroup][2][4],
                                            float scale_log2, uint16_t* lds_p, WaveState& st,
                                            int wave, int lane, int dpart, int first_ids, Prep&& prep) {
    BlockRegs<NP> r0, r1;
    constexpr size_t kUnitElems = (size_t)kBlockTok * kHeadDim;
#define KVC_LOAD_WIN(R, I)                                                                          \
    {                                                                                               \
        const size_t off_ = ((size_t)__builtin_amdgcn_readlane(my_id, (I)) * kKvHeads + h) * kUnitElems; \
        load_block<NP>(R, kpool + off_, vpool + off_, wave, lane, dpart);                          \
    }
#define KVC_NV(I) min(kBlockTok, L - (blk0 + w0 + (I)) * kBlockTok)
#define KVC_COMPUTE(R, I) compute_block<NP>(R, qv, KVC_NV(I), scale_log2, lds_p, st, wave, lane)
// blocks [i, wn) of the window at w0: groups of 4, then a tail of 1-3
#define KVC_GROUPS                                  \
    for (; i + 4 <= wn; i += 4) {                   \
        KVC_LOAD_WIN(r0, i)                         \
        KVC_LOAD_WIN(r1, i + 1)                     \
        KVC_COMPUTE(r0, i);                         \
        KVC_LOAD_WIN(r0, i + 2)                     \
        KVC_COMPUTE(r1, i + 1);                     \
        KVC_LOAD_WIN(r1, i + 3)                     \
        KVC_COMPUTE(r0, i + 2);                     \
        KVC_COMPUTE(r1, i + 3);                     \
    }                                               \
    {                                               \
        const int rem = wn - i;                     \
        if (rem == 1) {                             \
            KVC_LOAD_WIN(r0, i)                     \
            KVC_COMPUTE(r0, i);                     \
        } else if (rem == 2) {                      \
            KVC_LOAD_WIN(r0, i)                     \
            KVC_LOAD_WIN(r1, i + 1)                 \
            KVC_COMPUTE(r0, i);                     \
            KVC_COMPUTE(r1, i + 1);                 \
        } else if (rem == 3) {                      \
            KVC_LOAD_WIN(r0, i)                     \
            KVC_LOAD_WIN(r1, i + 1)                 \
            KVC_COMPUTE(r0, i);                     \
            KVC_LOAD_WIN(r0, i + 2)                 \
            KVC_COMPUTE(r1, i + 1);                 \
            KVC_COMPUTE(r0, i + 2);                 \
        }                                           \
    }
    // the first window is peeled off the loop in both forms, so that its ids
    // (first_ids) are no loop-carried value: the wait for them then covers
    // only the loads issued before them
    if constexpr (PREP) {
        // first window: the loads of blocks 0 and 1 (those that exist), prep
        // (inlined once: it runs once per launch, so its code stays small),
        // then the first group or the whole short window
        const int w0 = 0;
        const int wn = min(64, n_blk);
        const int my_id = first_ids;
        // blocks 0 and 1 are requested on every path (a short window's
        // missing ids read 0: block 0 of the pool, loaded and not used), so
        // the number of loads in flight at prep is fixed and prep waits for
        // its own inputs without waiting for these
        const int id0 = __builtin_amdgcn_readlane(my_id, 0), id1 = __builtin_amdgcn_readlane(my_id, 1);
        load_block<NP>(r0, kpool + ((size_t)id0 * kKvHeads + h) * kUnitElems,
                       vpool + ((size_t)id0 * kKvHeads + h) * kUnitElems, wave, lane, dpart);
        load_block<NP>(r1, kpool + ((size_t)id1 * kKvHeads + h) * kUnitElems,
                       vpool + ((size_t)id1 * kKvHeads + h) * kUnitElems, wave, lane, dpart);
        prep();
        if (wn >= 4) {
            KVC_COMPUTE(r0, 0);
            KVC_LOAD_WIN(r0, 2)
            KVC_COMPUTE(r1, 1);
            KVC_LOAD_WIN(r1, 3)
            KVC_COMPUTE(r0, 2);
            KVC_COMPUTE(r1, 3);
            int i = 4;
            KVC_GROUPS
        } else if (wn == 3) {
            KVC_COMPUTE(r0, 0);
            KVC_LOAD_WIN(r0, 2)
            KVC_COMPUTE(r1, 1);
            KVC_COMPUTE(r0, 2);
        } else if (wn == 2) {
            KVC_COMPUTE(r0, 0);
            KVC_COMPUTE(r1, 1);
        } else if (wn == 1) {
            KVC_COMPUTE(r0, 0);
        }
    } else if (n_blk > 0) {
        const int w0 = 0;
        const int wn = min(64, n_blk);
        const int my_id = first_ids;
        int i = 0;
        KVC_GROUPS
    }
    for (int w0 = 64; w0 < n_blk; w0 += 64) {
        const int wn = min(64, n_blk - w0);
        const int my_id = lane < wn ? trow[blk0 + w0 + lane] : 0;
        int i = 0;
        KVC_GROUPS
    }
#undef KVC_GROUPS
#undef KVC_COMPUTE
#undef KVC_NV
#undef KVC_LOAD_WIN
}

// ---------------------------------------------------------------------------
// Pieces of the attention producer's row arithmetic (per-head RMSNorm +
// partial RoPE) used by qkv_append_kernel and by the producing decode step,
// which must give the same bits.  A row is held by a 32-lane half-wave, 8 dims
// per lane.
template <bool BF16IN>
__device__ __forceinline__ void load_row8(const void* base, size_t off, float (&x)[8]) {
    if constexpr (BF16IN) {
        const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            x[2 * j] = bf16lo(u[j]);
            x[2 * j + 1] = bf16hi(u[j]);
        }
    } else {
        const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + off);
        const u32x4 f0 = src[0];
        const u32x4 f1 = src[1];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            x[j] = __uint_as_float(f0[j]);
            x[4 + j] = __uint_as_float(f1[j]);
        }
    }
}

// RNE to bf16 with v_cvt_pk_bf16_f32 (a NaN input stays a NaN)
__device__ __forceinline__ u32x4 pack_bf16x8(const float (&y)[8]) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; j++) w[j] = cvt_pk_bf16(y[2 * j], y[2 * j + 1]);
    return w;
}
__device__ __forceinline__ void store_bf16x8(uint16_t* dst, const float (&y)[8]) {
    __builtin_nontemporal_store(pack_bf16x8(y), reinterpret_cast<u32x4*>(dst));
}

// yp = y of lane ^ M (M < 32: ds_swizzle, no address arithmetic)
template <int M>
__device__ __forceinline__ void swap_lanes8(const float (&y)[8], float (&yp)[8]) {
#pragma unroll
    for (int j = 0; j < 8; j++) yp[j] = shfl_xor<M>(y[j]);
}

// sum over the 32 lanes of each wave half
__device__ __forceinline__ float half_wave_sum(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    x += dpp<kDppRowRor8>(x);
    return sum_xor16(x);
}

// RoPE coefficients of the 8 dims d0 .. d0+7 of a lane at position pos:
// table entries p0 .. p0+7 for rope_dim >= 16, entries 0..3 twice for
// rope_dim 8; cos 1 / sin 0 outside the rotated dims or with no RoPE.  The
// loads (rope8_load) and the selection (rope8_select) are split so that a
// caller can issue the loads early and consume them later: every lane loads,
// on every path (lanes outside the rotated dims read valid entries of the same
// row; with no RoPE, half == 0, the loads read the first 16 B of `rope`, which
// must then still point at valid memory, and the selection ignores them), so
// nothing between the two waits on the loads and the number of loads in
// flight does not depend on the RoPE width.
struct Rope8 {
    float4 c0, c1, s0, s1;
};
__device__ __forceinline__ void rope8_load(const float* rope, int rope_rows, int half, int pos, int d0, Rope8& r) {
    const int p0 = half >= 8 ? (d0 & (half - 1)) : 0;
    const int o1 = half >= 8 ? 4 : 0;
    const float* crow = rope + (size_t)pos * half + p0;
    const float* srow = rope + ((size_t)rope_rows + pos) * half + p0;
    r.c0 = *reinterpret_cast<const float4*>(crow);
    r.c1 = *reinterpret_cast<const float4*>(crow + o1);
    r.s0 = *reinterpret_cast<const float4*>(srow);
    r.s1 = *reinterpret_cast<const float4*>(srow + o1);
}
__device__ __forceinline__ void rope8_select(const Rope8& r, int half, int d0, float (&cs)[8], float (&sn)[8]) {
    const bool roped = d0 < 2 * half;
    const float c[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
    const float sv[8] = {r.s0.x, r.s0.y, r.s0.z, r.s0.w, r.s1.x, r.s1.y, r.s1.z, r.s1.w};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        cs[j] = roped ? c[j] : 1.f;
        sn[j] = roped ? sv[j] : 0.f;
    }
}

// qkv_append_kernel's row arithmetic on NR rows at once (row r of each
// half-wave in x[r], 8 dims per lane at d0 = 8 x lane in the half), all with
// weights wn: per-head RMSNorm, then partial NeoX RoPE (partner of dim
// p < half is p + half: lane ^ (half / 8), or inside the lane for rope_dim
// 8), in the reference's order (src/engine.cpp:3497-3512): (x * r) * w, then
// x0 c - x1 s and x1 c + x0 s, without contraction.  The same operations in
// the same order as the producer kernel, so the same bits; the partner is
// fetched with ds_bpermute at a run-time address (one code path for every
// RoPE width, where the producer kernel has a ds_swizzle per width), for code
// that runs once per launch and should stay short.
template <int NR>
__device__ __forceinline__ void norm_rope_rows8(const float (&x)[NR][8], const float (&wn)[8], float eps,
                                                int half, int d0, const float (&cs)[8], const float (&sn)[8],
                                                float (&y)[NR][8]) {
#pragma clang fp contract(off)
    float ss[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        ss[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) ss[r] += x[r][j] * x[r][j];
    }
#pragma unroll
    for (int r = 0; r < NR; r++) ss[r] = half_wave_sum(ss[r]);
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const float rs = 1.0f / sqrtf(ss[r] / kHeadDim + eps);
#pragma unroll
        for (int j = 0; j < 8; j++) y[r][j] = x[r][j] * rs * wn[j];
    }
    const bool roped = d0 < 2 * half;
    if (half >= 8) {  // uniform
        const int src = (__lane_id() ^ (half >> 3)) << 2;
        float yp[NR][8];
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                yp[r][j] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(y[r][j])));
        if (roped) {
            const bool low = d0 < half;
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int j = 0; j < 8; j++)
                    y[r][j] = low ? y[r][j] * cs[j] - yp[r][j] * sn[j] : y[r][j] * cs[j] + yp[r][j] * sn[j];
        }
    } else if (half == 4 && roped) {  // rope_dim 8: pairs inside the lane's dims 0..7
#pragma unroll
        for (int r = 0; r < NR; r++) {
            float z[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                z[j] = y[r][j] * cs[j] - y[r][j + 4] * sn[j];
                z[j + 4] = y[r][j + 4] * cs[j + 4] + y[r][j] * sn[j + 4];
            }
#pragma unroll
            for (int j = 0; j < 8; j++) y[r][j] = z[j];
        }
    }
}

// The new key's 8-dim pieces c and c + 16 (c = lane % 16) and this lane's 4
// dims of the new value (bf16 rows knew / vnew of this kv head), as
// fold_token_v takes them.
template <int NP>
__device__ __forceinline__ void load_new_token(const uint16_t* knew, const uint16_t* vnew, int lane, int dpart,
                                               u32x4& k0, u32x4& k1, uint2& v) {
    const int c = lane & 15;
    k0 = *reinterpret_cast<const u32x4*>(knew + c * 8);
    k1 = *reinterpret_cast<const u32x4*>(knew + (c + 16) * 8);
    v = *reinterpret_cast<const uint2*>(vnew + dpart * (kHeadDim / NP) + (lane % (64 / NP)) * 4);
}

// Fold one extra key (the fused-append token) into a wave's finalized state
// (uniform m, l).  Each group of 16 lanes holds all 256 dims of q.  Every
// lane rescales its acc; only the lanes of token subset 0 add p * v (the
// subsets are summed afterwards).
template <int NP>
__device__ __forceinline__ void fold_token_v(WaveState& st, const uint32_t (&qv)[kGroup][2][4], const u32x4& k0,
                                             const u32x4& k1, uint2 v, float scale_log2, int lane) {
    float sc[kGroup];
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        float x = dot2_bf16(qv[g][0][0], k0[0], 0.f);
        x = dot2_bf16(qv[g][0][1], k0[1], x);
        x = dot2_bf16(qv[g][0][2], k0[2], x);
        x = dot2_bf16(qv[g][0][3], k0[3], x);
        x = dot2_bf16(qv[g][1][0], k1[0], x);
        x = dot2_bf16(qv[g][1][1], k1[1], x);
        x = dot2_bf16(qv[g][1][2], k1[2], x);
        x = dot2_bf16(qv[g][1][3], k1[3], x);
        x += dpp<kDppXor1>(x);
        x += dpp<kDppXor2>(x);
        x += dpp<kDppHalfMirror>(x);  // after xor 1, 2 every lane of a quad agrees
        x += dpp<kDppRowRor8>(x);
        sc[g] = readlane(x, 0) * scale_log2;
    }
    constexpr int kLanesD = 64 / NP;
    const float vs = lane < kLanesD ? 1.f : 0.f;
    const float vf[4] = {bf16lo(v.x) * vs, bf16hi(v.x) * vs, bf16lo(v.y) * vs, bf16hi(v.y) * vs};
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        const float mn = fmaxf(st.m[g], sc[g]);
        const float cg = fast_exp2(st.m[g] - mn);
        const float p = fast_exp2(sc[g] - mn);
        st.l[g] = fmaf(st.l[g], cg, p);
#pragma unroll
        for (int j = 0; j < 4; j++) st.acc[g][j] = fmaf(st.acc[g][j], cg, p * vf[j]);
        st.m[g] = mn;
    }
}

template <int NP>
__device__ __forceinline__ void fold_token(WaveState& st, const uint32_t (&qv)[kGroup][2][4],
                                           const uint16_t* knew, const uint16_t* vnew,
                                           float scale_log2, int lane, int dpart) {
    u32x4 k0, k1;
    uint2 v;
    load_new_token<NP>(knew, vnew, lane, dpart, k0, k1, v);
    fold_token_v<NP>(st, qv, k0, k1, v, scale_log2, lane);
}

// ---------------------------------------------------------------------------
// Split-K GQA decode.  Work item = (kv head, chunk of chunk_blocks blocks of
// one sequence, output-dim part); items of one (seq, head) are consecutive
// and are spread over the 8 XCDs in contiguous runs (workgroup b runs on XCD
// b % 8), so the NP parts of a chunk share an XCD and its L2.  Each item
// writes (m, l, acc) for its 4 q heads and its 256/NP dims; the last item of
// a (seq, head, part) to arrive (device-scope counter) combines them and
// writes the output.  NP = 2 is used when one part per chunk would leave CUs
// idle: it doubles the workgroups and halves what each combiner pulls, at
// the price of a second (L2-served) read of each chunk's K.
constexpr int kCombineBatch = 32;

// Phase stamps of the decode kernel, compiled in only for the
// KVC_PHASE_STAMPS build (libkvc_phases.so, read by bench.py --phases): lane 0
// of each wave writes s_memrealtime (100 MHz) at fixed points into
// phase_stamps[workgroup][wave][point].  A stamp adds a counter read and one
// 8-B vector store and skips no work.  Points: 0 entry, 1 block walk done,
// 2 wave merge done, 3 partial stores complete, 4 arrival atomic returned,
// 5 partials loaded (combiner), 6 folded (combiner), 7 output written (the
// wave that writes it: the combiner, or every wave of a one-chunk launch),
// 8 q rows built (producing decode step only, after their LDS read-back),
// 9 q row arithmetic begins (producing decode step only), 10 the wave merge's
// barrier passed (two-part launches).
#ifdef KVC_PHASE_STAMPS
constexpr int kStampWgs = 4096, kStampPoints = 11;
__device__ uint64_t phase_stamps[kStampWgs * kWaves * kStampPoints];
__device__ __forceinline__ void phase_stamp(int point) {
    uint64_t t;
    asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
    if ((threadIdx.x & 63) == 0 && blockIdx.x < kStampWgs)
        phase_stamps[(blockIdx.x * kWaves + (threadIdx.x >> 6)) * kStampPoints + point] = t;
}
#define KVC_STAMP(P) phase_stamp(P)
#define KVC_STAMP_WAIT_LOADS() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")
#else
#define KVC_STAMP(P) ((void)0)
#define KVC_STAMP_WAIT_LOADS() ((void)0)
#endif

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kDppXor1>(x));
    x = fmaxf(x, dpp<kDppXor2>(x));
    x = fmaxf(x, dpp<kDppHalfMirror>(x));  // quads already uniform: pairs quad 0 with quad 1
    x = fmaxf(x, dpp<kDppRowRor8>(x));
    x = max_xor16(x);
    return max_xor32(x);
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    x += dpp<kDppRowRor8>(x);
    x = sum_xor16(x);
    return sum_xor32(x);
}

// Fold partials [item0, item0 + nk) (nk <= NB) of q head g into (Mc, Lc, Ac).
// All NB acc loads (indices past nk clamped, weight 0) and the (m, l) load of
// lane k's partial are issued before any is consumed.
template <int NB>
__device__ __forceinline__ void combine_batch(__amdgpu_buffer_rsrc_t prs, int item0, int nk, int g, int d0,
                                              int lane, float& Mc, float& Lc, float (&Ac)[4]) {
    const int kl = min(lane, nk - 1);
    const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(
        prs, ((item0 + kl) * kItemFloats + kGroup * kHeadDim + 2 * g) * 4, 0, kCpolSC1);
    u32x4 pa[NB];
#pragma unroll
    for (int k = 0; k < NB; k++)
        pa[k] = __builtin_amdgcn_raw_buffer_load_b128(
            prs, ((item0 + min(k, nk - 1)) * kItemFloats + g * kHeadDim + d0) * 4, 0, kCpolSC1);
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first use
    const bool own = lane < nk;
    const float m_l = own ? __uint_as_float(ml[0]) : kNegBig;
    const float mb = fmaxf(Mc, wave_max(m_l));
    const float cc = fast_exp2(Mc - mb);
    Mc = mb;
    const float w_l = own ? fast_exp2(m_l - mb) : 0.f;
    Lc = fmaf(Lc, cc, wave_sum(w_l * __uint_as_float(ml[1])));
#pragma unroll
    for (int j = 0; j < 4; j++) Ac[j] *= cc;
#pragma unroll
    for (int k = 0; k < NB; k++) {
        const float w = readlane(w_l, k);
#pragma unroll
        for (int j = 0; j < 4; j++) Ac[j] = fmaf(w, __uint_as_float(pa[k][j]), Ac[j]);
    }
}

// PROD != 0: the decode step with the attention producer fused in (one query
// token per sequence, projection rows a.qkv in bf16 (PROD 1) or fp32 (PROD
// 2), converted as qkv_append_kernel converts them).  The rows are split over
// the waves, one row per 32-lane half: waves 0 and 1 build q rows 2w + sub of
// the group, and wave 2 of the workgroup that owns the new position builds its
// k row (sub 0) and stages its v row (sub 1, RNE bf16), all with the producer's row
// arithmetic (per-head RMSNorm + partial RoPE at position L - 1, RNE bf16;
// norm_rope_rows8 gives qkv_append_kernel's bits).  The raw rows, weights and
// RoPE coefficients are requested before the block walk; the arithmetic runs
// after the walk's first loads are issued (prep), the rows go to LDS
// (qstage), and after one workgroup barrier every wave reads q in load_q's
// layout.  The fused-append path then folds and appends k / v from LDS.  The
// gate is read straight from the projection row (fp32 gates rounded to bf16
// first, as the producer writes them).
template <int NP, int PROD>
__global__ __launch_bounds__(kWaves * 64) void decode_kernel(DecodeArgs a) {
    constexpr bool PRODUCE = PROD != 0;
    constexpr bool F32IN = PROD == 2;
    __shared__ DecodeSmem sm;
    KVC_STAMP(0);
    constexpr int kLanesD = 64 / NP;  // lanes per token subset
    const int b = blockIdx.x;
    const int item = (b & 7) * a.per_xcd + (b >> 3);
    if (item >= a.n_items) return;
    const int dpart = item % NP;
    const int hc = item / NP;
    const int h = hc / a.total_chunks;
    const int chunk = hc - h * a.total_chunks;
    int s = 0;
    while (s + 1 < a.n_seqs && a.chunk_begin[s + 1] <= chunk) s++;
    const int c = chunk - a.chunk_begin[s];
    const int n_chunks = a.chunk_begin[s + 1] - a.chunk_begin[s];
    const int L = a.kv_len[s];
    const int n_blocks = (L + kBlockTok - 1) / kBlockTok;
    const int blk0 = c * a.chunk_blocks;
    const int blk1 = min(blk0 + a.chunk_blocks, n_blocks);
    const int32_t* trow = a.table + (size_t)a.slot[s] * a.table_stride;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool fused_new = PRODUCE || a.k_new != nullptr;
    const int new_pos = fused_new ? L - 1 : -1;
    // PRODUCE: the built rows in LDS: q heads 0..3 of the group, then the new
    // token's k and v
    __shared__ __align__(16) uint16_t qstage[PRODUCE ? kGroup + 2 : 1][kHeadDim];
    const uint16_t* knew;
    const uint16_t* vnew;
    if constexpr (PRODUCE) {
        knew = qstage[kGroup];
        vnew = qstage[kGroup + 1];
    } else {
        knew = a.k_new ? a.k_new + ((size_t)s * kKvHeads + h) * kHeadDim : nullptr;
        vnew = a.v_new ? a.v_new + ((size_t)s * kKvHeads + h) * kHeadDim : nullptr;
    }

    // keys [0, Lw) come from the pool; with a fused append the last key
    // (position L-1) comes from knew/vnew and is folded in by wave 0 of the
    // chunk that owns it, whose part 0 also writes it into the pool
    const int Lw = fused_new ? L - 1 : L;
    const int wblk1 = min(blk1, (Lw + kBlockTok - 1) / kBlockTok);
    const int n_walk = max(0, wblk1 - blk0);
    // the ids of the chunk's first 64 blocks (the walk's and the new token's)
    // are requested before q: the wait for them (the load counter completes
    // in order) then does not also wait for q
    const int first_ids = lane < min(64, blk1 - blk0) ? trow[blk0 + lane] : 0;
    __builtin_amdgcn_sched_barrier(0);

    uint32_t qv[kGroup][2][4];
    // PRODUCE inputs, held from here to prep: lane hl = lane % 32 of half
    // sub = lane / 32 has dims pd0 .. pd0 + 7 of its row (raw bf16 in xr[0],
    // or fp32 in xr[0..1]), the row's norm weights and the RoPE coefficients
    // of position L - 1
    const int sub = lane >> 5, pd0 = (lane & 31) * 8;
    const bool q_wave = wave < 2;
    const bool make_new = PRODUCE && wave == 2 && new_pos >= blk0 * kBlockTok && new_pos < blk1 * kBlockTok;
    u32x4 xr[F32IN ? 2 : 1];
    float wr[8];
    Rope8 rp;
    if constexpr (PRODUCE) {
        // every wave loads (the waves that build no row read the group's
        // first q row), so the loads need no branch and the wait for the
        // first block ids covers exactly the loads issued before them
        {
            constexpr size_t kKOff = (size_t)kQHeads * 2 * kHeadDim;  // k rows, then v rows
            const int qr = q_wave ? 2 * wave + sub : 0;
            const size_t ro = (size_t)s * kQkvRow + pd0 +
                              (make_new ? kKOff + (size_t)(sub * kKvHeads + h) * kHeadDim
                                        : (size_t)(h * kGroup + qr) * 2 * kHeadDim);
            if constexpr (F32IN) {
                const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const float*>(a.qkv) + ro);
                xr[0] = src[0];
                xr[1] = src[1];
            } else {
                xr[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.qkv) + ro);
            }
            const float* wrow = (make_new ? a.k_norm : a.q_norm) + pd0;
            const float4 w0 = *reinterpret_cast<const float4*>(wrow);
            const float4 w1 = *reinterpret_cast<const float4*>(wrow + 4);
            wr[0] = w0.x; wr[1] = w0.y; wr[2] = w0.z; wr[3] = w0.w;
            wr[4] = w1.x; wr[5] = w1.y; wr[6] = w1.z; wr[7] = w1.w;
            rope8_load(a.rope_half ? a.rope : a.q_norm, a.rope_rows, a.rope_half, new_pos, pd0, rp);
        }
        // keep these loads here, ahead of the walk's (the compiler would
        // otherwise move them to their first use, behind the block loads)
        asm volatile("" ::: "memory");
    } else {
        load_q(qv, a.q + ((size_t)s * kQHeads + h * kGroup) * kHeadDim, lane);
    }
    auto prep = [&]() {
        if constexpr (PRODUCE) {
            KVC_STAMP(9);
            if (q_wave || make_new) {
                float cs[8], sn[8];
                rope8_select(rp, a.rope_half, pd0, cs, sn);
                float x[1][8], y[1][8];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if constexpr (F32IN) {
                        x[0][j] = __uint_as_float(xr[0][j]);
                        x[0][4 + j] = __uint_as_float(xr[1][j]);
                    } else {
                        x[0][2 * j] = bf16lo(xr[0][j]);
                        x[0][2 * j + 1] = bf16hi(xr[0][j]);
                    }
                }
                norm_rope_rows8<1>(x, wr, a.eps, a.rope_half, pd0, cs, sn, y);  // v half: unused
                const int row = q_wave ? 2 * wave + sub : kGroup + sub;
                // the v row: a copy of bf16 input, RNE of fp32 input
                const u32x4 vrow = F32IN ? pack_bf16x8(x[0]) : xr[0];
                *reinterpret_cast<u32x4*>(&qstage[row][pd0]) = make_new && sub ? vrow : pack_bf16x8(y[0]);
            }
            __syncthreads();
            load_q(qv, &qstage[0][0], lane);
#ifdef KVC_PHASE_STAMPS
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
            KVC_STAMP(8);
        }
    };
    WaveState st;
    init_state(st);
    walk_blocks<NP, PRODUCE>(a.kpool, a.vpool, trow, h, blk0, n_walk, Lw, qv, a.scale_log2, sm.p16[wave], st,
                             wave, lane, dpart, first_ids, prep);
    finalize_l(st);
    const bool owns_new = new_pos >= blk0 * kBlockTok && new_pos < blk1 * kBlockTok;
    if (owns_new) {
        // the new token's block id: from the chunk's ids (read before q) when
        // it is among the first 64
        const int nb = new_pos / kBlockTok - blk0;
        const int blk = nb < 64 ? __builtin_amdgcn_readlane(first_ids, nb) : trow[new_pos / kBlockTok];
        if (wave == 0) {
            fold_token<NP>(st, qv, knew, vnew, a.scale_log2, lane, dpart);
            if (dpart == 0)
                append_new_token(const_cast<uint16_t*>(a.kpool), const_cast<uint16_t*>(a.vpool), blk, h, new_pos,
                                 *reinterpret_cast<const u32x4*>(((lane >> 5) ? vnew : knew) + (lane & 31) * 8));
        }
    }
    KVC_STAMP(1);

    const int t = threadIdx.x, g = t >> 6;
    float M, Lsum, A[4];
    int d0;
    bool act = true;  // this thread holds output dims d0 .. d0 + 3
    if constexpr (NP == 1) {
        merge_waves(st, sm, wave, lane, M, Lsum, A);
        d0 = (t & 63) * 4;
    } else {
        // sum the token subsets of each dim (lanes l and l ^ 32), then merge
        // the 4 waves through LDS; lanes dl < 32 hold dims dpart*128 + dl*4
#pragma unroll
        for (int gg = 0; gg < kGroup; gg++)
#pragma unroll
            for (int j = 0; j < 4; j++) st.acc[gg][j] = sum_xor32(st.acc[gg][j]);
        static_assert(NP == 2, "d-split decode is built for 2 parts");
        const int dl = lane % kLanesD;
        act = lane < kLanesD;
        if (act) {
#pragma unroll
            for (int gg = 0; gg < kGroup; gg++)
                *reinterpret_cast<float4*>(&sm.acc[wave][gg][dl * 4]) =
                    make_float4(st.acc[gg][0], st.acc[gg][1], st.acc[gg][2], st.acc[gg][3]);
        }
        if (lane == 0) {
#pragma unroll
            for (int gg = 0; gg < kGroup; gg++) {
                sm.ml[wave][gg][0] = st.m[gg];
                sm.ml[wave][gg][1] = st.l[gg];
            }
        }
        __syncthreads();
        KVC_STAMP(10);
        M = kNegBig;
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, sm.ml[w][g][0]);
        Lsum = 0.f;
        A[0] = A[1] = A[2] = A[3] = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float wt = fast_exp2(sm.ml[w][g][0] - M);
            Lsum = fmaf(wt, sm.ml[w][g][1], Lsum);
            const float4 x = *reinterpret_cast<const float4*>(&sm.acc[w][g][dl * 4]);
            A[0] = fmaf(wt, x.x, A[0]);
            A[1] = fmaf(wt, x.y, A[1]);
            A[2] = fmaf(wt, x.z, A[2]);
            A[3] = fmaf(wt, x.w, A[3]);
        }
        d0 = dpart * (kHeadDim / NP) + dl * 4;
    }
    KVC_STAMP(2);
    const size_t orow = ((size_t)s * kQHeads + h * kGroup + g) * kHeadDim;
    const bool has_gate = PRODUCE || a.gate != nullptr;
    // gate of q head h * kGroup + g, dims d0 .. d0 + 3 as packed bf16: from
    // its own tensor, or from the projection row (fp32 rounded to nearest even)
    const size_t gro = (size_t)s * kQkvRow + (size_t)(h * kGroup + g) * 2 * kHeadDim + kHeadDim + d0;
    // the gate's raw words (fp32 input: 4 floats, rounded when used)
    u32x4 graw = {0u, 0u, 0u, 0u};
    auto load_gate = [&]() {
        if constexpr (F32IN) {
            graw = *reinterpret_cast<const u32x4*>(static_cast<const float*>(a.qkv) + gro);
        } else if constexpr (PRODUCE) {
            const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.qkv) + gro);
            graw[0] = w.x;
            graw[1] = w.y;
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(a.gate + orow + d0);
            graw[0] = w.x;
            graw[1] = w.y;
        }
    };
    // the gate words of this thread's dims as packed bf16
    auto gate_words = [&](const u32x4& r) -> uint2 {
        if constexpr (F32IN)
            return make_uint2(cvt_pk_bf16(__uint_as_float(r[0]), __uint_as_float(r[1])),
                              cvt_pk_bf16(__uint_as_float(r[2]), __uint_as_float(r[3])));
        else
            return make_uint2(r[0], r[1]);
    };
    if (n_chunks == 1) {
        if (has_gate && act) load_gate();
        float gs[4] = {1.f, 1.f, 1.f, 1.f};
        if (has_gate) gate_factors(gate_words(graw), a.gate_ref, gs);
        if (act) write_out(a.out, a.out_bf16, orow, d0, has_gate, gs, Lsum, A);
#ifdef KVC_PHASE_STAMPS
        __builtin_amdgcn_s_waitcnt(0);
        KVC_STAMP(7);
#endif
        return;
    }
    // Wave g publishes q head g's (m, l, acc) with agent-coherent stores;
    // once they have completed (its own s_waitcnt 0) it bumps head g's
    // arrival counter.  The last wave to arrive for (s, h, part, g) reads the
    // partials back with agent-coherent loads and writes head g's output.
    // Each wave arrives on its own: no workgroup barrier and no LDS
    // broadcast of the arrival lie on the path to the combine.
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.part, a.part_bytes);
    const int ibase = item * kItemFloats * 4;
    const int aoff = g * kHeadDim + (d0 - dpart * (kHeadDim / NP));  // acc slot of this thread's dims
    if (act) {
        u32x4 av;
        av[0] = __float_as_uint(A[0]);
        av[1] = __float_as_uint(A[1]);
        av[2] = __float_as_uint(A[2]);
        av[3] = __float_as_uint(A[3]);
        __builtin_amdgcn_raw_buffer_store_b128(av, prs, ibase + aoff * 4, 0, kCpolSC1);
    }
    if (lane == 0) {
        u32x2 mlv;
        mlv[0] = __float_as_uint(M);
        mlv[1] = __float_as_uint(Lsum);
        __builtin_amdgcn_raw_buffer_store_b64(mlv, prs, ibase + (kGroup * kHeadDim + 2 * g) * 4, 0, kCpolSC1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    KVC_STAMP(3);
    // one 128-B line per counter: arrivals on different counters do not
    // contend for one line
    int32_t* ctr = a.counters + (((s * kKvHeads + h) * kMaxDParts + dpart) * kGroup + g) * kCounterStride;
    int prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the gate words ride along with the arrival: requested after it, they
    // arrive while it completes, so a combiner does not wait on them after
    // its fold and no wave waits on them before its arrival
    asm volatile("" ::: "memory");
    if (has_gate && act) load_gate();
    const bool last = __builtin_amdgcn_readfirstlane(prev) == n_chunks - 1;
    KVC_STAMP(4);
    if (!last) return;
    float Mc = kNegBig, Lc = 0.f, Ac[4] = {0.f, 0.f, 0.f, 0.f};
    float gs[4] = {1.f, 1.f, 1.f, 1.f};  // gate factors (the split-D combine: under its first loads)
    if constexpr (NP == 1) {
        // combine the n_chunks partials of (s, h): wave g takes q head g; every
        // partial of a batch is requested at once (lane k also fetches partial
        // k's (m, l)), then the acc rows are folded in arrival order
        const int first = h * a.total_chunks + a.chunk_begin[s];
        for (int k0 = 0; k0 < n_chunks; k0 += kCombineBatch) {
            const int nk = min(kCombineBatch, n_chunks - k0);
            if (nk <= 8)
                combine_batch<8>(prs, first + k0, nk, g, d0, lane, Mc, Lc, Ac);
            else if (nk <= 16)
                combine_batch<16>(prs, first + k0, nk, g, d0, lane, Mc, Lc, Ac);
            else
                combine_batch<32>(prs, first + k0, nk, g, d0, lane, Mc, Lc, Ac);
        }
    } else {
        // wave g takes q head g; lane = psub * 32 + dl folds chunks k0 + 2k +
        // psub of dims dl*4 .. +3 of this part; lane j also fetches chunk
        // k0 + j's (m, l), so the batch max and the weights come from wave
        // reductions and only the acc rows are summed over the two lane halves
        const int psub = lane / kLanesD, dl = lane % kLanesD;
        const int first = (h * a.total_chunks + a.chunk_begin[s]) * NP + dpart;
        constexpr int kNB = kCombineBatch / NP;
        for (int k0 = 0; k0 < n_chunks; k0 += kCombineBatch) {
            const int nk = min(kCombineBatch, n_chunks - k0);
            const int kl = min(lane, nk - 1);
            const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(
                prs, ((first + (k0 + kl) * NP) * kItemFloats + kGroup * kHeadDim + 2 * g) * 4, 0, kCpolSC1);
            u32x4 pa[kNB];
#pragma unroll
            for (int k = 0; k < kNB; k++) {
                const int cc = min(k0 + k * NP + psub, n_chunks - 1);
                pa[k] = __builtin_amdgcn_raw_buffer_load_b128(
                    prs, ((first + cc * NP) * kItemFloats + g * kHeadDim + dl * 4) * 4, 0, kCpolSC1);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first use
            if (k0 == 0) {
                // the gate words were requested before these loads: their
                // sigmoids run while the partials are in flight (the empty
                // asm pins them below the loads)
                if (has_gate) {
                    u32x4 g2 = graw;
                    asm volatile("" : "+v"(g2));
                    gate_factors(gate_words(g2), a.gate_ref, gs);
                }
                __builtin_amdgcn_sched_barrier(0);
                KVC_STAMP_WAIT_LOADS();
                KVC_STAMP(5);
            }
            const bool own = lane < nk;
            const float m_l = own ? __uint_as_float(ml[0]) : kNegBig;
            const float mb = fmaxf(Mc, wave_max(m_l));
            const float cs = fast_exp2(Mc - mb);
            Mc = mb;
            const float w_l = own ? fast_exp2(m_l - mb) : 0.f;  // 0 for chunks past nk
            Lc = fmaf(Lc, cs, wave_sum(w_l * __uint_as_float(ml[1])));
#pragma unroll
            for (int j = 0; j < 4; j++) Ac[j] *= cs;
            // each lane fetches the weights of its own partials (chunk
            // k NP + psub lives in lane k NP + psub) with ds_bpermute: no
            // per-partial readlane or select (a readlane under a
            // lane-dependent condition compiles to a divergent branch per
            // partial, measured 0.7 us per launch at config b)
            float wk[kNB];
#pragma unroll
            for (int k = 0; k < kNB; k++)
                wk[k] = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (k * NP + psub), __float_as_int(w_l)));
#pragma unroll
            for (int k = 0; k < kNB; k++)
#pragma unroll
                for (int j = 0; j < 4; j++) Ac[j] = fmaf(wk[k], __uint_as_float(pa[k][j]), Ac[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) Ac[j] = sum_xor32(Ac[j]);
    }
    if constexpr (NP == 1) {
        if (has_gate) gate_factors(gate_words(graw), a.gate_ref, gs);
    }
    KVC_STAMP(6);
    if (act) write_out(a.out, a.out_bf16, orow, d0, has_gate, gs, Lc, Ac);
    if (lane == 0) *ctr = 0;
#ifdef KVC_PHASE_STAMPS
    __builtin_amdgcn_s_waitcnt(0);
    KVC_STAMP(7);
#endif
}

// ---------------------------------------------------------------------------
// Causal chunked prefill with bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Workgroup = (sequence, kv head, 32 consecutive query positions); each wave
// handles one q head of the GQA group and 16 * NT of the 32 rows, so each
// 64-key K/V tile staged in LDS serves 4 q heads.  Per tile and wave:
//   S^T[64 keys x 16 NT rows]  = K[keys x 256] . Q^T       (A = K rows, LDS)
//   P^T = 2^(S^T - m)          (online softmax, log2 domain, bf16)
//   O^T[256 d x 16 NT rows]   += V^T[d x keys] . P^T       (A = V^T, LDS)
// Working on transposes keeps each lane on one query row (row = lane % 16)
// in both products, so the row statistics need no lane shuffles and P^T
// leaves the S^T accumulator already in B-operand order.  Keys inside one
// 32-key MFMA step are taken in the order (4q + i, 16 + 4q + i) for lane group
// q = lane / 16, i = 0..3, on both operands (a consistent permutation of the
// summation index).  K and V tiles go straight from global memory into LDS
// (global_load_lds_dwordx4, no register staging), double buffered: tile t+1
// is in flight while tile t is computed, one barrier per tile.  Tile rows are
// 512 B with their 16-B chunks XOR-swizzled by the row, with one pattern for
// K and another for V (kswz, vswz), so that both operand reads are free of
// bank conflicts.  The V^T operand is read with ds_read_b64_tr_b16, which hands
// lane i of each 16-lane group element i%4 of the 8-B pieces addressed by
// lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4 -- a 4 x 16 transpose.  Rows past the
// sequence end are loaded from the last valid key (finite data; their weight
// is 0).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
constexpr int kPfRows = 32;                 // query positions per workgroup
constexpr int kPfKeys = 64;                 // keys per tile
constexpr int kTileElems = kPfKeys * kHeadDim;
#ifndef KVC_PF_AHEAD
#define KVC_PF_AHEAD 4
#endif
constexpr int kPfAhead = KVC_PF_AHEAD;      // operand fragments read ahead of their MFMAs
constexpr int kSgMfma = 0x008;              // sched_group_barrier masks: MFMA,
constexpr int kSgDsRead = 0x100;            //   LDS read
#ifndef KVC_PF_NT
#define KVC_PF_NT 1
#endif
constexpr int kPfNT = KVC_PF_NT;            // 16-row query tiles per prefill wave (1 or 2)

struct PrefillSmem {  // [buffer][row * 256 + swizzled column]; V first, so V^T reads reach
    uint16_t v[2][kTileElems];   // both buffers with 16-bit immediate offsets from one base
    uint16_t k[2][kTileElems];
};

// Tile swizzles: 16-B chunk c of row r sits at position c ^ kswz(r) (K) or
// c ^ vswz(r) (V).  A K fragment read
// takes one chunk of 16 rows r16 = 0..15: their positions differ in the low 4
// bits.  A V^T read (ds_read_b64_tr_b16) takes, per 16-lane group, one chunk
// pair of 4 rows 4i .. 4i+3: vswz puts the 4 rows on 4 different pairs.
__device__ __forceinline__ int kswz(int r) { return r & 15; }
__device__ __forceinline__ int vswz(int r) { return (r & 15) << 1; }

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 B per lane from global memory straight into LDS (global_load_lds_dwordx4,
// scalar-base form): lane i copies gbase + voff[i] (gbase uniform, in SGPRs)
// into LDS bytes [lds_off + 16i, +16).  Issued from inline asm so the
// compiler does not treat the in-flight copy as a pending write to every LDS
// object (it would otherwise wait for it before the current tile's reads);
// callers order it with an explicit s_waitcnt vmcnt(0) and barrier.  M0 is
// set here and used by nothing else in the prefill kernel.
__device__ __forceinline__ void lds_dma16s(const void* gbase, uint32_t voff, uint32_t lds_off) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_off), "v"(voff),
                 "s"(gbase)
                 : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_ptr_t)(p);
}
// LDS reads at byte address base + off; off is a compile-time constant that
// folds into the instruction's offset field.
__device__ __forceinline__ u32x4 lds_load16(uint32_t base, uint32_t off) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)(base + off));
}
__device__ __forceinline__ u32x2 lds_load_tr16(uint32_t base, uint32_t off) {
    const i16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (i16x4_t __attribute__((address_space(3)))*)((uintptr_t)(base + off)));
    return __builtin_bit_cast(u32x2, r);
}


// a compile-time integer as a value (tile buffer index, register distance)
template <int B>
struct PfBuf {
    static constexpr int value = B;
};

// One q row of the prefill step in the prefill's B-operand layout: lane (q4,
// r16) holds dims 32 ks + 8 q4 .. +7 (ks = 0..7) of its row, so a row's 256
// dims sit on lanes r16, r16 + 16, r16 + 32, r16 + 48.  The arithmetic is
// qkv_append_kernel's (per-head RMSNorm, partial NeoX RoPE at position pos,
// RNE bf16; src/engine.cpp:2861-2883), with its bits: the sum of squares
// takes the producer's tree (each 8-dim group g = d / 8 summed in order, then
// the groups paired by bit 0 of g, bit 1, ..., bit 4, as its half-wave sum
// pairs lanes ^ 1, ^ 2, the half-row mirror, the row rotate by 8 and ^ 16);
// here bits 0 and 1 of g are lane bits 4 and 5 and bits 2..4 are ks.  The
// RoPE partner of dim d < half is d + half: register ks ^ (half / 32) for
// half >= 32, lane ^ 16 / ^ 32 for half 8 / 16, the lane's own dims for half
// 4.  qb receives the bf16 words XOR qflip (the sign of a negative scale).
template <bool F32IN>
__device__ __forceinline__ void prefill_q_row(const void* qkv, size_t row, const float* q_norm,
                                              const float* rope, int rope_rows, int half, int pos, float eps,
                                              int q4, uint32_t qflip, bf16x8_t (&qb)[8]) {
#pragma clang fp contract(off)
    float x[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const size_t e = row + 32 * ks + 8 * q4;
        if constexpr (F32IN) {
            const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const float*>(qkv) + e);
            const u32x4 f0 = src[0], f1 = src[1];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                x[ks][j] = __uint_as_float(f0[j]);
                x[ks][4 + j] = __uint_as_float(f1[j]);
            }
        } else {
            const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(qkv) + e);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                x[ks][2 * j] = bf16lo(u[j]);
                x[ks][2 * j + 1] = bf16hi(u[j]);
            }
        }
    }
    float gs[8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        gs[ks] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) gs[ks] += x[ks][j] * x[ks][j];
    }
#pragma unroll
    for (int ks = 0; ks < 8; ks++) gs[ks] += shfl_xor<16>(gs[ks]);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) gs[ks] += shfl_xor<32>(gs[ks]);
    const float ss = ((gs[0] + gs[1]) + (gs[2] + gs[3])) + ((gs[4] + gs[5]) + (gs[6] + gs[7]));
    const float rs = 1.0f / sqrtf(ss / kHeadDim + eps);
    float y[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const float4 w0 = *reinterpret_cast<const float4*>(q_norm + 32 * ks + 8 * q4);
        const float4 w1 = *reinterpret_cast<const float4*>(q_norm + 32 * ks + 8 * q4 + 4);
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) y[ks][j] = x[ks][j] * rs * w[j];
    }
    // RoPE coefficients of dims d0 .. d0 + 7 (d0 = 32 ks + 8 q4 < 2 half):
    // entries p0 .. p0 + 7 of the position's row (entries 0..3 twice for half 4)
    auto coef = [&](int d0, float (&c)[8], float (&sn)[8]) {
        const int p0 = half >= 8 ? (d0 & (half - 1)) : 0;
        const int o1 = half >= 8 ? 4 : 0;
        const float* crow = rope + (size_t)pos * half + p0;
        const float* srow = rope + ((size_t)rope_rows + pos) * half + p0;
        const float4 c0 = *reinterpret_cast<const float4*>(crow);
        const float4 c1 = *reinterpret_cast<const float4*>(crow + o1);
        const float4 s0 = *reinterpret_cast<const float4*>(srow);
        const float4 s1 = *reinterpret_cast<const float4*>(srow + o1);
        c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w; c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
        sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    };
    // half >= 32: registers ks < 2 PM rotate, partner register ks ^ PM
    auto rotate_regs = [&](auto pmc) {
        constexpr int PM = decltype(pmc)::value;
        float z[2 * PM][8];
#pragma unroll
        for (int ks = 0; ks < 2 * PM; ks++) {
            float c[8], sn[8];
            coef(32 * ks + 8 * q4, c, sn);
#pragma unroll
            for (int j = 0; j < 8; j++)
                z[ks][j] = ks < PM ? y[ks][j] * c[j] - y[ks ^ PM][j] * sn[j] : y[ks][j] * c[j] + y[ks ^ PM][j] * sn[j];
        }
#pragma unroll
        for (int ks = 0; ks < 2 * PM; ks++)
#pragma unroll
            for (int j = 0; j < 8; j++) y[ks][j] = z[ks][j];
    };
    if (half == 32) {  // uniform
        rotate_regs(PfBuf<1>{});
    } else if (half == 64) {
        rotate_regs(PfBuf<2>{});
    } else if (half == 128) {
        rotate_regs(PfBuf<4>{});
    } else if (half >= 8) {  // 8 or 16: register 0 only, partner lane ^ 16 (half 8) or ^ 32 (half 16)
        float yp[8];
#pragma unroll
        for (int j = 0; j < 8; j++) yp[j] = half == 8 ? shfl_xor<16>(y[0][j]) : shfl_xor<32>(y[0][j]);
        const int d0 = 8 * q4;
        if (d0 < 2 * half) {
            float c[8], sn[8];
            coef(d0, c, sn);
            const bool low = d0 < half;
#pragma unroll
            for (int j = 0; j < 8; j++) y[0][j] = low ? y[0][j] * c[j] - yp[j] * sn[j] : y[0][j] * c[j] + yp[j] * sn[j];
        }
    } else if (half == 4 && q4 == 0) {  // rope_dim 8: pairs (j, j + 4) inside the lane's dims 0..7
        float c[8], sn[8];
        coef(0, c, sn);
        float z[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            z[j] = y[0][j] * c[j] - y[0][j + 4] * sn[j];
            z[j + 4] = y[0][j + 4] * c[j + 4] + y[0][j] * sn[j + 4];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) y[0][j] = z[j];
    }
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = cvt_pk_bf16(y[ks][2 * i], y[ks][2 * i + 1]) ^ qflip;
        qb[ks] = as_bf16x8(w);
    }
}

// NT = 16-row query tiles per wave: NT = 2 runs 4 waves (one per q head of
// the group, 32 rows each); NT = 1 runs 8 waves (q head, row half), two per
// SIMD, so one wave's MFMAs overlap the other's LDS reads and softmax.
//
// The per-tile VALU work is kept small:
//  - tiles are fetched with the scalar-base form of the LDS DMA, with
//    per-lane offsets fixed at kernel start (a tile that runs past the last
//    key clamps its rows per lane);
//  - the loop is unrolled over the two buffers, so every operand-fragment
//    address is a per-lane base plus an immediate;
//  - scores stay unscaled on full tiles: the tile max is scaled once and the
//    scale enters the exponent through an FMA (a negative scale is moved into
//    Q, whose sign flip is exact, so the scale used is |scale| >= 0); only
//    tiles that reach the diagonal or the sequence end are masked;
//  - the softmax denominator comes from two more MFMAs per tile, with an
//    all-ones A operand against the same bf16 P^T (so it sums exactly the
//    weights that P.V uses).

// PROD != 0: the prefill step, q and gate taken from the projection rows a.qkv
// (bf16: PROD 1, fp32: PROD 2): each wave builds its q rows in the B-operand
// layout with the producer's arithmetic (prefill_q_row) and reads the gate
// from the rows in the epilogue (fp32 rounded to bf16 first, as the producer
// writes it), so the result has the bits of kvc_qkv_append + the plain
// kernel.
template <int NT, int PROD>
__global__ __launch_bounds__(64 * 8 / NT) __attribute__((amdgpu_waves_per_eu(2 / NT, 2 / NT)))
void prefill_mfma_kernel(PrefillArgs a) {
    constexpr bool PRODUCE = PROD != 0;
    constexpr bool F32IN = PROD == 2;
    constexpr int kWavesPf = 8 / NT;
    constexpr int kRowsPerWave = 16 * NT;
    constexpr int kLoadRows = kPfKeys / kWavesPf;  // tile rows each wave loads
    __shared__ PrefillSmem sm;
    // Workgroup b runs on XCD b % 8.  The n_pb query blocks of one (sequence,
    // kv head) group share its K/V, so they go to one XCD (one L2), in
    // consecutive dispatch rounds; groups are taken most keys first (the
    // sequence order is sorted on the host) and, inside a group, the later
    // (longer) query blocks first.
    const int n_pb = (a.n_q + kPfRows - 1) / kPfRows;
    const int xcd = blockIdx.x & 7, round = blockIdx.x >> 3;
    const int grp = (round / n_pb) * 8 + xcd;
    if (grp >= a.n_groups) return;
    const int pb = n_pb - 1 - round % n_pb;
    const int h = grp % kKvHeads;
    const int s = a.seq_order[grp / kKvHeads];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (LDS DMA base)
    const int q4 = lane >> 4, r16 = lane & 15;
    const int g = wave & 3;            // q head of the group
    const int rw0 = (wave >> 2) * kRowsPerWave;  // first row of the wave within the tile
    const int pos0 = a.q_pos0[s];
    const int row0 = pb * kPfRows;                     // first query row of the tile
    const int rows = min(kPfRows, a.n_q - row0);
    const int kmax = pos0 + row0 + rows;               // keys [0, kmax) are visible
    const int n_tiles = (kmax + kPfKeys - 1) / kPfKeys;
    const int n_blocks = (kmax + kBlockTok - 1) / kBlockTok;
    const int32_t* trow = a.table + (size_t)a.slot[s] * a.table_stride;
    constexpr size_t kUnitElems = (size_t)kBlockTok * kHeadDim;
    const float c = fabsf(a.scale_log2);
    const uint32_t qflip = a.scale_log2 < 0.f ? 0x80008000u : 0u;

    // block ids of a 64-block window sit in one VGPR (lane i = block w0 + i)
    // and are read with v_readlane: no dependent table load on the fetch
    // path.  The first window's are requested before Q, so the wait for them
    // (the load counter completes in order) does not also wait for Q.
    int idw0 = 0;
    int idv = lane < n_blocks ? trow[lane] : 0;
    __builtin_amdgcn_sched_barrier(0);

    // Q^T as the B operand: qb[nt][ks] = q[row rw0 + 16nt + r16][d 32ks + 8q4 .. +7]
    bf16x8_t qb[NT][8];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int r = row0 + min(rw0 + 16 * nt + r16, rows - 1);
        if constexpr (PRODUCE) {
            const size_t row = ((size_t)s * a.n_q + r) * kQkvRow + (size_t)(h * kGroup + g) * 2 * kHeadDim;
            prefill_q_row<F32IN>(a.qkv, row, a.q_norm, a.rope, a.rope_rows, a.rope_half, pos0 + r, a.eps, q4, qflip,
                                 qb[nt]);
        } else {
            const uint16_t* qr = a.q + (((size_t)s * a.n_q + r) * kQHeads + h * kGroup + g) * kHeadDim;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                u32x4 x = *reinterpret_cast<const u32x4*>(qr + 32 * ks + 8 * q4);
                x[0] ^= qflip;
                x[1] ^= qflip;
                x[2] ^= qflip;
                x[3] ^= qflip;
                qb[nt][ks] = as_bf16x8(x);
            }
        }
    }

    // wave w loads tile rows kLoadRows*w .., two per instruction (lanes 0-31:
    // row r0, lanes 32-63: the next row); lane l fills chunk position l % 32
    // of its row, i.e. global chunk (l % 32) ^ swz(row).  A wave's rows lie in
    // one of the tile's two blocks (half = 0 or 1).
    const int half = (kLoadRows * wave) / kBlockTok;
    // Byte offset inside a (block, head) unit of the 16 B lane l fills for
    // instruction j: row part ((r0 & 31) + l / 32) * 512, chunk part
    // ((l % 32) ^ swz(r)) * 16.  Since r % 16 = s0 | 2j with s0 = (r0(0) % 16)
    // | l / 32 (disjoint bits), the chunk part is cb ^ (j * 32) for K (swz =
    // r % 16) and cb ^ (j * 64) for V (swz = 2 (r % 16)).
    static_assert(kLoadRows == 8 || kLoadRows == 16, "s0 and 2j occupy disjoint bits");
    const int s0 = ((kLoadRows * wave) & 15) | (lane >> 5);
    const uint32_t cbk = (((lane & 31) ^ s0) << 4) + (lane >> 5) * 512;
    const uint32_t cbv = (((lane & 31) ^ (s0 << 1)) << 4) + (lane >> 5) * 512;
    // Rows past the last key are loaded from the last key (finite data,
    // weight 0).  The clamped rows of a wave still lie in one block: a wave
    // of the second half reads block 2t + 1 if the last key is in it, else
    // the last key of block 2t.
    auto issue_rows = [&](const uint16_t* pool, uint32_t cb, int jsh, uint32_t lds_tile, int t) {
        const int last = kmax - 1 - t * kPfKeys;  // last key row of the tile
        const int id = __builtin_amdgcn_readlane(idv, 2 * t + (half && last >= kBlockTok ? 1 : 0) - idw0);
        const uint16_t* base = pool + ((size_t)id * kKvHeads + h) * kUnitElems;
        const bool full = last >= kPfKeys - 1;  // uniform
#pragma unroll
        for (int j = 0; j < kLoadRows / 2; j++) {
            const int r0 = kLoadRows * wave + 2 * j;
            uint32_t off = (cb ^ (j << jsh)) + (r0 & (kBlockTok - 1)) * 512;
            if (!full) off = (min(r0 + (lane >> 5), last) & (kBlockTok - 1)) * 512 | (off & 511);
            lds_dma16s(base, off, lds_tile + r0 * kHeadDim * 2);
        }
    };
    auto issue_k = [&](int t, int buf) { issue_rows(a.kpool, cbk, 5, lds_addr(&sm.k[buf][0]), t); };
    auto issue_v = [&](int t, int buf) { issue_rows(a.vpool, cbv, 6, lds_addr(&sm.v[buf][0]), t); };

    // With NT = 2 the accumulators outgrow the VGPRs: an (empty) statement
    // with an AGPR operand makes the compiler select the AGPR-accumulator form
    // of the MFMAs, so O^T lives in AGPRs.
    if constexpr (NT == 2) asm volatile("" ::"a"(0));
    f32x4 o[16][NT], ol[NT];  // ol: the all-ones row block (softmax denominator)
    float m_run[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int dt = 0; dt < 16; dt++) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        ol[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run[nt] = kNegBig;
    }
    const bf16x8_t ones = as_bf16x8(u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

    // Per-lane LDS byte addresses of the operand fragments in buffer 0 (the
    // XOR swizzles make them lane dependent); the fragment and buffer parts
    // are immediates:
    //   K (kt, ks = 4hi + j): kaddr[j] + 256 hi + 8192 kt + 32768 buf
    //   V^T (dt, kk, lo/hi):  vaddr[dt] + 16384 kk + 8192 (hi) + 32768 buf
    uint32_t kaddr[4], vaddr[16];
    const uint32_t k0 = lds_addr(&sm.k[0][0]), v0 = lds_addr(&sm.v[0][0]);
#pragma unroll
    for (int j = 0; j < 4; j++) kaddr[j] = k0 + r16 * 512 + 16 * ((4 * j + q4) ^ r16);
    {
        const int w = 4 * q4 + (r16 >> 2);  // V row % 16 of this lane
#pragma unroll
        for (int dt = 0; dt < 16; dt++)
            vaddr[dt] = v0 + w * 512 + 16 * (2 * (dt ^ w) + ((r16 & 3) >> 1)) + 8 * (r16 & 1);
    }

    // S^T tiles: s[kt][nt], lane holds keys 16kt + 4q4 + i of row 16nt + r16.
    // Steps i = (ks, kt) run d-slice outer, key subtile inner, so consecutive
    // MFMAs feed different accumulators; the 32 K fragments are read kPfAhead
    // steps ahead of their MFMAs through a register ring.
    auto compute_s = [&](auto bufc, f32x4 (&s)[4][NT]) {
        constexpr uint32_t kOff = decltype(bufc)::value * (uint32_t)sizeof(sm.k[0]);
        bf16x8_t kf[kPfAhead];
        auto read_kfrag = [&](int i) {
            const int ks = i >> 2, kt = i & 3;
            kf[i % kPfAhead] = as_bf16x8(lds_load16(kaddr[ks & 3], kOff + 256 * (ks >> 2) + 8192 * kt));
        };
#pragma unroll
        for (int i = 0; i < kPfAhead; i++) read_kfrag(i);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int ks = i >> 2, kt = i & 3;
            const bf16x8_t ka = kf[i % kPfAhead];
            if (i + kPfAhead < 32) read_kfrag(i + kPfAhead);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                s[kt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[nt][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[kt][nt], 0, 0, 0);
        }
    };

    // Per 64-key tile t (K(t) and V(t) in buffers t & 1): after the barrier
    // tile t is resident and every wave is done with buffer (t + 1) & 1, which
    // then receives tile t + 1 while tile t is computed.
    auto step = [&](auto bufc, int t) {
        constexpr int B = decltype(bufc)::value;
        constexpr uint32_t kVOff = B * (uint32_t)sizeof(sm.v[0]);
        // re-define the fragment bases here (empty asm) so base + buffer
        // offset is not hoisted out of the loop into extra registers: the
        // offset then folds into each read's immediate
#pragma unroll
        for (int j = 0; j < 4; j++) asm volatile("" : "+v"(kaddr[j]));
#pragma unroll
        for (int dt = 0; dt < 16; dt++) asm volatile("" : "+v"(vaddr[dt]));
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (t + 1 < n_tiles) {
            if (2 * (t + 1) + 1 - idw0 >= 64 && 2 * (t + 1) < n_blocks) {  // uniform: next id window
                idw0 = 2 * (t + 1);
                idv = idw0 + lane < n_blocks ? trow[idw0 + lane] : 0;
            }
            issue_k(t + 1, B ^ 1);
            issue_v(t + 1, B ^ 1);
        }
        f32x4 st[4][NT];
        // the MFMA runs (S here, P.V below) issue at raised wave priority, so
        // on a SIMD the wave feeding the matrix pipe goes ahead of the other
        // wave's softmax VALU work
        __builtin_amdgcn_s_setprio(1);
        compute_s(PfBuf<B>{}, st);
        // pin the pipeline: kPfAhead reads, then (1 read, NT MFMAs) per step
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, kPfAhead, 0);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            if (i + kPfAhead < 32) __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSgMfma, NT, 0);
        }
        __builtin_amdgcn_s_setprio(0);

        // Tile max in the log2 domain.  A full tile (all keys exist and
        // precede the wave's first row) keeps raw scores: the max is scaled
        // once (c >= 0 keeps the order).  A tile that reaches the diagonal or
        // the sequence end is scaled and masked in a branch of its own (the
        // empty asm keeps the compiler from turning it into selects on every
        // tile), and its exponent scale is then 1.
        const bool full = t * kPfKeys + kPfKeys - 1 <= pos0 + row0 + rw0 && t * kPfKeys + kPfKeys <= kmax;
        if (!full) {
            asm volatile("");
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int qpos = pos0 + row0 + rw0 + 16 * nt + r16;
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int kp = t * kPfKeys + 16 * kt + 4 * q4 + i;
                        st[kt][nt][i] = (kp <= qpos && kp < kmax) ? st[kt][nt][i] * c : kNegBig;
                    }
            }
        }
        const float cs = full ? c : 1.f;
        bool need = false;
        float mt[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float mx = kNegBig;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) mx = fmaxf(mx, st[kt][nt][i]);
            mx = max_xor16(mx);
            mx = max_xor32(mx);
            mt[nt] = full ? mx * c : mx;
            need |= mt[nt] > m_run[nt] + kRescaleSlack;
        }
        if (__builtin_amdgcn_ballot_w64(need) != 0) {  // uniform; rows that keep their max scale by 1
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const bool up = mt[nt] > m_run[nt] + kRescaleSlack;
                const float cr = up ? fast_exp2(m_run[nt] - mt[nt]) : 1.f;
                m_run[nt] = up ? mt[nt] : m_run[nt];
                // the scaled values re-enter the accumulators through an MFMA
                // with zero operands, which keeps them in the MFMA register class
                const bf16x8_t z8 = {};
#pragma unroll
                for (int dt = 0; dt < 16; dt++)
                    o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(z8, z8, o[dt][nt] * cr, 0, 0, 0);
                ol[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(z8, z8, ol[nt] * cr, 0, 0, 0);
            }
        }
        // P^T as the B operand (bf16), k-slot order (4q4 + i, 16 + 4q4 + i);
        // p = 2^(s * cs - m) with one rounding before the exponential
        bf16x8_t pb_[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const float nm = -m_run[nt];
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                u32x4 w;
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const f32x4 sv = st[2 * kk + hf][nt];
                    w[2 * hf] = cvt_pk_bf16(fast_exp2(fmaf(sv[0], cs, nm)), fast_exp2(fmaf(sv[1], cs, nm)));
                    w[2 * hf + 1] = cvt_pk_bf16(fast_exp2(fmaf(sv[2], cs, nm)), fast_exp2(fmaf(sv[3], cs, nm)));
                }
                pb_[nt][kk] = as_bf16x8(w);
            }
        }

        // O^T += V^T . P^T; the V^T operand of lane (q4, r16) is V[keys
        // 32kk + 4q4 + e (+16)][16dt + r16]: lane J of the group addresses
        // row 32kk + 4q4 + J/4 (+16), dims 16dt + 4(J%4) .. +3
        // V^T fragments (dt, kk), read kPfAhead steps ahead of their MFMAs
        bf16x8_t vf[kPfAhead];
        auto read_vfrag = [&](int i) {  // step i = (kk, dt): consecutive MFMAs feed different o[dt]
            const int kk = i >> 4, dt = i & 15;
            const u32x2 lo = lds_load_tr16(vaddr[dt], kVOff + 16384 * kk);
            const u32x2 hi = lds_load_tr16(vaddr[dt], kVOff + 16384 * kk + 8192);
            u32x4 w;
            w[0] = lo[0];
            w[1] = lo[1];
            w[2] = hi[0];
            w[3] = hi[1];
            vf[i % kPfAhead] = as_bf16x8(w);
        };
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < kPfAhead; i++) read_vfrag(i);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int kk = i >> 4, dt = i & 15;
            const bf16x8_t va = vf[i % kPfAhead];
            if (i + kPfAhead < 32) read_vfrag(i + kPfAhead);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb_[nt][kk], o[dt][nt], 0, 0, 0);
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int kk = 0; kk < 2; kk++)
                ol[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb_[nt][kk], ol[nt], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2 * kPfAhead, 1);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            if (i + kPfAhead < 32) __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 1);
            __builtin_amdgcn_sched_group_barrier(kSgMfma, NT, 1);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    issue_k(0, 0);
    issue_v(0, 0);
    for (int t = 0; t < n_tiles; t += 2) {
        step(PfBuf<0>{}, t);
        if (t + 1 < n_tiles) step(PfBuf<1>{}, t + 1);
    }
    // epilogue: every row of a lane's ol block holds its query row's
    // denominator; normalise, gate, store
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const float l = ol[nt][0];
        const int rl = rw0 + 16 * nt + r16;
        if (rl >= rows) continue;
        const size_t orow = (((size_t)s * a.n_q + row0 + rl) * kQHeads + h * kGroup + g) * kHeadDim;
        const float inv = __builtin_amdgcn_rcpf(l);
#pragma unroll
        for (int dt = 0; dt < 16; dt++) {
            const int d0 = 16 * dt + 4 * q4;
            float v4[4] = {o[dt][nt][0] * inv, o[dt][nt][1] * inv, o[dt][nt][2] * inv, o[dt][nt][3] * inv};
            if (PRODUCE || a.gate) {
                uint2 gw;
                if constexpr (PRODUCE) {
                    const size_t ge = ((size_t)s * a.n_q + row0 + rl) * kQkvRow +
                                      (size_t)(h * kGroup + g) * 2 * kHeadDim + kHeadDim + d0;
                    if constexpr (F32IN) {
                        const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(a.qkv) + ge);
                        gw = make_uint2(cvt_pk_bf16(f.x, f.y), cvt_pk_bf16(f.z, f.w));
                    } else {
                        gw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.qkv) + ge);
                    }
                } else {
                    gw = *reinterpret_cast<const uint2*>(a.gate + orow + d0);
                }
                v4[0] *= gate_sigmoid(bf16lo(gw.x), a.gate_ref);
                v4[1] *= gate_sigmoid(bf16hi(gw.x), a.gate_ref);
                v4[2] *= gate_sigmoid(bf16lo(gw.y), a.gate_ref);
                v4[3] *= gate_sigmoid(bf16hi(gw.y), a.gate_ref);
            }
            if (a.out_bf16) {
                uint2 w;
                w.x = pack_bf16x2(v4[0], v4[1]);
                w.y = pack_bf16x2(v4[2], v4[3]);
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + orow + d0) = w;
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(a.out) + orow + d0) =
                    make_float4(v4[0], v4[1], v4[2], v4[3]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Append: one workgroup per (sequence, 4 consecutive tokens) moves those
// tokens' K and V rows (4 heads x 512 B each); thread t copies one 16-B piece
// of every token: kv = t / 128, head = (t / 32) % 4, piece = t % 32.  All of a
// thread's loads are issued before its stores.  The sequence and positions are
// workgroup-uniform (scalar), so no lane does index division.  The pool store
// is non-temporal (streamed past L2): for 64 x 128 tokens, 1 token per
// workgroup ran 11.9 us with non-temporal stores (14.9 us with plain ones) and
// 4 tokens per workgroup run 9.8 us.
constexpr int kAppendTok = 4;  // tokens per append workgroup
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    const int per_seq = (a.n_tok + kAppendTok - 1) / kAppendTok;
    const int s = blockIdx.x / per_seq;
    const int tok0 = (blockIdx.x - s * per_seq) * kAppendTok;
    const int t = threadIdx.x;
    const int kv = t >> 7, h = (t >> 5) & 3, part = t & 31;
    const uint16_t* from = kv ? a.v : a.k;
    uint16_t* to = kv ? a.vpool : a.kpool;
    const int32_t* trow = a.table + (size_t)a.slot[s] * a.table_stride;
    u32x4 x[kAppendTok];
#pragma unroll
    for (int i = 0; i < kAppendTok; i++) {
        const int tok = min(tok0 + i, a.n_tok - 1);
        const size_t src = (((size_t)s * a.n_tok + tok) * kKvHeads + h) * kHeadDim + part * 8;
        x[i] = *reinterpret_cast<const u32x4*>(from + src);
    }
#pragma unroll
    for (int i = 0; i < kAppendTok; i++) {
        if (tok0 + i >= a.n_tok) break;
        const int pos = a.pos0[s] + tok0 + i;
        const int blk = trow[pos / kBlockTok];
        const size_t dst = (((size_t)blk * kKvHeads + h) * kBlockTok + pos % kBlockTok) * kHeadDim + part * 8;
        __builtin_nontemporal_store(x[i], reinterpret_cast<u32x4*>(to + dst));
    }
}

// ---------------------------------------------------------------------------
// Attention producer + append: one 320-thread workgroup (5 waves) per
// (sequence, token).  A wave works on two head rows at once, one per 32-lane
// half, each lane holding 8 dims (16 B of bf16 input, 32 B of fp32):
//   normalized rows, pairs (2i, 2i+1) of [q heads 0..15, k heads 0..3]:
//     wave w takes rows 4w .. 4w+3 (wave 4: the k heads), per-head RMSNorm,
//     partial NeoX RoPE, RNE bf16;
//   copied rows [gate heads 0..15, v heads 0..3], same split: RNE bf16.
// The sum of squares is a tree sum inside each 32-lane half.  The RoPE
// partner of dim p < rope_dim/2 is p + rope_dim/2: lane ^ (rope_dim/16) for
// rope_dim >= 16, the other half of the lane's own 8 dims for rope_dim = 8.
// Arithmetic follows the reference's order (src/engine.cpp:3497-3512,
// :2422-2432): (x * r) * w, then x0 c - x1 s and x1 c + x0 s without
// contraction.  Every output is written once and goes non-temporal; the
// projection rows are read with plain loads (64 x 128 tokens of bf16 input:
// 57.7 us, against 61.0 us with non-temporal loads).
constexpr int kQkvWaves = 5;

// tokens per producer workgroup (all their rows are loaded first); 2 and 4
// tokens measured no faster than 1
constexpr int kQkvTok = 1;
// KVONLY: neither q nor gate is written out (the prefill step builds q
// itself), so only the k / v rows have work: a 256-thread workgroup takes 4
// consecutive tokens, one per wave, each wave doing what wave 4 does above
constexpr int kQkvKvWaves = 4;
template <bool BF16IN, bool KVONLY>
__global__ __launch_bounds__(kQkvWaves * 64) void qkv_append_kernel(QkvArgs a) {
#pragma clang fp contract(off)
    constexpr int kTokPerWg = KVONLY ? kQkvKvWaves : kQkvTok;
    const int per_seq = (a.n_tok + kTokPerWg - 1) / kTokPerWg;
    const int s = blockIdx.x / per_seq;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tok0 = (blockIdx.x - s * per_seq) * kTokPerWg + (KVONLY ? wave : 0);
    if (KVONLY && tok0 >= a.n_tok) return;  // whole wave
    const int rw = KVONLY ? kQkvWaves - 1 : wave;  // row group: 4 rw .. 4 rw + 3
    const int hl = lane & 31, sub = lane >> 5;  // lane in the half, which half
    const int d0 = hl * 8;
    const bool kv_wave = rw == kQkvWaves - 1;  // rows 16..19: the kv heads
    // with neither q nor gate written out only the kv wave has work (the
    // host launches the KVONLY form then; this keeps the other correct)
    if (!kv_wave && !a.q_out && !a.gate_out) return;
    constexpr size_t kKOff = (size_t)kQHeads * 2 * kHeadDim;  // k rows, then v rows
    const int half = a.rope_half;
    const bool roped = d0 < 2 * half;
    const int32_t* trow = a.table + (size_t)a.slot[s] * a.table_stride;

    // every input row of this lane, for every token of the workgroup, is
    // requested before anything is stored: rows 4w + 2i + sub of [q 0..15,
    // k 0..3] (normalized) and of [gate 0..15, v 0..3] (copied); copied rows
    // of bf16 input go through as raw 16-B pieces (RNE of a bf16 value is
    // itself), fp32 input is converted
    float x[kQkvTok][2][8], c[kQkvTok][2][8];
    u32x4 craw[kQkvTok][2];
    float cs[kQkvTok][8], sn[kQkvTok][8];
#pragma unroll
    for (int tt = 0; tt < kQkvTok; tt++) {
        const int tok = min(tok0 + tt, a.n_tok - 1);
        const size_t row = ((size_t)s * a.n_tok + tok) * kQkvRow;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = rw * 4 + i * 2 + sub;
            const size_t xo = kv_wave ? row + kKOff + (size_t)(r - kQHeads) * kHeadDim : row + (size_t)r * 2 * kHeadDim;
            const size_t co = kv_wave ? row + kKOff + (size_t)(kKvHeads + r - kQHeads) * kHeadDim
                                      : row + (size_t)r * 2 * kHeadDim + kHeadDim;
            load_row8<BF16IN>(a.qkv, xo + d0, x[tt][i]);
            if (kv_wave || a.gate_out) {
                if constexpr (BF16IN)
                    craw[tt][i] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.qkv) + co + d0);
                else
                    load_row8<BF16IN>(a.qkv, co + d0, c[tt][i]);
            }
        }
        // RoPE coefficients of this lane's 8 dims: table entries p0 .. p0+7
        // for rope_dim >= 16, entries 0..3 twice for rope_dim 8
        const int pos = a.pos0[s] + tok;
        if (roped) {
            const int p0 = half >= 8 ? (d0 & (half - 1)) : 0;
            const float* crow = a.rope + (size_t)pos * half + p0;
            const float* srow = a.rope + ((size_t)a.rope_rows + pos) * half + p0;
            const float4 c0 = *reinterpret_cast<const float4*>(crow);
            const float4 s0 = *reinterpret_cast<const float4*>(srow);
            const float4 c1 = half >= 8 ? *reinterpret_cast<const float4*>(crow + 4) : c0;
            const float4 s1 = half >= 8 ? *reinterpret_cast<const float4*>(srow + 4) : s0;
            cs[tt][0] = c0.x; cs[tt][1] = c0.y; cs[tt][2] = c0.z; cs[tt][3] = c0.w;
            cs[tt][4] = c1.x; cs[tt][5] = c1.y; cs[tt][6] = c1.z; cs[tt][7] = c1.w;
            sn[tt][0] = s0.x; sn[tt][1] = s0.y; sn[tt][2] = s0.z; sn[tt][3] = s0.w;
            sn[tt][4] = s1.x; sn[tt][5] = s1.y; sn[tt][6] = s1.z; sn[tt][7] = s1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                cs[tt][j] = 1.f;
                sn[tt][j] = 0.f;
            }
        }
    }
    const float* wrow = (kv_wave ? a.k_norm : a.q_norm) + d0;
    const float4 w0 = *reinterpret_cast<const float4*>(wrow);
    const float4 w1 = *reinterpret_cast<const float4*>(wrow + 4);
    const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};

#pragma unroll
    for (int tt = 0; tt < kQkvTok; tt++) {
        if (tok0 + tt >= a.n_tok) break;  // uniform
        const int tok = tok0 + tt;
        const int pos = a.pos0[s] + tok;
        const size_t orow = ((size_t)s * a.n_tok + tok) * kQHeads * kHeadDim;
        const int blk = trow[pos / kBlockTok];
        // copied rows: gate heads, or (wave 4) the v heads
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = rw * 4 + i * 2 + sub;
            if (kv_wave) {
                const size_t slot =
                    (((size_t)blk * kKvHeads + (r - kQHeads)) * kBlockTok + pos % kBlockTok) * kHeadDim + d0;
                if constexpr (BF16IN)
                    __builtin_nontemporal_store(craw[tt][i], reinterpret_cast<u32x4*>(a.vpool + slot));
                else
                    store_bf16x8(a.vpool + slot, c[tt][i]);
            } else if (a.gate_out) {
                if constexpr (BF16IN)
                    __builtin_nontemporal_store(craw[tt][i],
                                                reinterpret_cast<u32x4*>(a.gate_out + orow + (size_t)r * kHeadDim + d0));
                else
                    store_bf16x8(a.gate_out + orow + (size_t)r * kHeadDim + d0, c[tt][i]);
            }
        }
        // normalized rows: RMSNorm, RoPE, bf16
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = rw * 4 + i * 2 + sub;  // 0..15 q heads, 16..19 k heads
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) ss += x[tt][i][j] * x[tt][i][j];
            ss = half_wave_sum(ss);
            const float rs = 1.0f / sqrtf(ss / kHeadDim + a.eps);
            float y[8];
#pragma unroll
            for (int j = 0; j < 8; j++) y[j] = x[tt][i][j] * rs * wn[j];
            if (half >= 8) {
                float yp[8];
                switch (half) {  // partner lane ^ (half / 8), uniform
                    case 8: swap_lanes8<1>(y, yp); break;
                    case 16: swap_lanes8<2>(y, yp); break;
                    case 32: swap_lanes8<4>(y, yp); break;
                    case 64: swap_lanes8<8>(y, yp); break;
                    default: swap_lanes8<16>(y, yp); break;
                }
                if (roped) {
                    const bool low = d0 < half;
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        y[j] = low ? y[j] * cs[tt][j] - yp[j] * sn[tt][j] : y[j] * cs[tt][j] + yp[j] * sn[tt][j];
                }
            } else if (half == 4 && roped) {  // rope_dim 8: pairs inside the lane's dims 0..7
                float z[8];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    z[j] = y[j] * cs[tt][j] - y[j + 4] * sn[tt][j];
                    z[j + 4] = y[j + 4] * cs[tt][j + 4] + y[j] * sn[tt][j + 4];
                }
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] = z[j];
            }
            if (kv_wave) {
                const size_t slot =
                    (((size_t)blk * kKvHeads + (r - kQHeads)) * kBlockTok + pos % kBlockTok) * kHeadDim + d0;
                store_bf16x8(a.kpool + slot, y);
            } else if (a.q_out) {
                store_bf16x8(a.q_out + orow + (size_t)r * kHeadDim + d0, y);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Gated-DeltaNet step (src/engine.cpp:3197-3327 decode, :2600-2716 prefill),
// in place on the library's recurrent state [32][128 v][128 k] and conv window
// [3][8192] of one layer.  Workgroup = (sequence, k-head kh): it owns the q and
// k channels of kh and the v channels of the two v-heads kh and kh + 16 that
// read them (v-head vh uses k-head vh % 16), so every conv channel and every
// state row has exactly one owner and the whole step is one launch.
//   state rows: wave w takes v-head kh + 16 (w / 4) and rows
//     32 (w % 4) + 4 r + lane / 16 (r = 0..7); lane l holds k-columns
//     4c .. 4c+3 and 64+4c .. 64+4c+3 (c = l % 16) of its rows, so each 16-B
//     access of a row group is one contiguous 256-B run and a row's dot
//     products reduce over one 16-lane DPP row (4 steps, no cross-row
//     traffic);
//   conv: thread t owns channel t of [q_kh | k_kh | v_vh0 | v_vh1] with its
//     3-row window in registers.
// Per token: conv + SiLU -> LDS, barrier; q, k L2-normalised; decay and beta;
// the delta rule row by row (S *= decay; S += k beta (v_i - S.k); o_i = S.q *
// scale); barrier; gated RMSNorm with SiLU(z).  beta, SiLU and the softplus
// exp follow the reference's Schraudolph forms by default (dn_gates,
// dn_silu below), the hardware units with KVC_FLAG_EXACT_MATH.  Two kernels
// share the row arithmetic (dn_row),
// so a token gives the same bits through either: deltanet_kernel keeps both
// state slabs in registers across a chunk of tokens; deltanet_decode_kernel
// (one token) streams the rows -- loaded ahead, stored as soon as updated.
constexpr int kDnThreads = 512;
constexpr int kDnCols = 8;   // k-columns per lane (16 lanes per state row)
constexpr int kDnRows = 8;   // state rows per lane
constexpr int kDnBlk = 8;    // tokens per block of the chunk kernel

template <bool BF16IN>
__device__ __forceinline__ float load_f(const void* base, size_t off) {
    if constexpr (BF16IN)
        return bf16f(static_cast<const uint16_t*>(base)[off]);
    else
        return static_cast<const float*>(base)[off];
}
// The same element as raw bits, widened by raw_f where it is used: an input
// requested ahead of its use then holds no wait at the request.
template <bool BF16IN>
__device__ __forceinline__ uint32_t load_raw(const void* base, size_t off) {
    if constexpr (BF16IN)
        return static_cast<const uint16_t*>(base)[off];
    else
        return __float_as_uint(static_cast<const float*>(base)[off]);
}
// Raw element of a projection row through a buffer resource: the lane's
// byte offset in a VGPR, the row's (wave-uniform) byte offset in an SGPR, so
// no lane holds a 64-bit address.
template <bool BF16IN>
__device__ __forceinline__ uint32_t load_raw_buf(__amdgpu_buffer_rsrc_t rs, uint32_t lane_off, uint32_t row_off) {
    if constexpr (BF16IN)
        return __builtin_amdgcn_raw_buffer_load_b16(rs, lane_off, row_off, 0);
    else
        return __builtin_amdgcn_raw_buffer_load_b32(rs, lane_off, row_off, 0);
}
template <bool BF16IN>
__device__ __forceinline__ float raw_f(uint32_t r) {
    return __uint_as_float(BF16IN ? r << 16 : r);
}

// Gated-DeltaNet transcendentals on the hardware units (v_exp_f32, v_log_f32,
// v_rcp_f32, v_rsq_f32; each within 2 ulp of the exact value).  The decay's
// exp, the softplus log and the norms' rsqrt always use them; the sigmoid and
// SiLU below use them only with KVC_FLAG_EXACT_MATH (REF = false).  Every
// DeltaNet kernel shares these helpers, so a token gives the same bits
// through any of them.
__device__ __forceinline__ float dn_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float dn_log(float x) { return __builtin_amdgcn_logf(x) * 0.6931471805599453f; }
__device__ __forceinline__ float dn_rsqrt(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + dn_exp(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }

// Reference math (REF, the default; KVC_FLAG_EXACT_MATH clears it): the
// reference's Schraudolph forms.  beta = fast_sigmoidf(beta_raw) (scalar exp,
// truncating conversion, src/engine.cpp:2674 / :3281): the reference's
// scalar division is an IEEE divide even in its fast-math build, so beta
// takes the correctly rounded quotient of sigmoid_ref and matches it bit for
// bit.  SiLU of the conv output and of z is the AVX-512 form (exp converted
// to nearest even, :2626, :2714, :3227, :3321; truncation gives the same
// SiLU bits, see schraudolph_exp), whose fast-math build divides
// by an approximate reciprocal: here v_rcp_f32 (1 ulp), so no exact bits
// exist to match there and the bound is tested against the oracle.  softplus
// takes log(1 + fast_expf(b)) (:2671, :3278).
template <bool REF>
__device__ __forceinline__ float dn_beta(float x) {
    if constexpr (REF)
        return sigmoid_ref(x);
    else
        return sigmoid_f(x);
}
template <bool REF>
__device__ __forceinline__ float dn_silu(float x) {
    if constexpr (REF)
        return x * __builtin_amdgcn_rcpf(1.0f + schraudolph_exp(0.0f - x));
    else
        return silu_f(x);
}

// Workgroup barrier for LDS traffic only: this wave's LDS accesses complete,
// then s_barrier.  Unlike __syncthreads() (a release fence), it does not wait
// for outstanding global loads, so inputs requested ahead of their use stay in
// flight across it.  Only for kernels whose waves exchange data through LDS
// alone.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// sum over the 16 lanes of a DPP row (every lane gets the sum)
__device__ __forceinline__ float sum16(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);  // quads uniform: pairs quad 0 with quad 1
    return x + dpp<kDppRowRor8>(x);
}

// One state row (this lane's 8 columns): decay, delta-rule update; returns
// the row's output dot S_i.q (before the scale).
__device__ __forceinline__ float dn_row(float (&st)[kDnCols], const float (&k)[kDnCols], const float (&q)[kDnCols],
                                        float decay, float beta, float vi) {
#pragma clang fp contract(off)
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int j = 0; j < kDnCols; j += 2) {
        st[j] *= decay;
        st[j + 1] *= decay;
        s0 = fmaf(st[j], k[j], s0);
        s1 = fmaf(st[j + 1], k[j + 1], s1);
    }
    const float sk = sum16(s0 + s1);
    const float dd = beta * (vi - sk);
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int j = 0; j < kDnCols; j += 2) {
        st[j] = fmaf(k[j], dd, st[j]);
        st[j + 1] = fmaf(k[j + 1], dd, st[j + 1]);
        o0 = fmaf(st[j], q[j], o0);
        o1 = fmaf(st[j + 1], q[j + 1], o1);
    }
    return sum16(o0 + o1);
}

// Shared per-token front end: this lane's normalised q and k columns, decay
// and beta of the wave's v-head (conv_lds holds the token's SiLU'd conv).
__device__ __forceinline__ void dn_qk(const float* conv_lds, int col0, float eps, float (&q)[kDnCols],
                                      float (&k)[kDnCols]) {
#pragma clang fp contract(off)
    float qn = 0.f, kn = 0.f;
#pragma unroll
    for (int j = 0; j < kDnCols; j += 4) {
        const int c = col0 + (j ? kSsmDk / 2 : 0);  // columns 4c.. and 64+4c..
        const float4 qq = *reinterpret_cast<const float4*>(conv_lds + c);
        const float4 kk = *reinterpret_cast<const float4*>(conv_lds + 128 + c);
        q[j] = qq.x; q[j + 1] = qq.y; q[j + 2] = qq.z; q[j + 3] = qq.w;
        k[j] = kk.x; k[j + 1] = kk.y; k[j + 2] = kk.z; k[j + 3] = kk.w;
    }
#pragma unroll
    for (int j = 0; j < kDnCols; j++) {
        qn = fmaf(q[j], q[j], qn);
        kn = fmaf(k[j], k[j], kn);
    }
    qn = sum16(qn);
    kn = sum16(kn);
    const float qs = dn_rsqrt(qn + eps), ks = dn_rsqrt(kn + eps);
#pragma unroll
    for (int j = 0; j < kDnCols; j++) {
        q[j] *= qs;
        k[j] *= ks;
    }
}

template <bool REF>
__device__ __forceinline__ void dn_gates(float alpha, float braw, float dtb, float av, float& decay, float& beta) {
#pragma clang fp contract(off)
    const float biased = alpha + dtb;
    const float ex = REF ? schraudolph_exp(biased) : dn_exp(biased);
    const float sp = biased > 20.0f ? biased : dn_log(1.0f + ex);
    decay = dn_exp(sp * av);
    beta = dn_beta<REF>(braw);
}

// gated RMSNorm of one v-head's 128 outputs (o_row) and the store of dims
// 32 wi .. +31 (lanes 0..31)
template <bool REF>
__device__ __forceinline__ void dn_norm_out(const DeltaNetArgs& a, const float* o_row, int lane, int wi, int vh,
                                            size_t out_row, float z) {
#pragma clang fp contract(off)
    const float o0 = o_row[lane], o1 = o_row[lane + 64];
    const float ss = wave_sum(fmaf(o0, o0, o1 * o1));
    const float rms = dn_rsqrt(ss / kSsmDv + a.eps);
    if (lane < 32) {
        const int d = wi * 32 + lane;
        const float y = o_row[d] * rms * a.norm_w[d] * dn_silu<REF>(z);
        const size_t oi = out_row + (size_t)vh * kSsmDv + d;
        if (a.out_bf16)
            static_cast<uint16_t*>(a.out)[oi] = (uint16_t)f32_to_bf16_rne(y);
        else
            static_cast<float*>(a.out)[oi] = y;
    }
}

__device__ __forceinline__ int dn_channel(int t, int kh) {
    const int part = t >> 7, ci = t & 127;
    return part == 0   ? kh * kSsmDk + ci
           : part == 1 ? kSsmKHeads * kSsmDk + kh * kSsmDk + ci
                       : 2 * kSsmKHeads * kSsmDk + (kh + kSsmKHeads * (part - 2)) * kSsmDv + ci;
}

// Streaming access to the recurrent state for the kernels whose wave
// instructions each cover whole 256-B row pieces: each element is read once
// and written once per step, so the loads and stores are non-temporal (no
// cache allocation for data that will not be reused before it is evicted).
// Measured on the one-token step: 58.9 -> 51.1 us per layer at config e, most
// of it from the stores.  The matrix-form kernel's slices are 16-B pieces
// 128 B apart per instruction; there non-temporal access was slower.
__device__ __forceinline__ float4 nt_ld4(const float* p) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void nt_st4(float* p, float x, float y, float z, float w) {
    __builtin_nontemporal_store(f32x4{x, y, z, w}, reinterpret_cast<f32x4*>(p));
}

template <bool BF16IN, bool REF, bool MULTI>
__global__ __launch_bounds__(kDnThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void deltanet_kernel(DeltaNetArgs a) {
#pragma clang fp contract(off)
    // Tokens go in blocks of kDnBlk.  Per block:
    //   P1 (token-parallel) thread t = owned channel: conv1d + SiLU of the
    //      block's tokens, window in registers -> xs[tok][t];
    //   P2 (token-parallel) 16-lane group g normalises token g's q and k in
    //      place (dn_qk, same lanes as the one-token kernel); lanes 0..2nb-1
    //      compute (decay, beta) of (token, v-head);
    //   P3 (sequential) every lane updates its 8 state rows token after token
    //      (dn_row) with no barrier inside the block -> os[tok][vl][row]; the
    //      last block stores the state right after it;
    //   P4 (token-parallel) wave w writes the gated RMSNorm of (token,
    //      v-head) pairs w, w + 8, ...
    // A block's inputs (conv inputs and taps, gate inputs and weights, z) are
    // requested before the state (first block) or during the block before,
    // and are used or staged in LDS in P1, so no phase waits for state loads
    // it does not read and no input stays live in registers through the
    // delta rule.  The barriers wait for LDS traffic only.  The
    // arithmetic is that of the one-token kernel, so a token gives the same
    // bits.
    __shared__ float xs[kDnBlk][4 * 128];        // q_kh, k_kh, v_vh0, v_vh1 of each token
    __shared__ float2 gs[kDnBlk][2];             // (decay, beta) per token and v-head
    __shared__ float os[kDnBlk][2][kSsmDv];      // scaled recurrence outputs
    __shared__ float zs[2][kDnBlk][2][kSsmDv];   // z of each token and v-head (by block parity)
    __shared__ float nws[kSsmDv];                // output-norm weights
    const int b = blockIdx.x;
    const int s = b / kSsmKHeads;
    const int kh = b - s * kSsmKHeads;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: head data in SGPRs
    const int vl = wave >> 2, wi = wave & 3;
    const int vh = kh + kSsmKHeads * vl;
    const int rg = lane >> 4, col0 = (lane & 15) * 4;
    const int rbase = wi * 32 + rg;  // rows rbase + 4 r

    uint8_t* slot = a.state + (size_t)a.slot[s] * a.state_bytes + a.layer_off;
    float* S = reinterpret_cast<float*>(slot) + (size_t)vh * kSsmDv * kSsmDk + col0;
    float* conv = reinterpret_cast<float*>(slot + a.rec_bytes);
    constexpr size_t kZ = kSsmC, kAlpha = kSsmC + kSsmVHeads * kSsmDv, kBeta = kAlpha + kSsmVHeads;
    constexpr int kZPer = kDnBlk * 2 * kSsmDv / kDnThreads;  // z values each thread stages
    const size_t prow0 = (size_t)s * a.n_tok * kSsmProj;
    const int g16 = t >> 4;  // 16-lane group of P2
    const int ch = dn_channel(t, kh);
    // gate thread t < 2 kDnBlk serves (token t / 2, v-head t % 2)
    const int gt = t >> 1, gvh = kh + kSsmKHeads * (t & 1);

    // one block's inputs: conv inputs and taps of channel ch, the gate
    // inputs and weights, and kZPer z values (flat index t + 512 j of
    // [token][v-head][dim]).  Every load is unconditional, its token index
    // clamped to the call (values of tokens past the end are never used): a
    // load under a branch is followed by a wait for it at the branch's end.
    float xin[kDnBlk], zr[kZPer];
    float4 cw;
    float gal, gbr, gdtb, gav;
    auto tok_row = [&](int tok) { return prow0 + (size_t)min(tok, a.n_tok - 1) * kSsmProj; };
    auto load_inputs = [&](int tok0) {
        cw = make_float4(a.conv_w[ch], a.conv_w[kSsmC + ch], a.conv_w[2 * kSsmC + ch], a.conv_w[3 * kSsmC + ch]);
#pragma unroll
        for (int i = 0; i < kDnBlk; i++) xin[i] = load_f<BF16IN>(a.proj, tok_row(tok0 + i) + ch);
        {
            const size_t row = tok_row(tok0 + (gt & (kDnBlk - 1)));
            gal = load_f<BF16IN>(a.proj, row + kAlpha + gvh);
            gbr = load_f<BF16IN>(a.proj, row + kBeta + gvh);
            gdtb = a.dt_bias[gvh];
            gav = a.a[gvh];
        }
#pragma unroll
        for (int j = 0; j < kZPer; j++) {
            const int f = t + kDnThreads * j, zt = f / (2 * kSsmDv), zv = (f / kSsmDv) & 1, d = f % kSsmDv;
            zr[j] = load_f<BF16IN>(a.proj, tok_row(tok0 + zt) + kZ + (size_t)(kh + kSsmKHeads * zv) * kSsmDv + d);
        }
    };
    float w0 = conv[ch], w1 = conv[kSsmC + ch], w2 = conv[2 * kSsmC + ch];  // window, oldest first
    const float nwr = a.norm_w[t & (kSsmDv - 1)];
    load_inputs(0);

    float st[kDnRows][kDnCols];
#pragma unroll
    for (int r = 0; r < kDnRows; r++) {
        const float* src = S + (size_t)(rbase + 4 * r) * kSsmDk;
        const float4 x0 = nt_ld4(src);
        const float4 x1 = nt_ld4(src + kSsmDk / 2);
        st[r][0] = x0.x; st[r][1] = x0.y; st[r][2] = x0.z; st[r][3] = x0.w;
        st[r][4] = x1.x; st[r][5] = x1.y; st[r][6] = x1.z; st[r][7] = x1.w;
    }
    nws[t & (kSsmDv - 1)] = nwr;  // every thread: no branch for the load to sink into

    // one block of nb tokens from tok0; LAST: the call's last block, which
    // stores the state.  A second block requests its inputs at its start
    // (the state has arrived by then).
    auto run_block = [&](auto last_c, int tok0, int nb) {
        constexpr bool LAST = decltype(last_c)::value;
        const int zb = (tok0 / kDnBlk) & 1;
        if (tok0 > 0) load_inputs(tok0);
        // P1: conv1d + SiLU, window pushed per token; gates; z staged (the
        // previous block's P3 is done with gs, and its P4 reads the other zs)
        if (t < 2 * nb) {
            float decay, beta;
            dn_gates<REF>(gal, gbr, gdtb, gav, decay, beta);
            gs[gt][t & 1] = make_float2(decay, beta);
        }
#pragma unroll
        for (int j = 0; j < kZPer; j++) (&zs[zb][0][0][0])[t + kDnThreads * j] = zr[j];
#pragma unroll
        for (int i = 0; i < kDnBlk; i++) {
            if (i < nb) {
                const float x = xin[i];
                float sum = w0 * cw.x;
                sum = fmaf(w1, cw.y, sum);
                sum = fmaf(w2, cw.z, sum);
                sum = fmaf(x, cw.w, sum);
                xs[i][t] = dn_silu<REF>(sum);
                w0 = w1;
                w1 = w2;
                w2 = x;
            }
        }
        lds_barrier();
        // P2: q/k normalisation in place
        if (g16 < nb) {
            float q[kDnCols], k[kDnCols];
            dn_qk(xs[g16], col0, a.eps, q, k);
#pragma unroll
            for (int j = 0; j < kDnCols; j += 4) {
                const int c = col0 + (j ? kSsmDk / 2 : 0);
                *reinterpret_cast<float4*>(&xs[g16][c]) = make_float4(q[j], q[j + 1], q[j + 2], q[j + 3]);
                *reinterpret_cast<float4*>(&xs[g16][128 + c]) = make_float4(k[j], k[j + 1], k[j + 2], k[j + 3]);
            }
        }
        lds_barrier();
        // P3: the delta rule, token after token; the 16 lanes of a row hold
        // the same output and all store it (one LDS word, same value)
        {
            for (int i = 0; i < nb; i++) {
                float q[kDnCols], k[kDnCols];
#pragma unroll
                for (int j = 0; j < kDnCols; j += 4) {
                    const int c = col0 + (j ? kSsmDk / 2 : 0);
                    const float4 qq = *reinterpret_cast<const float4*>(&xs[i][c]);
                    const float4 kk = *reinterpret_cast<const float4*>(&xs[i][128 + c]);
                    q[j] = qq.x; q[j + 1] = qq.y; q[j + 2] = qq.z; q[j + 3] = qq.w;
                    k[j] = kk.x; k[j + 1] = kk.y; k[j + 2] = kk.z; k[j + 3] = kk.w;
                }
                const float2 gb = gs[i][vl];
#pragma unroll
                for (int r = 0; r < kDnRows; r++)
                    os[i][vl][rbase + 4 * r] =
                        dn_row(st[r], k, q, gb.x, gb.y, xs[i][256 + vl * 128 + rbase + 4 * r]) * a.out_scale;
            }
            if constexpr (LAST) {
#pragma unroll
                for (int r = 0; r < kDnRows; r++) {
                    float* dst = S + (size_t)(rbase + 4 * r) * kSsmDk;
                    nt_st4(dst, st[r][0], st[r][1], st[r][2], st[r][3]);
                    nt_st4(dst + kSsmDk / 2, st[r][4], st[r][5], st[r][6], st[r][7]);
                }
            }
        }
        lds_barrier();
        // P4: gated RMSNorm of (token, v-head) pairs, all 128 dims per wave
#pragma unroll
        for (int pi = 0; pi < 2; pi++) {
            const int p = wave + 8 * pi;
            if (p >= 2 * nb) break;
            const int pt = p >> 1, pv = p & 1, pvh = kh + kSsmKHeads * pv;
            const float* o_row = os[pt][pv];
            const float o0 = o_row[lane], o1 = o_row[lane + 64];
            const float ss = wave_sum(fmaf(o0, o0, o1 * o1));
            const float rms = dn_rsqrt(ss / kSsmDv + a.eps);
            const size_t out_row = ((size_t)s * a.n_tok + tok0 + pt) * (kSsmVHeads * kSsmDv) + (size_t)pvh * kSsmDv;
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++) {
                const int d = lane + 64 * h2;
                const float y = o_row[d] * rms * nws[d] * dn_silu<REF>(zs[zb][pt][pv][d]);
                if (a.out_bf16)
                    static_cast<uint16_t*>(a.out)[out_row + d] = (uint16_t)f32_to_bf16_rne(y);
                else
                    static_cast<float*>(a.out)[out_row + d] = y;
            }
        }
    };
    // MULTI: kDnBlk + 1 .. kDnMatrixMin - 1 tokens (longer calls run the matrix
    // form); otherwise 2 .. kDnBlk.  Separate instantiations keep the common
    // one-block call free of the second block's register pressure.
    if constexpr (MULTI) {
        run_block(std::false_type{}, 0, kDnBlk);
        run_block(std::true_type{}, kDnBlk, a.n_tok - kDnBlk);
    } else {
        run_block(std::true_type{}, 0, a.n_tok);
    }
    conv[ch] = w0;
    conv[kSsmC + ch] = w1;
    conv[2 * kSsmC + ch] = w2;
}

// ---------------------------------------------------------------------------
// Gated-DeltaNet over chunks of 16 tokens in matrix form, on fp32 MFMA
// (v_mfma_f32_16x16x4_f32).  Same workgroup (sequence, k-head kh, both
// v-heads), front end (conv, q/k norms, gates) and output norm as
// deltanet_kernel; the token loop of the delta rule is replaced by products
// of 16-token blocks.  With a_t the decay, g_t = sum_{r<=t} log a_r (within
// the chunk), S the state at the chunk start and U the rows
// dd_t = beta_t (v_t - a_t S_{t-1} k_t):
//   W1 = K S^T, W2 = Q S^T                                   [16 x 128]
//   L  = I + diag(beta) (strict lower of e^{g_t - g_s} K K^T), T = L^-1
//   U  = T diag(beta) (V - diag(e^g) W1)
//   O  = diag(e^g) W2 + (lower incl. diagonal of e^{g_t - g_s} Q K^T) U
//   S^T <- e^{g_C} S^T + Kt^T U,  Kt[s] = e^{g_C - g_s} k_s
// which unrolls the per-token recurrence exactly (in real arithmetic); the
// fp32 rounding differs from the token-by-token order.
//
// Wave w holds v-columns 32 (w % 4) .. +31 of v-head kh + 16 (w / 4): its
// state slice is kept as MFMA B fragments, lane (g = l / 16, c = l % 16)
// holding S^T[16 m + 4 g + e][i0 + c] in register e of fragment m (the k-dim
// order of every product is k = 16 m + 4 g + e, so the four lane groups of a
// state row hold 64 contiguous bytes of it per fragment), and the state
// update's MFMA m, whose A rows are k = 16 m .. 16 m + 15, lands in that same
// layout.
// Token rows of W1, U and O are taken in the order sigma(r) = 4 (r % 4) + r / 4
// so that lane group g, register r of each of them is token 4 r + g: the
// B fragment of a 4-token step j of the next product is then register j.
// Tokens past the end of the last chunk enter as zero rows with beta = 0
// and log decay 0, which leaves U, O and S unchanged.
constexpr int kDnChunk = 16;
// Calls of this many tokens or more run the matrix form (one partial block
// below 16).  Measured at config e (64 sessions, interleaved): the blocked
// kernel takes 84.0-85.4 / 89.9-90.2 us per layer at 12 / 13 tokens, the
// matrix form 86.8 / 86.9-87.1; the two meet between 12 and 13.
constexpr int kDnMatrixMin = 13;
static_assert(kDnMatrixMin <= 2 * kDnBlk, "the blocked kernel covers calls of at most two blocks");

__device__ __forceinline__ int dn_sigma(int r) { return 4 * (r & 3) + (r >> 2); }

// Two fp32 values times a power of two s, each as two fp16 parts: h = RNE
// fp16 of x s (v_fma_mixlo/hi_f16), m = x s - h (exact, v_fma_mix_f32)
// rounded toward zero to fp16.  x s = h + m within 2^-21 |x s| as long as
// |x s| < 65504 and m is not subnormal; products on fp16 MFMA then take
// h.h' + h.m' + m.h' (the dropped m.m' is below 2^-22 of the product).
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ void dn_split2(float x0, float x1, float s, uint32_t& hp, uint32_t& mp) {
    uint32_t h;
    float r0, r1;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "=v"(h) : "v"(x0), "v"(s));
    asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "+v"(h) : "v"(x1), "v"(s));
    asm("v_fma_mix_f32 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=v"(r0) : "v"(x0), "v"(s), "v"(h));
    asm("v_fma_mix_f32 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(r1) : "v"(x1), "v"(s), "v"(h));
    hp = h;
    mp = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}
__device__ __forceinline__ void dn_split8(const float (&x)[8], float s, f16x8_t& h, f16x8_t& m) {
    u32x4 hw, mw;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t a, b;
        dn_split2(x[2 * i], x[2 * i + 1], s, a, b);
        hw[i] = a;
        mw[i] = b;
    }
    h = __builtin_bit_cast(f16x8_t, hw);
    m = __builtin_bit_cast(f16x8_t, mw);
}
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
// dn_split2 with a scale per value (both powers of two, or any positive
// factors: m = x s - h is then the fp32 rounding of the exact difference)
__device__ __forceinline__ void dn_split2s(float x0, float x1, float s0, float s1, uint32_t& hp, uint32_t& mp) {
    uint32_t h;
    float r0, r1;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "=v"(h) : "v"(x0), "v"(s0));
    asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "+v"(h) : "v"(x1), "v"(s1));
    asm("v_fma_mix_f32 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=v"(r0) : "v"(x0), "v"(s0), "v"(h));
    asm("v_fma_mix_f32 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(r1) : "v"(x1), "v"(s1), "v"(h));
    hp = h;
    mp = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}
__device__ __forceinline__ void dn_split4(const float (&x)[4], const float (&s)[4], f16x4_t& h, f16x4_t& m) {
    u32x2 hw, mw;
    uint32_t a, b;
    dn_split2s(x[0], x[1], s[0], s[1], a, b);
    hw[0] = a;
    mw[0] = b;
    dn_split2s(x[2], x[3], s[2], s[3], a, b);
    hw[1] = a;
    mw[1] = b;
    h = __builtin_bit_cast(f16x4_t, hw);
    m = __builtin_bit_cast(f16x4_t, mw);
}
// largest |entry| of a column held as 4 lane groups x N registers -> the
// split scale 2^(141 - e) and the inverse of (scale x 2^14), 2^(e - 155), for
// the column's biased exponent e clamped to [29, 254]
__device__ __forceinline__ float dn_col_scale(float mx, float& sc, float& inv) {
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const int ex = min(max((int)(__float_as_uint(mx) >> 23), 29), 254);
    sc = __uint_as_float((uint32_t)(268 - ex) << 23);
    inv = __uint_as_float((uint32_t)(ex - 28) << 23);
    return mx;
}
__device__ __forceinline__ f32x4 dn_mfma3(const f16x8_t& ah, const f16x8_t& am, const f16x8_t& bh,
                                          const f16x8_t& bm, f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bm, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
}

// One wave: A B for 16 x 16 row-major fp32 matrices in LDS; lane (g, c)
// returns rows 4 g .. 4 g + 3 of column c.
__device__ __forceinline__ f32x4 dn_m16(const float (*A)[kDnChunk], const float (*B)[kDnChunk], int g, int c) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; j++)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[c][4 * j + g], B[4 * j + g][c], acc, 0, 0, 0);
    return acc;
}

// Waves 0-7 hold the state (as above) and run the block products; waves 8-15
// run everything that does not depend on the state, ahead of it.  Per block
// b, two phases separated by LDS-only barriers:
//   A: W1, W2 of block b     | L and T (helpers 0, 1, one v-head each), M
//                              (helpers 2, 3) of block b; q/k norms of
//                              block b + 1 (helpers 4..7)
//   B: U, O, state update    | K K^T, Q K^T (helpers 0, 1) and prefix sums
//      of block b              (helper 2) of block b + 1; conv and gates of
//                              block b + 2; output norm of block b - 1
// The loop starts two blocks early (b = -2, -1 run only the helpers' part),
// so that the first blocks take the same code path as the rest.  Inputs are
// requested a phase or more ahead of their use: conv inputs with alpha and
// beta one iteration ahead, z values one phase.  A SIMD holds two state
// waves and two helper waves, so the helpers' memory and LDS latency
// overlaps the state waves' MFMAs.  Their VALU work does not: measured phase
// times come out as the SIMD's MFMA time plus the helpers' VALU time.
// Per-block LDS data are triple buffered (token rows, gate data: written two
// blocks ahead) or double buffered (outputs).  The kernel is persistent (one
// workgroup per CU, items taken in turn), so "block b" is a position in the
// workgroup's stream of blocks over its items; the two-block pipeline fill
// happens once per workgroup, not once per item.
constexpr int kDnMathWaves = 8;
constexpr int kDnHelpWaves = 8;
constexpr int kDnMfmaThreads = 64 * (kDnMathWaves + kDnHelpWaves);

template <bool BF16IN, bool BF16OUT, bool REF>
__global__ __launch_bounds__(kDnMfmaThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void deltanet_mfma_kernel(DeltaNetArgs a) {
#pragma clang fp contract(off)
    // q_kh, k_kh (normalised), v_vh0, v_vh1 of each token; rows padded by 4
    // floats so that lanes reading one column of 16 token rows hit 16
    // different 4-bank groups
    __shared__ float xs[3][kDnChunk][4 * 128 + 4];
    __shared__ float lg[3][2][kDnChunk];          // log decay per v-head and token, then g_t
    __shared__ float bt[3][2][kDnChunk];          // beta
    __shared__ float eg[3][2][kDnChunk];          // e^{g_t}
    __shared__ float fc[3][2][kDnChunk];          // e^{g_C - g_t}
    __shared__ float kk[kDnChunk][kDnChunk];      // K K^T
    __shared__ float qk[kDnChunk][kDnChunk];      // Q K^T
    __shared__ float lm[2][kDnChunk][kDnChunk];   // strict lower of L, then T = L^-1
    __shared__ float mm[2][kDnChunk][kDnChunk];   // e^{g_t - g_s} Q K^T, s <= t
    __shared__ float sc[2][3][kDnChunk][kDnChunk];  // N^2 (then the running product), N^4, N^8
    // K and Q of the next block as fp16 MFMA fragments, split into two parts
    // after a scale of 2^14: [K, Q][32-k step][lane group][h, m][row in
    // sigma order], 16 B each (consecutive rows on consecutive 16 B)
    __shared__ u32x4 kqf[2][4][4][2][kDnChunk];
    __shared__ float os[2][kDnChunk][2][kSsmDv];  // scaled recurrence outputs
    // Persistent: workgroup w runs items (sequence, k-head) w, w + G, ...
    // (G = grid size) as one stream of blocks; position q of the stream is
    // block q % nblk of item w + (q / nblk) G.  The helpers' pipeline runs
    // across item boundaries, and a state wave's switch to the next item is
    // one store and one load of its slice.
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int nblk = (a.n_tok + kDnChunk - 1) / kDnChunk;
    const int n_items = a.n_seqs * kSsmKHeads;
    const int n_my = ((int)(n_items - blockIdx.x) + (int)gridDim.x - 1) / (int)gridDim.x;  // >= 1
    const int n_pos = n_my * nblk;
    auto item_at = [&](int q) { return (int)blockIdx.x + (max(min(q, n_pos - 1), 0) / nblk) * (int)gridDim.x; };
    auto slot_of = [&](int item) {
        return a.state + (size_t)a.slot[item / kSsmKHeads] * a.state_bytes + a.layer_off;
    };

    // The state waves and the helper waves run separate loops with the same
    // number of barriers (two per iteration), so that neither holds the
    // other's registers.
    if (wave < kDnMathWaves) {
        // v-head hl, v-columns ibase .. +31 (two 16-column tiles); state
        // slice as B fragments: st[vt][m] = S^T[16 m + 4 g .. +3][ibase + 16 vt + c].
        // The k order k = 16 m + 4 g + e (every product uses it) puts the four
        // lane groups of a state row on 64 contiguous bytes, so each load or
        // store instruction of a slice covers 16 rows x 64 B
        const int hl = wave >> 2;
        const int ibase = 32 * (wave & 3);
        auto slice_of = [&](int item) {
            return reinterpret_cast<float*>(slot_of(item)) + (size_t)(item % kSsmKHeads + kSsmKHeads * hl) * kSsmDv * kSsmDk;
        };
        f32x4 st[2][8];
        auto load_state = [&](const float* S) {
#pragma unroll
            for (int vt = 0; vt < 2; vt++) {
                const float* src = S + (size_t)(ibase + 16 * vt + c) * kSsmDk + 4 * g;
#pragma unroll
                for (int m = 0; m < 8; m++) st[vt][m] = *reinterpret_cast<const f32x4*>(src + 16 * m);
            }
        };
        // The registers hold S^T / dk: the blocks' decays e^{g_C} multiply the
        // wave-uniform factor dk instead of the 64 state values, so an update
        // adds its product scaled by 1 / dk with one fma per value.  Once dk
        // falls below 2^-80 the next update folds it back (S^T dk e^{g_C} +
        // the product, as without the factor) and dk restarts at 1.  Slices
        // are stored and loaded in true units.
        float dk = 1.f;
        auto store_state = [&](float* S) {
#pragma unroll
            for (int vt = 0; vt < 2; vt++) {
                float* dst = S + (size_t)(ibase + 16 * vt + c) * kSsmDk + 4 * g;
#pragma unroll
                for (int m = 0; m < 8; m++) *reinterpret_cast<f32x4*>(dst + 16 * m) = st[vt][m] * dk;
            }
        };
        // smax[vt]: an upper bound of |S^T| over column c of tile vt, exact
        // after each slice load and carried through the updates as
        // e^{g_C} smax + 16 max|fc U| (|K| <= 1 after the normalisation, 16
        // tokens per block); the phase-A split scales come from it.  An
        // overestimate by 2^k costs the split nothing while k < 17.
        float smax[2];
        auto col_max = [&] {
#pragma unroll
            for (int vt = 0; vt < 2; vt++) {
                float mx = 0.f;
#pragma unroll
                for (int m = 0; m < 8; m++)
#pragma unroll
                    for (int e = 0; e < 4; e++) mx = fmaxf(mx, fabsf(st[vt][m][e]));
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                smax[vt] = fmaxf(mx, __shfl_xor(mx, 32));
            }
        };
        load_state(slice_of(item_at(0)));
        col_max();
        lds_barrier();  // positions -2, -1
        lds_barrier();
        lds_barrier();
        lds_barrier();
        for (int bb = 0; bb < n_pos; bb++) {
            if (bb > 0 && bb % nblk == 0) {  // next item: this slice out, the next one in
                store_state(slice_of(item_at(bb - 1)));
                load_state(slice_of(item_at(bb)));
                dk = 1.f;
                col_max();
            }
            const int cur = bb % 3;
            const float(*x)[4 * 128 + 4] = xs[cur];
            // Phase A: W1 = K S^T and W2 = Q S^T (rows in sigma order) on
            // fp16 MFMA (v_mfma_f32_16x16x32_f16, 32 k per step in the order
            // 4 g + e, 16 + 4 g + e of both operands), each operand split
            // into two fp16 parts after a power-of-two scale: K and Q by 2^14
            // (entries at most 1 after the normalisation), each state column
            // so that its largest entry lies in [2^14, 2^15).
            f32x4 w1a[2] = {}, w2a[2] = {};
            {
                float ssc[2], sinv[2];
#pragma unroll
                for (int vt = 0; vt < 2; vt++) {
                    const int ex = min(max((int)(__float_as_uint(smax[vt]) >> 23), 29), 254);
                    ssc[vt] = __uint_as_float((uint32_t)(268 - ex) << 23);   // 2^(141 - ex)
                    sinv[vt] = __uint_as_float((uint32_t)(ex - 28) << 23) * dk;  // dk 2^-14 / ssc
                }
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    const f16x8_t kh = __builtin_bit_cast(f16x8_t, kqf[0][ks][g][0][c]);
                    const f16x8_t km = __builtin_bit_cast(f16x8_t, kqf[0][ks][g][1][c]);
                    const f16x8_t qh = __builtin_bit_cast(f16x8_t, kqf[1][ks][g][0][c]);
                    const f16x8_t qm = __builtin_bit_cast(f16x8_t, kqf[1][ks][g][1][c]);
#pragma unroll
                    for (int vt = 0; vt < 2; vt++) {
                        const float sv[8] = {st[vt][2 * ks][0],     st[vt][2 * ks][1],     st[vt][2 * ks][2],
                                             st[vt][2 * ks][3],     st[vt][2 * ks + 1][0], st[vt][2 * ks + 1][1],
                                             st[vt][2 * ks + 1][2], st[vt][2 * ks + 1][3]};
                        f16x8_t sh, sm;
                        dn_split8(sv, ssc[vt], sh, sm);
                        w1a[vt] = dn_mfma3(kh, km, sh, sm, w1a[vt]);
                        w2a[vt] = dn_mfma3(qh, qm, sh, sm, w2a[vt]);
                    }
                }
#pragma unroll
                for (int vt = 0; vt < 2; vt++) {
                    w1a[vt] *= sinv[vt];
                    w2a[vt] *= sinv[vt];
                }
            }
            lds_barrier();
            // Phase B: U = T diag(beta) (V - diag(e^g) W1); O = diag(e^g) W2 + M U;
            // S^T <- e^{g_C} S^T + Kt^T U.  Lane group g, register r <-> token 4 r + g.
            const float egc = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(eg[cur][hl][kDnChunk - 1])));  // uniform
            f32x4 uu[2];
#pragma unroll
            for (int vt = 0; vt < 2; vt++) {
                const int i = ibase + 16 * vt + c;
                f32x4 rhs;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int tau = 4 * r + g;
                    rhs[r] = bt[cur][hl][tau] * (x[tau][256 + 128 * hl + i] - eg[cur][hl][tau] * w1a[vt][r]);
                }
                f32x4 acc = {};
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(lm[hl][dn_sigma(c)][4 * j + g], rhs[j], acc, 0, 0, 0);
                uu[vt] = acc;
                f32x4 o;
#pragma unroll
                for (int r = 0; r < 4; r++) o[r] = eg[cur][hl][4 * r + g] * w2a[vt][r];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    o = __builtin_amdgcn_mfma_f32_16x16x4f32(mm[hl][dn_sigma(c)][4 * j + g], uu[vt][j], o, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) os[bb & 1][4 * r + g][hl][i] = o[r] * a.out_scale;
            }
            // state update on fp16 MFMA (v_mfma_f32_16x16x16_f16: the block's
            // 16 tokens in one step, lane group g element r = token 4 r + g,
            // the layout U already has): Kt^T U = K^T (diag(fc) U), K^T as
            // fragments the helpers split in phase A (scale 2^14), diag(fc) U
            // split per column with the factors fc in the split's multipliers;
            // the product is scaled back and added to e^{g_C} S^T
            f16x4_t uh[2], um[2];
            float uinv[2];
            float fcv[4];
            const float dkn = dk * egc;
            const bool fold = !(dkn >= 0x1p-80f);  // uniform
            const float rdk = fold ? 1.f : 1.f / dkn;
#pragma unroll
            for (int r = 0; r < 4; r++) fcv[r] = fc[cur][hl][4 * r + g];
#pragma unroll
            for (int vt = 0; vt < 2; vt++) {
                const float uv[4] = {uu[vt][0] * fcv[0], uu[vt][1] * fcv[1], uu[vt][2] * fcv[2], uu[vt][3] * fcv[3]};
                float usc;
                const float mu = dn_col_scale(fmaxf(fmaxf(fabsf(uv[0]), fabsf(uv[1])), fmaxf(fabsf(uv[2]), fabsf(uv[3]))),
                                              usc, uinv[vt]);
                const float us[4] = {usc, usc, usc, usc};
                dn_split4(uv, us, uh[vt], um[vt]);
                smax[vt] = fold ? fmaf(16.f, mu, dkn * smax[vt]) : fmaf(16.f * mu, rdk, smax[vt]);
                uinv[vt] *= rdk;
            }
            const u32x4* ktf = reinterpret_cast<const u32x4*>(&x[lane >> 5][0]) + (lane & 31);
            if (fold) {  // uniform
#pragma unroll
                for (int vt = 0; vt < 2; vt++)
#pragma unroll
                    for (int m = 0; m < 8; m++) st[vt][m] *= dkn;
            }
            dk = fold ? 1.f : dkn;
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const u32x4 kf = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(ktf) + 2 * m * sizeof(x[0]));
                const f16x4_t kh = __builtin_bit_cast(f16x4_t, u32x2{kf[0], kf[1]});
                const f16x4_t km = __builtin_bit_cast(f16x4_t, u32x2{kf[2], kf[3]});
#pragma unroll
                for (int vt = 0; vt < 2; vt++) {
                    f32x4 t = __builtin_amdgcn_mfma_f32_16x16x16f16(km, uh[vt], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, um[vt], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, uh[vt], t, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; e++) st[vt][m][e] = fmaf(t[e], uinv[vt], st[vt][m][e]);
                }
            }
            lds_barrier();
        }
        store_state(slice_of(item_at(n_pos - 1)));
        return;
    }

    // ---- helper waves: thread u owns conv channel u (and xs column u) of
    // the current item ----
    // The helpers issue ahead of the state waves on their SIMD (wave
    // priority 2 against 0): their phase work is a latency chain, and with
    // equal priority the older state waves' MFMA streams delay it.
    __builtin_amdgcn_s_setprio(2);
    constexpr size_t kZ = kSsmC, kAlpha = kSsmC + kSsmVHeads * kSsmDv, kBeta = kAlpha + kSsmVHeads;
    const int last_tok = a.n_tok - 1;
    const int u = t - 64 * kDnMathWaves;
    const int hw = wave - kDnMathWaves;
    // Buffer resources over one sequence's projection rows (the launch
    // checks that they span less than 2 GiB) and outputs.  Loads take the
    // row's byte offset in an SGPR and the element's in a VGPR, with token
    // indices clamped to the sequence; a store whose offset is past the end
    // (kDrop) is discarded by the hardware, so every output pair is stored
    // unconditionally.
    constexpr uint32_t kElt = BF16IN ? 2u : 4u;
    constexpr uint32_t osz = BF16OUT ? 2u : 4u;
    auto proj_rs = [&](int seq) {
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(static_cast<const char*>(a.proj) + (size_t)seq * a.n_tok * kSsmProj * kElt), 0,
            (int)((uint32_t)a.n_tok * (uint32_t)kSsmProj * kElt), 0x00020000);
    };
    auto out_rs = [&](int seq) {
        return __builtin_amdgcn_make_buffer_rsrc(
            static_cast<char*>(a.out) + (size_t)seq * a.n_tok * (kSsmVHeads * kSsmDv) * osz, 0,
            (int)((uint32_t)a.n_tok * (uint32_t)(kSsmVHeads * kSsmDv) * osz), 0x00020000);
    };
    auto row_off = [&](int tok) { return (uint32_t)max(min(tok, last_tok), 0) * (uint32_t)kSsmProj * kElt; };
    constexpr uint32_t kDrop = 0xFFFFFF00u;
    // gate pair (token ab_t, v-head offset ab_h) of lane u % 32 (helper 3's
    // lanes 0..31 compute theirs); norm lanes: helpers 4..7, token g16,
    // columns of c
    const int ab_t = (u >> 1) & (kDnChunk - 1), ab_h = u & 1;
    const float nw0 = a.norm_w[lane], nw1 = a.norm_w[lane + 64];
    const int g16 = (u - 256) >> 4, col0 = c * 4;
    constexpr int kPairs = 2 * kDnChunk / kDnHelpWaves;  // output pairs per helper wave

    // conv channel, weights and window of the item whose conv runs next
    int cv_item = -1;
    float* conv = nullptr;
    int ch = 0;
    float4 cw = {};
    float w0 = 0.f, w1 = 0.f, w2 = 0.f, dtb_g = 0.f, a_g = 0.f;
    auto conv_item = [&](int item) {
        conv = reinterpret_cast<float*>(slot_of(item) + a.rec_bytes);
        const int kh = item % kSsmKHeads;
        ch = dn_channel(u, kh);
        cw = make_float4(a.conv_w[ch], a.conv_w[kSsmC + ch], a.conv_w[2 * kSsmC + ch], a.conv_w[3 * kSsmC + ch]);
        w0 = conv[ch];
        w1 = conv[kSsmC + ch];
        w2 = conv[2 * kSsmC + ch];
        dtb_g = a.dt_bias[kh + kSsmKHeads * ab_h];
        a_g = a.a[kh + kSsmKHeads * ab_h];
    };
    auto conv_done = [&] {
        conv[ch] = w0;
        conv[kSsmC + ch] = w1;
        conv[2 * kSsmC + ch] = w2;
    };

    // Requests: conv inputs, alpha and beta of a stream position; z values
    // of a position.  Each is issued unconditionally (positions and token
    // indices clamped) and marked used (use_x, use_z) at a fixed point of a
    // later phase, so that the waits the compiler places there are the same
    // on every path and cover only requests at least a phase old.
    uint32_t xin[kDnChunk], alpha_n, braw_n, zv[kPairs][2];
    auto request_x = [&](int q) {
        const int item = item_at(q), kh = item % kSsmKHeads;
        const int tb = (max(min(q, n_pos - 1), 0) % nblk) * kDnChunk;
        const __amdgpu_buffer_rsrc_t prs = proj_rs(item / kSsmKHeads);
        const uint32_t ch_off = (uint32_t)dn_channel(u, kh) * kElt;
#pragma unroll
        for (int i = 0; i < kDnChunk; i++) xin[i] = load_raw_buf<BF16IN>(prs, ch_off, row_off(tb + i));
        const int tr = min(tb, last_tok);
        const uint32_t ro = row_off(tr);
        const uint32_t lt = (uint32_t)min(ab_t, last_tok - tr) * (uint32_t)kSsmProj * kElt;
        const int vh = kh + kSsmKHeads * ab_h;
        alpha_n = load_raw_buf<BF16IN>(prs, lt + (uint32_t)(kAlpha + vh) * kElt, ro);
        braw_n = load_raw_buf<BF16IN>(prs, lt + (uint32_t)(kBeta + vh) * kElt, ro);
    };
    auto use_x = [&] {
#pragma unroll
        for (int i = 0; i < kDnChunk; i++) asm volatile("" ::"v"(xin[i]));
        asm volatile("" ::"v"(alpha_n), "v"(braw_n));
    };
    auto request_z = [&](int q) {
        const int item = item_at(q), kh = item % kSsmKHeads;
        const int tb = (max(min(q, n_pos - 1), 0) % nblk) * kDnChunk;
        const __amdgpu_buffer_rsrc_t prs = proj_rs(item / kSsmKHeads);
#pragma unroll
        for (int k = 0; k < kPairs; k++) {
            const int p = hw + k * kDnHelpWaves;
            const int pt = p >> 1, pvh = kh + kSsmKHeads * (p & 1);
            const uint32_t ro = row_off(tb + pt), lo = (uint32_t)(kZ + pvh * kSsmDv + lane) * kElt;
            zv[k][0] = load_raw_buf<BF16IN>(prs, lo, ro);
            zv[k][1] = load_raw_buf<BF16IN>(prs, lo + 64 * kElt, ro);
        }
    };
    auto use_z = [&] {
#pragma unroll
        for (int k = 0; k < kPairs; k++) asm volatile("" ::"v"(zv[k][0]), "v"(zv[k][1]));
    };
    // conv1d + SiLU of stream position q into its rows (zero rows past the
    // end); log decay and beta (0 and 0 past the end) of its tokens
    auto conv_pass = [&](int q) {
        const int nb = min(kDnChunk, a.n_tok - (q % nblk) * kDnChunk);
        float(*x)[4 * 128 + 4] = xs[q % 3];
#pragma unroll
        for (int i = 0; i < kDnChunk; i++) {
            if (i < nb) {
                const float xv = raw_f<BF16IN>(xin[i]);
                float sum = w0 * cw.x;
                sum = fmaf(w1, cw.y, sum);
                sum = fmaf(w2, cw.z, sum);
                sum = fmaf(xv, cw.w, sum);
                x[i][u] = dn_silu<REF>(sum);
                w0 = w1;
                w1 = w2;
                w2 = xv;
            } else {
                x[i][u] = 0.f;
            }
        }
        if (hw == 3 && lane < 2 * kDnChunk) {
            float l_a = 0.f, be = 0.f;
            if (ab_t < nb) {
                const float biased = raw_f<BF16IN>(alpha_n) + dtb_g;
                const float ex = REF ? schraudolph_exp(biased) : dn_exp(biased);
                const float sp = biased > 20.0f ? biased : dn_log(1.0f + ex);
                l_a = sp * a_g;
                be = dn_beta<REF>(raw_f<BF16IN>(braw_n));
            }
            lg[q % 3][ab_h][ab_t] = l_a;
            bt[q % 3][ab_h][ab_t] = be;
        }
    };
    // q/k normalisation in place (helpers 4..7) of stream position q
    auto norm_pass = [&](int q) {
        const int nb = min(kDnChunk, a.n_tok - (q % nblk) * kDnChunk);
        if (hw >= 4 && g16 < nb) {
            float(*x)[4 * 128 + 4] = xs[q % 3];
            float qv[kDnCols], kv[kDnCols];
            dn_qk(x[g16], col0, a.eps, qv, kv);
#pragma unroll
            for (int j = 0; j < kDnCols; j += 4) {
                const int cc = col0 + (j ? kSsmDk / 2 : 0);
                *reinterpret_cast<float4*>(&x[g16][cc]) = make_float4(qv[j], qv[j + 1], qv[j + 2], qv[j + 3]);
                *reinterpret_cast<float4*>(&x[g16][128 + cc]) = make_float4(kv[j], kv[j + 1], kv[j + 2], kv[j + 3]);
            }
        }
    };
    // K K^T (helper 0), Q K^T (helper 1), natural token order; prefix sums of
    // the log decays, e^g and e^{g_C - g} (helper 2, lanes 0, 1) of block bb
    auto gram_pass = [&](int bb) {
        const int cur = bb % 3;
        if (hw < 2) {
            const float(*x)[4 * 128 + 4] = xs[cur];
            f32x4 acc = {};
            const float* kr = &x[c][128 + 32 * g];
            const float* ar = hw == 0 ? kr : &x[c][32 * g];
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const float4 k4 = *reinterpret_cast<const float4*>(kr + 4 * m);
                const float4 a4 = *reinterpret_cast<const float4*>(ar + 4 * m);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, k4.x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, k4.y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, k4.z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, k4.w, acc, 0, 0, 0);
            }
            float(*dst)[kDnChunk] = hw == 0 ? kk : qk;
#pragma unroll
            for (int r = 0; r < 4; r++) dst[4 * g + r][c] = acc[r];
        } else if (hw == 2 && lane < 2) {
            float run = 0.f;
            for (int i = 0; i < kDnChunk; i++) {
                run += lg[cur][lane][i];
                lg[cur][lane][i] = run;
                eg[cur][lane][i] = dn_exp(run);
            }
            for (int i = 0; i < kDnChunk; i++) fc[cur][lane][i] = dn_exp(run - lg[cur][lane][i]);
        }
    };
    // K and Q of position bb (normalised in place by norm_pass) as fp16
    // fragments for the state waves' phase A: helper 4 + ks takes 32-k step
    // ks, lane (row r, group g) the 8 k of that step's lane group g in row r
    // (sigma order)
    auto split_pass = [&](int bb) {
        const float(*x)[4 * 128 + 4] = xs[bb % 3];
        const int ks = hw - 4;
        const float* row = &x[dn_sigma(c)][32 * ks + 4 * g];
#pragma unroll
        for (int part = 0; part < 2; part++) {
            const float4 a0 = *reinterpret_cast<const float4*>(row + 128 * (1 - part));
            const float4 a1 = *reinterpret_cast<const float4*>(row + 128 * (1 - part) + 16);
            const float v8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            f16x8_t h, m;
            dn_split8(v8, 16384.f, h, m);
            kqf[part][ks][g][0][c] = __builtin_bit_cast(u32x4, h);
            kqf[part][ks][g][1][c] = __builtin_bit_cast(u32x4, m);
        }
    };
    // K^T of position bb as the state update's fp16 A fragments (scale 2^14):
    // fragment m (k rows 16 m .. +15) for lane (row c, group g) holds
    // K[4 r + g][16 m + c], r = 0..3, split into h and m (8 B each).  They go
    // to the Q columns of the block's own rows, which nothing reads after the
    // block's gram and split passes: fragment m in rows 2 m (lanes 0..31) and
    // 2 m + 1 (lanes 32..63).  Helpers 2..5 take fragments 2 (hw - 2) + 0, 1.
    auto kt_pass = [&](int bb) {
        float(*x)[4 * 128 + 4] = xs[bb % 3];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int m = 2 * (hw - 2) + i;
            const float kv[4] = {x[g][128 + 16 * m + c], x[4 + g][128 + 16 * m + c], x[8 + g][128 + 16 * m + c],
                                 x[12 + g][128 + 16 * m + c]};
            const float ks[4] = {16384.f, 16384.f, 16384.f, 16384.f};
            f16x4_t h, mm_;
            dn_split4(kv, ks, h, mm_);
            const u32x2 hw2 = __builtin_bit_cast(u32x2, h), mw2 = __builtin_bit_cast(u32x2, mm_);
            *(reinterpret_cast<u32x4*>(&x[2 * m + (lane >> 5)][0]) + (lane & 31)) = u32x4{hw2[0], hw2[1], mw2[0], mw2[1]};
        }
    };
    // gated RMSNorm of stream position q's (token, v-head) pairs, 128 dims
    // per wave; pairs past the end or of a position before the first are
    // computed on stale data and their stores discarded
    auto out_pass = [&](int q) {
        const int item = item_at(q), seq = item / kSsmKHeads, kh = item % kSsmKHeads;
        const int tok0 = (max(q, 0) % nblk) * kDnChunk;
        const int nb = min(kDnChunk, a.n_tok - tok0);
        const __amdgpu_buffer_rsrc_t ors = out_rs(seq);
#pragma unroll
        for (int k = 0; k < kPairs; k++) {
            const int p = hw + k * kDnHelpWaves;
            const int pt = p >> 1, pvl = p & 1, pvh = kh + kSsmKHeads * pvl;
            const float* o_row = os[q & 1][pt][pvl];
            const float o0 = o_row[lane], o1 = o_row[lane + 64];
            const float ss = wave_sum(fmaf(o0, o0, o1 * o1));
            const float rms = dn_rsqrt(ss / kSsmDv + a.eps);
            const bool ok = q >= 0 && p < 2 * nb;  // uniform
            const uint32_t ob = ((uint32_t)(tok0 + pt) * (kSsmVHeads * kSsmDv) + (uint32_t)pvh * kSsmDv) * osz;
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++) {
                const int d = lane + 64 * h2;
                const float y = o_row[d] * rms * (h2 ? nw1 : nw0) * dn_silu<REF>(raw_f<BF16IN>(zv[k][h2]));
                const uint32_t off = ok ? ob + (uint32_t)d * osz : kDrop;
                if constexpr (BF16OUT)
                    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f32_to_bf16_rne(y), ors, off, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), ors, off, 0, 0);
            }
        }
    };

    // Memory operations before the loop in the order of a loop iteration's
    // (conv inputs, output stores, z values), so that the waits hold on entry.
    request_x(0);
    out_pass(-4);
    request_z(-3);
    for (int bb = -2; bb < n_pos; bb++) {
        const int cur = bb < 0 ? 0 : bb % 3;
        // Phase A: L, T (helpers 0, 1) and M (helpers 2, 3) of position bb;
        // norms of position bb + 1
        if (bb >= 0) {
            if (hw < 2) {
                // L for v-head hw: strict lower, beta_t e^{g_t - g_s} k_t.k_s
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int idx = lane + 64 * e, ti = idx >> 4, si = idx & 15;
                    const float dg = dn_exp(lg[cur][hw][ti] - lg[cur][hw][si]);
                    lm[hw][ti][si] = si < ti ? bt[cur][hw][ti] * (dg * kk[ti][si]) : 0.f;
                }
                // T = (I + N)^-1 for the strictly lower N held in lm.  N is
                // nilpotent (N^16 = 0), so T = (I - N)(I + N^2)(I + N^4)(I + N^8)
                // exactly: six 16 x 16 products on MFMA through LDS (a wave's
                // LDS accesses complete in order).
                float(*n1)[kDnChunk] = lm[hw];
                float(*n2)[kDnChunk] = sc[hw][0];
                float(*n4)[kDnChunk] = sc[hw][1];
                float(*n8)[kDnChunk] = sc[hw][2];
                float(*xm)[kDnChunk] = sc[hw][0];  // N^2 is dead once X is formed
                f32x4 pr = dn_m16(n1, n1, g, c);
#pragma unroll
                for (int r = 0; r < 4; r++) n2[4 * g + r][c] = pr[r];
                pr = dn_m16(n2, n2, g, c);
#pragma unroll
                for (int r = 0; r < 4; r++) n4[4 * g + r][c] = pr[r];
                pr = dn_m16(n4, n4, g, c);
#pragma unroll
                for (int r = 0; r < 4; r++) n8[4 * g + r][c] = pr[r];
                pr = dn_m16(n1, n2, g, c);  // X = I - N + N^2 - N N^2
#pragma unroll
                for (int r = 0; r < 4; r++)
                    xm[4 * g + r][c] = ((4 * g + r == c) ? 1.f : 0.f) - n1[4 * g + r][c] + n2[4 * g + r][c] - pr[r];
                pr = dn_m16(xm, n4, g, c);  // X <- X + X N^4
#pragma unroll
                for (int r = 0; r < 4; r++) xm[4 * g + r][c] += pr[r];
                pr = dn_m16(xm, n8, g, c);  // T = X + X N^8
#pragma unroll
                for (int r = 0; r < 4; r++) n1[4 * g + r][c] = xm[4 * g + r][c] + pr[r];
            } else if (hw < 4) {
                // M: e^{g_t - g_s} Q K^T, s <= t, both v-heads
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int idx = (u - 128) + 128 * e, h = idx >> 8, ti = (idx >> 4) & 15, si = idx & 15;
                    const float dg = dn_exp(lg[cur][h][ti] - lg[cur][h][si]);
                    mm[h][ti][si] = si <= ti ? dg * qk[ti][si] : 0.f;
                }
            }
        }
        if (bb >= 0 && hw >= 2 && hw < 6) kt_pass(bb);
        if (bb + 1 >= 0 && bb + 1 < n_pos) norm_pass(bb + 1);
        lds_barrier();
        // Phase B: K K^T, Q K^T, prefix sums of position bb + 1; conv and
        // gates of position bb + 2 (switching items at a boundary); output
        // norm of position bb - 1
        if (bb + 1 >= 0 && bb + 1 < n_pos) {
            gram_pass(bb + 1);
            if (hw >= 4) split_pass(bb + 1);
        }
        use_x();
        if (bb + 2 < n_pos) {
            if ((bb + 2) % nblk == 0) {
                if (cv_item >= 0) conv_done();
                cv_item = item_at(bb + 2);
                conv_item(cv_item);
            }
            conv_pass(bb + 2);
        }
        request_x(bb + 3);
        use_z();
        out_pass(bb - 1);
        request_z(bb);
        lds_barrier();
    }
    use_z();
    out_pass(n_pos - 1);
    conv_done();
}

constexpr int kDnPf = 4;  // rows loaded ahead in the streaming kernel (2, 6 and 8 measured slower)

template <bool BF16IN, bool REF>
__global__ __launch_bounds__(kDnThreads) void deltanet_decode_kernel(DeltaNetArgs a) {
#pragma clang fp contract(off)
    __shared__ float conv_lds[4 * 128];
    __shared__ float o_lds[2][kSsmDv];
    const int b = blockIdx.x;
    const int s = b / kSsmKHeads;
    const int kh = b - s * kSsmKHeads;
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int vl = wave >> 2, wi = wave & 3;
    const int vh = kh + kSsmKHeads * vl;
    const int rg = lane >> 4, col0 = (lane & 15) * 4;
    const int rbase = wi * 32 + rg;

    uint8_t* slot = a.state + (size_t)a.slot[s] * a.state_bytes + a.layer_off;
    float* S = reinterpret_cast<float*>(slot) + (size_t)vh * kSsmDv * kSsmDk + col0;
    float* conv = reinterpret_cast<float*>(slot + a.rec_bytes);

    float4 buf[kDnPf][2];
#pragma unroll
    for (int p = 0; p < kDnPf; p++) {
        const float* src = S + (size_t)(rbase + 4 * p) * kSsmDk;
        buf[p][0] = nt_ld4(src);
        buf[p][1] = nt_ld4(src + kSsmDk / 2);
    }
    const int ch = dn_channel(t, kh);
    const size_t prow = (size_t)s * kSsmProj;
    constexpr size_t kZ = kSsmC, kAlpha = kSsmC + kSsmVHeads * kSsmDv, kBeta = kAlpha + kSsmVHeads;
    const int zd = wi * 32 + (lane & 31);
    const float x = load_f<BF16IN>(a.proj, prow + ch);
    const float z = load_f<BF16IN>(a.proj, prow + kZ + (size_t)vh * kSsmDv + zd);
    const float alpha = load_f<BF16IN>(a.proj, prow + kAlpha + vh);
    const float braw = load_f<BF16IN>(a.proj, prow + kBeta + vh);
    const float c0 = conv[ch], c1 = conv[kSsmC + ch], c2 = conv[2 * kSsmC + ch];
    float sum = c0 * a.conv_w[ch];
    sum = fmaf(c1, a.conv_w[kSsmC + ch], sum);
    sum = fmaf(c2, a.conv_w[2 * kSsmC + ch], sum);
    sum = fmaf(x, a.conv_w[3 * kSsmC + ch], sum);
    conv_lds[t] = dn_silu<REF>(sum);
    conv[ch] = c1;
    conv[kSsmC + ch] = c2;
    conv[2 * kSsmC + ch] = x;
    __syncthreads();

    float q[kDnCols], k[kDnCols], decay, beta;
    dn_qk(conv_lds, col0, a.eps, q, k);
    dn_gates<REF>(alpha, braw, a.dt_bias[vh], a.a[vh], decay, beta);
#pragma unroll
    for (int r = 0; r < kDnRows; r++) {
        float st[kDnCols] = {buf[r % kDnPf][0].x, buf[r % kDnPf][0].y, buf[r % kDnPf][0].z, buf[r % kDnPf][0].w,
                             buf[r % kDnPf][1].x, buf[r % kDnPf][1].y, buf[r % kDnPf][1].z, buf[r % kDnPf][1].w};
        if (r + kDnPf < kDnRows) {
            const float* src = S + (size_t)(rbase + 4 * (r + kDnPf)) * kSsmDk;
            buf[r % kDnPf][0] = nt_ld4(src);
            buf[r % kDnPf][1] = nt_ld4(src + kSsmDk / 2);
        }
        o_lds[vl][rbase + 4 * r] = dn_row(st, k, q, decay, beta, conv_lds[256 + vl * 128 + rbase + 4 * r]) * a.out_scale;
        float* dst = S + (size_t)(rbase + 4 * r) * kSsmDk;
        nt_st4(dst, st[0], st[1], st[2], st[3]);
        nt_st4(dst + kSsmDk / 2, st[4], st[5], st[6], st[7]);
    }
    __syncthreads();
    dn_norm_out<REF>(a, o_lds[vl], lane, wi, vh, (size_t)s * (kSsmVHeads * kSsmDv), z);
}

// ---------------------------------------------------------------------------
// Zero-fill of whole per-sequence state slots: a fresh or reset sequence's
// recurrent and conv state starts at zero, as reset_state() zero-fills it
// (src/engine.cpp:4164-4176).  Grid (pieces, slot), 16 B per thread per step.
__global__ __launch_bounds__(256) void zero_state_kernel(ZeroStateArgs a) {
    uint4* base = reinterpret_cast<uint4*>(a.state + (size_t)a.slot[blockIdx.y] * a.state_bytes);
    const size_t n = (size_t)a.state_bytes / 16;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        base[i] = make_uint4(0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Gather: work item = (sequence, 32 consecutive output tokens), split over 4
// workgroups = (K or V) x (16-token half); output rows are [tok][kv_head][d]
// packed back to back.  A workgroup moves 32 KiB: each thread 8 x 16 B, all
// loads issued before the stores.  The half's at most two block ids are read
// once per workgroup (scalar loads), so no table load precedes a data load.
// Pool reads are plain loads, output stores non-temporal: for config c's
// 16 x 8192 tokens x 8 layers, 8-token quarters with non-temporal loads ran
// 157 us, 16-token halves with plain loads run 127 us.
constexpr int kGatherTok = kBlockTok / kGatherQ;     // tokens per workgroup (kGatherQ per chunk and K|V)
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
    const int item = blockIdx.x / kGatherWgsPerItem;
    const int kv = (blockIdx.x / kGatherQ) & 1, q8 = blockIdx.x % kGatherQ;
    int s = 0;
    while (s + 1 < a.n_seqs && a.item_begin[s + 1] <= item) s++;
    const int c = item - a.item_begin[s];
    const int n_tok = a.out_begin[s + 1] - a.out_begin[s];
    const int t0 = c * kBlockTok + q8 * kGatherTok;
    const int nt = min(kGatherTok, n_tok - t0);
    if (nt <= 0) return;
    const int32_t* trow = a.table + (size_t)a.slot[s] * a.table_stride;
    const int p0 = a.tok0 + t0;
    const int blk_a = p0 / kBlockTok;
    const int id_a = trow[blk_a], id_b = trow[(p0 + nt - 1) / kBlockTok];
    const uint16_t* __restrict__ pool = kv ? a.vpool : a.kpool;
    uint16_t* __restrict__ outp = (kv ? a.v_out : a.k_out) + ((size_t)a.out_begin[s] + t0) * kKvHeads * kHeadDim;
    constexpr int kRowUnits = kHeadDim * 2 / 16;  // 32 x 16 B per (token, head) row
    constexpr int kPer = kGatherTok * kKvHeads * kRowUnits / 256;  // 16-B pieces per thread
    u32x4 buf[kPer];
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int u = j * 256 + (int)threadIdx.x;
        const int tok = u / (kKvHeads * kRowUnits);
        const int hh = (u / kRowUnits) % kKvHeads;
        const int part = u % kRowUnits;
        const int pos = p0 + min(tok, nt - 1);
        const int id = pos / kBlockTok == blk_a ? id_a : id_b;
        const size_t src = (((size_t)id * kKvHeads + hh) * kBlockTok + pos % kBlockTok) * kHeadDim + part * 8;
        buf[j] = *reinterpret_cast<const u32x4*>(pool + src);
    }
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int u = j * 256 + (int)threadIdx.x;
        if (u / (kKvHeads * kRowUnits) < nt)
            __builtin_nontemporal_store(buf[j], reinterpret_cast<u32x4*>(outp + (size_t)u * 8));
    }
}

// Snapshot save/restore: per pair, the sequence's whole recurrent state then
// the K/V segment of every attention layer (either part can be skipped).
// Each thread moves kSnapUnroll x 16 B (one piece per thread and many small
// workgroups stream best).
constexpr int kSnapUnroll = 1;
__device__ __forceinline__ int64_t snap_units_begin(const SnapshotArgs& a) {
    return a.do_state ? 0 : a.state_bytes / 16;
}
__device__ __forceinline__ int64_t snap_units_end(const SnapshotArgs& a) {
    const int64_t seg_bytes = (int64_t)a.n_layers * 2 * a.seg_blocks * (int64_t)kBlockBytes;
    return a.do_kv ? (a.state_bytes + seg_bytes) / 16 : a.state_bytes / 16;
}
// ---------------------------------------------------------------------------
// K/V checksums, one per (block, K|V, kv head) unit of 16 KiB: one 256-thread
// workgroup reads one unit, 4 x 16 B per thread, all loads issued before any
// is used, and folds its 32-bit words w_j (j = token * 128 + word of the
// 512-B head row) into two sums, sum(w_j) and sum(w_j ^ j); the second makes
// the checksum depend on where each word sits.  Slots past the sequence end
// are read (whole units stream best) but not summed.  No atomics and no
// exchange between workgroups: each writes its unit's 8 bytes.  A
// read-only kernel of exactly known size: the bench uses it as the
// single-launch read floor of a decode's K/V and for counter calibration.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t x) {
    x += __builtin_amdgcn_update_dpp(0u, x, kDppXor1, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, kDppXor2, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, kDppHalfMirror, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, kDppRowRor8, 0xF, 0xF, false);
    auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = r16[0] + r16[1];
    auto r32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return r32[0] + r32[1];
}

__global__ __launch_bounds__(256) void checksum_kernel(ChecksumArgs a) {
    __shared__ uint32_t red[4][2];
    const int u = blockIdx.x;
    int s = 0;
    while (s + 1 < a.n_seqs && a.unit_begin[s + 1] <= u) s++;
    const int lu = u - a.unit_begin[s];
    const int blk = lu >> 3, kv = (lu >> 2) & 1, hh = lu & 3;
    const int L = a.kv_len[s];
    const int32_t id = a.table[(size_t)a.slot[s] * a.table_stride + blk];
    const uint16_t* unit = (kv ? a.vpool : a.kpool) + ((size_t)id * kKvHeads + hh) * (kBlockTok * kHeadDim);
    const int t = threadIdx.x;
    u32x4 w[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(unit) + j * 256 + t);
    uint32_t lo = 0, hi = 0;
    const int n_valid = min(kBlockTok, L - blk * kBlockTok);  // tokens of this block in the sequence
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tok = j * 8 + (t >> 5);  // 32 x 16 B per token row
        if (tok < n_valid) {
            const uint32_t j0 = (uint32_t)(j * 256 + t) * 4;  // word index in the unit
#pragma unroll
            for (int k = 0; k < 4; k++) {
                lo += w[j][k];
                hi += w[j][k] ^ (j0 + k);
            }
        }
    }
    lo = wave_sum_u32(lo);
    hi = wave_sum_u32(hi);
    if ((t & 63) == 0) {
        red[t >> 6][0] = lo;
        red[t >> 6][1] = hi;
    }
    __syncthreads();
    if (t == 0) {
        uint2 r;
        r.x = red[0][0] + red[1][0] + red[2][0] + red[3][0];
        r.y = red[0][1] + red[1][1] + red[2][1] + red[3][1];
        reinterpret_cast<uint2*>(a.out)[u] = r;
    }
}

__global__ __launch_bounds__(256) void snapshot_kernel(SnapshotArgs a) {
    const int p = blockIdx.y;
    const int64_t u0 = snap_units_begin(a), u1 = snap_units_end(a);
    uint8_t* live = a.state_base + (int64_t)a.seq_slot[p] * a.state_bytes;
    uint8_t* snap = a.snap_base + (int64_t)a.snap_slot[p] * a.snap_bytes;
    const int32_t* trow = a.table + (size_t)a.seq_slot[p] * a.table_stride + a.first_block[p];
    const int64_t base = u0 + ((int64_t)blockIdx.x * blockDim.x * kSnapUnroll) + threadIdx.x;
    u32x4 buf[kSnapUnroll];
    uint8_t* dst[kSnapUnroll];
#pragma unroll
    for (int k = 0; k < kSnapUnroll; k++) {
        const int64_t u = base + (int64_t)k * blockDim.x;
        dst[k] = nullptr;
        if (u >= u1) continue;
        const int64_t off = u * 16;
        uint8_t* lp;
        if (off < a.state_bytes) {
            lp = live + off;
        } else {
            const int64_t so = off - a.state_bytes;
            const int64_t piece = so / (int64_t)kBlockBytes;
            const int64_t within = so - piece * (int64_t)kBlockBytes;
            const int layer = (int)(piece / (2 * a.seg_blocks));
            const int kv = (int)((piece / a.seg_blocks) & 1);
            const int bi = (int)(piece % a.seg_blocks);
            lp = a.pool_base + (int64_t)(layer * 2 + kv) * a.layer_kv_bytes +
                 (int64_t)trow[bi] * (int64_t)kBlockBytes + within;
        }
        uint8_t* sp = snap + off;
        const uint8_t* src = a.restore ? sp : lp;
        dst[k] = a.restore ? lp : sp;
        buf[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
    }
#pragma unroll
    for (int k = 0; k < kSnapUnroll; k++)
        if (dst[k]) __builtin_nontemporal_store(buf[k], reinterpret_cast<u32x4*>(dst[k]));
}

// Block copy (copy-on-write): blockIdx.y = pair; all layers, K and V.
__global__ __launch_bounds__(256) void block_copy_kernel(BlockCopyArgs a) {
    const int p = blockIdx.y;
    const int64_t units = (int64_t)a.n_layers * 2 * (int64_t)(kBlockBytes / 16);
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    constexpr int64_t kBlkUnits = kBlockBytes / 16;
    const int64_t lk = u / kBlkUnits;  // layer * 2 + kv
    const int64_t w = u - lk * kBlkUnits;
    const uint8_t* src = a.pool_base + lk * a.layer_kv_bytes + (int64_t)a.src[p] * (int64_t)kBlockBytes + w * 16;
    uint8_t* dst = a.pool_base + lk * a.layer_kv_bytes + (int64_t)a.dst[p] * (int64_t)kBlockBytes + w * 16;
    *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
}

// ---------------------------------------------------------------------------
// Synthetic N(0,1)*scale bf16: value 2j, 2j+1 from the j-th splitmix64 output
// of `seed` through Box-Muller (float math on the device; the host generator
// evaluates the same transform in double, so values can differ in the last
// bf16 bit -- tests never compare the two).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
__global__ __launch_bounds__(256) void fill_normal_kernel(uint16_t* dst, int64_t n, uint64_t seed,
                                                          float scale) {
    const int64_t pairs = (n + 1) / 2;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < pairs;
         j += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t draw = mix64(seed + (uint64_t)(j + 1) * 0x9E3779B97F4A7C15ULL);
        const float u1 = (float)((draw >> 40) + 1) * (1.0f / 16777216.0f);
        const float u2 = (float)((draw >> 16) & 0xFFFFFFULL) * (1.0f / 16777216.0f);
        const float rr = sqrtf(-2.0f * logf(u1));
        float sn, cs;
        sincosf(6.283185307179586f * u2, &sn, &cs);
        const uint32_t lo = f32_to_bf16_rne(rr * cs * scale);
        const uint32_t hi = f32_to_bf16_rne(rr * sn * scale);
        if (2 * j + 1 < n) {
            *reinterpret_cast<uint32_t*>(dst + 2 * j) = lo | (hi << 16);
        } else {
            dst[2 * j] = (uint16_t)lo;
        }
    }
}

// ---------------------------------------------------------------------------
int launch_table_update(const TableUpdateArgs& a, void* stream) {
    hipLaunchKernelGGL(table_update_kernel, dim3(1), dim3(512), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Static decode workspace for kvc_decode_attn_static: split-K partials of up
// to kStaticItems items, then the arrival counters.  Each GPU the library runs
// on holds its own copy until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol):
// the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) uint8_t scratch[kStaticPartBytes + kCounterBytes];

__global__ __launch_bounds__(256) void zero_words_kernel(int32_t* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

namespace {
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int static_scratch(int device, float** part, int32_t** counters) {
    if (device < 0 || device >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        // the counters must start at zero (the kernels reset them after use);
        // a fill kernel, not a memset, in case a caller captures later work
        int32_t* ctr = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(ptr) + kStaticPartBytes);
        const int n = (int)(kCounterBytes / 4);
        hipLaunchKernelGGL(zero_words_kernel, dim3((n + 255) / 256), dim3(256), 0, nullptr, ctr, n);
        if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(nullptr)) != hipSuccess) return (int)e;
        g_scratch_ptr[device] = static_cast<uint8_t*>(ptr);
    }
    *part = reinterpret_cast<float*>(g_scratch_ptr[device]);
    *counters = reinterpret_cast<int32_t*>(g_scratch_ptr[device] + kStaticPartBytes);
    return (int)hipSuccess;
}

int launch_decode(const DecodeArgs& a, void* stream) {
    const int grid = a.per_xcd * 8;
    const hipStream_t st = (hipStream_t)stream;
    if (a.qkv && a.qkv_f32) {
        if (a.d_parts == 2)
            hipLaunchKernelGGL((decode_kernel<2, 2>), dim3(grid), dim3(kWaves * 64), 0, st, a);
        else
            hipLaunchKernelGGL((decode_kernel<1, 2>), dim3(grid), dim3(kWaves * 64), 0, st, a);
    } else if (a.qkv) {
        if (a.d_parts == 2)
            hipLaunchKernelGGL((decode_kernel<2, 1>), dim3(grid), dim3(kWaves * 64), 0, st, a);
        else
            hipLaunchKernelGGL((decode_kernel<1, 1>), dim3(grid), dim3(kWaves * 64), 0, st, a);
    } else if (a.d_parts == 2) {
        hipLaunchKernelGGL((decode_kernel<2, 0>), dim3(grid), dim3(kWaves * 64), 0, st, a);
    } else {
        hipLaunchKernelGGL((decode_kernel<1, 0>), dim3(grid), dim3(kWaves * 64), 0, st, a);
    }
    return (int)hipGetLastError();
}

#ifdef KVC_PHASE_STAMPS
// Device address and shape of the decode phase stamps (this build only).
extern "C" __attribute__((visibility("default"))) int kvc_phase_stamps(void** buf, int32_t* wgs, int32_t* waves,
                                                                     int32_t* points) {
    if (!buf || !wgs || !waves || !points) return (int)hipErrorInvalidValue;
    *wgs = kStampWgs;
    *waves = kWaves;
    *points = kStampPoints;
    return (int)hipGetSymbolAddress(buf, HIP_SYMBOL(phase_stamps));
}
#endif

int launch_checksum(const ChecksumArgs& a, void* stream) {
    hipLaunchKernelGGL(checksum_kernel, dim3((unsigned)a.n_units), dim3(256), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_prefill(const PrefillArgs& a, void* stream) {
    const int grid = 8 * ((a.n_groups + 7) / 8) * ((a.n_q + kPfRows - 1) / kPfRows);
    const hipStream_t st = (hipStream_t)stream;
    if (a.qkv && a.qkv_f32)
        hipLaunchKernelGGL((prefill_mfma_kernel<kPfNT, 2>), dim3(grid), dim3(64 * 8 / kPfNT), 0, st, a);
    else if (a.qkv)
        hipLaunchKernelGGL((prefill_mfma_kernel<kPfNT, 1>), dim3(grid), dim3(64 * 8 / kPfNT), 0, st, a);
    else
        hipLaunchKernelGGL((prefill_mfma_kernel<kPfNT, 0>), dim3(grid), dim3(64 * 8 / kPfNT), 0, st, a);
    return (int)hipGetLastError();
}

int launch_append(const AppendArgs& a, void* stream) {
    static_assert(2 * kKvHeads * kHeadDim * 2 / 16 == 256, "one 16-B piece of each token per thread of a 256-thread workgroup");
    hipLaunchKernelGGL(append_kernel, dim3(a.n_seqs * ((a.n_tok + kAppendTok - 1) / kAppendTok)), dim3(256), 0,
                       (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_qkv_append(const QkvArgs& a, void* stream) {
    static_assert(kQkvWaves * 4 == kQHeads + kKvHeads, "two pairs of head rows per wave");
    if (!a.q_out && !a.gate_out) {  // k / v rows only: one token per wave
        const dim3 grid(a.n_seqs * ((a.n_tok + kQkvKvWaves - 1) / kQkvKvWaves)), block(kQkvKvWaves * 64);
        if (a.in_bf16)
            hipLaunchKernelGGL((qkv_append_kernel<true, true>), grid, block, 0, (hipStream_t)stream, a);
        else
            hipLaunchKernelGGL((qkv_append_kernel<false, true>), grid, block, 0, (hipStream_t)stream, a);
        return (int)hipGetLastError();
    }
    const dim3 grid(a.n_seqs * ((a.n_tok + kQkvTok - 1) / kQkvTok)), block(kQkvWaves * 64);
    if (a.in_bf16)
        hipLaunchKernelGGL((qkv_append_kernel<true, false>), grid, block, 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL((qkv_append_kernel<false, false>), grid, block, 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

template <bool REF>
static void launch_deltanet_t(const DeltaNetArgs& a, hipStream_t stream) {
    const dim3 grid(a.n_seqs * kSsmKHeads), block(kDnThreads);
    if (a.n_tok == 1) {
        if (a.in_bf16)
            hipLaunchKernelGGL((deltanet_decode_kernel<true, REF>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((deltanet_decode_kernel<false, REF>), grid, block, 0, stream, a);
    } else if (a.n_tok >= kDnMatrixMin) {
        // persistent: at most one workgroup per CU (its LDS needs a CU); the
        // CU count of the current device is looked up once per process
        static std::atomic<int> cu_count{0};
        int n_cu = cu_count.load(std::memory_order_relaxed);
        if (n_cu <= 0) {
            int dev = 0, v = 0;
            n_cu = (hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
                       ? v
                       : 256;
            cu_count.store(n_cu, std::memory_order_relaxed);
        }
        const dim3 mgrid(std::min(a.n_seqs * kSsmKHeads, n_cu)), mblock(kDnMfmaThreads);
        if (a.in_bf16 && a.out_bf16)
            hipLaunchKernelGGL((deltanet_mfma_kernel<true, true, REF>), mgrid, mblock, 0, stream, a);
        else if (a.in_bf16)
            hipLaunchKernelGGL((deltanet_mfma_kernel<true, false, REF>), mgrid, mblock, 0, stream, a);
        else if (a.out_bf16)
            hipLaunchKernelGGL((deltanet_mfma_kernel<false, true, REF>), mgrid, mblock, 0, stream, a);
        else
            hipLaunchKernelGGL((deltanet_mfma_kernel<false, false, REF>), mgrid, mblock, 0, stream, a);
    } else if (a.n_tok > kDnBlk) {
        if (a.in_bf16)
            hipLaunchKernelGGL((deltanet_kernel<true, REF, true>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((deltanet_kernel<false, REF, true>), grid, block, 0, stream, a);
    } else if (a.in_bf16) {
        hipLaunchKernelGGL((deltanet_kernel<true, REF, false>), grid, block, 0, stream, a);
    } else {
        hipLaunchKernelGGL((deltanet_kernel<false, REF, false>), grid, block, 0, stream, a);
    }
}

int launch_deltanet(const DeltaNetArgs& a, void* stream) {
    static_assert(kSsmVHeads == 2 * kSsmKHeads && kSsmDk == 128 && kSsmDv == 128,
                  "one workgroup per k-head and its two v-heads, 4 columns per lane");
    if (a.ref_math)
        launch_deltanet_t<true>(a, (hipStream_t)stream);
    else
        launch_deltanet_t<false>(a, (hipStream_t)stream);
    return (int)hipGetLastError();
}

int launch_zero_state(const ZeroStateArgs& a, void* stream) {
    hipLaunchKernelGGL(zero_state_kernel, dim3(512, a.n_slots), dim3(256), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_gather(const GatherArgs& a, void* stream) {
    if (a.n_items <= 0) return 0;
    hipLaunchKernelGGL(gather_kernel, dim3((unsigned)a.n_items * kGatherWgsPerItem), dim3(256), 0, (hipStream_t)stream,
                       a);
    return (int)hipGetLastError();
}

int launch_snapshot(const SnapshotArgs& a, void* stream) {
    const int64_t seg_bytes = (int64_t)a.n_layers * 2 * a.seg_blocks * (int64_t)kBlockBytes;
    const int64_t u0 = a.do_state ? 0 : a.state_bytes / 16;
    const int64_t u1 = a.do_kv ? (a.state_bytes + seg_bytes) / 16 : a.state_bytes / 16;
    const int64_t per_wg = 256 * kSnapUnroll;
    if (u1 <= u0 || a.n_pairs <= 0) return 0;
    hipLaunchKernelGGL(snapshot_kernel, dim3((unsigned)((u1 - u0 + per_wg - 1) / per_wg), a.n_pairs),
                       dim3(256), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_block_copy(const BlockCopyArgs& a, void* stream) {
    const int64_t units = (int64_t)a.n_layers * 2 * (int64_t)(kBlockBytes / 16);
    if (a.n <= 0) return 0;
    hipLaunchKernelGGL(block_copy_kernel, dim3((unsigned)((units + 255) / 256), a.n), dim3(256), 0,
                       (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_fill_normal(uint16_t* dst, int64_t n, uint64_t seed, float scale, void* stream) {
    const int64_t pairs = (n + 1) / 2;
    int64_t grid = (pairs + 255) / 256;
    if (grid > 65536) grid = 65536;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       dst, n, seed, scale);
    return (int)hipGetLastError();
}

}  // namespace kvc
