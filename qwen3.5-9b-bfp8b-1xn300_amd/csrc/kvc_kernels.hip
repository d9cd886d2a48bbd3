// kvc_kernels.hip -- gfx950 kernels of the KV-cache path: block-table update,
// append, split-K GQA decode attention (with fused append), causal prefill
// attention, gather, snapshot copy, synthetic fill.
//
// All K/V traffic is bf16; arithmetic is fp32 (v_dot2_f32_bf16 for q.k).
// Softmax runs in the log2 domain: s2 = (q.k) * scale * log2(e), p = 2^(s2-m).
#include "kvc_device.h"
#include "kvc_internal.h"

namespace kvc {

constexpr int kWaves = 4;           // waves per decode workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kTokPerWave = kBlockTok / kWaves;  // 8 tokens of a block per wave
constexpr float kNegBig = -1.0e30f;
constexpr float kRescaleSlack = 8.0f;  // lazy rescale: p may reach 2^8

// ---------------------------------------------------------------------------
// Block-table update: entries ride in the argument block.
__global__ void table_update_kernel(TableUpdateArgs a) {
    for (int i = threadIdx.x; i < a.n; i += blockDim.x) a.table[a.index[i]] = a.block[i];
}

// ---------------------------------------------------------------------------
// Per-wave online-softmax state.  m/l are wave-uniform; acc[g][j] holds
// output dims d = lane*4 + j of q head g of the group.
struct WaveState {
    float m[kGroup];
    float l[kGroup];
    float acc[kGroup][4];
};

// One block's K/V as held by one wave.
//   k[i]: token 2i + half of the wave's 8 tokens, dims seg*8 .. seg*8+7 (16 B)
//   v[j]: token j of the wave's 8 tokens, dims lane*4 .. lane*4+3 (8 B)
struct BlockRegs {
    uint4 k[4];
    uint2 v[kTokPerWave];
};

__device__ __forceinline__ void init_state(WaveState& st) {
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        st.m[g] = kNegBig;
        st.l[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) st.acc[g][j] = 0.f;
    }
}

// Load the wave's share of one (block, kv_head) unit.  Tokens >= n_valid read
// as zero.  The token at slot new_slot (if >= 0) comes from knew/vnew (one
// token row of this kv head) and is also written into the pool unit.
__device__ __forceinline__ void load_block(BlockRegs& r, const uint16_t* __restrict__ ku,
                                           const uint16_t* __restrict__ vu, int n_valid,
                                           int new_slot, const uint16_t* knew,
                                           const uint16_t* vnew, int wave, int lane) {
    const int half = lane >> 5, seg = lane & 31;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = wave * kTokPerWave + 2 * i + half;
        uint4 x = make_uint4(0, 0, 0, 0);
        if (t == new_slot) {
            x = *reinterpret_cast<const uint4*>(knew + seg * 8);
            *reinterpret_cast<uint4*>(const_cast<uint16_t*>(ku) + t * kHeadDim + seg * 8) = x;
        } else if (t < n_valid) {
            { const u32x4 y = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ku + t * kHeadDim + seg * 8)); x = make_uint4(y[0], y[1], y[2], y[3]); }
        }
        r.k[i] = x;
    }
#pragma unroll
    for (int j = 0; j < kTokPerWave; j++) {
        const int t = wave * kTokPerWave + j;
        uint2 x = make_uint2(0, 0);
        if (t == new_slot) {
            x = *reinterpret_cast<const uint2*>(vnew + lane * 4);
            *reinterpret_cast<uint2*>(const_cast<uint16_t*>(vu) + t * kHeadDim + lane * 4) = x;
        } else if (t < n_valid) {
            { const u32x2 y = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(vu + t * kHeadDim + lane * 4)); x = make_uint2(y[0], y[1]); }
        }
        r.v[j] = x;
    }
}

// Scores, online softmax update and P.V for one block held in registers.
// qv[g][c]: packed bf16 pairs of q head g, dims seg*8 + 2c, +1.
__device__ __forceinline__ void compute_block(const BlockRegs& r, const uint32_t (&qv)[kGroup][4],
                                              int n_valid, float scale_log2, float* lds_p,
                                              WaveState& st, int wave, int lane) {
    const int half = lane >> 5, seg = lane & 31;
    // partial q.k over this lane's 8 dims for 4 tokens x 4 heads
    float a[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int g = 0; g < kGroup; g++) {
            float s = dot2_bf16(qv[g][0], r.k[i].x, 0.f);
            s = dot2_bf16(qv[g][1], r.k[i].y, s);
            s = dot2_bf16(qv[g][2], r.k[i].z, s);
            s = dot2_bf16(qv[g][3], r.k[i].w, s);
            a[i * 4 + g] = s;
        }
    }
    // transpose-reduce over the 32 lanes of a half: after the steps over seg
    // bits 4..1, a[0] holds value index (seg >> 1) summed over 16 lanes.
#define KVC_TR_STEP(BIT, N)                                                  \
    {                                                                        \
        const bool sel = (seg >> BIT) & 1;                                   \
        _Pragma("unroll") for (int j = 0; j < N / 2; j++) {                  \
            float send = sel ? a[j] : a[j + N / 2];                          \
            float keep = sel ? a[j + N / 2] : a[j];                          \
            a[j] = keep + shfl_xor<(1 << BIT)>(send);                        \
        }                                                                    \
    }
    KVC_TR_STEP(4, 16)
    KVC_TR_STEP(3, 8)
    KVC_TR_STEP(2, 4)
    KVC_TR_STEP(1, 2)
#undef KVC_TR_STEP
    float sc = a[0] + shfl_xor<1>(a[0]);
    const int vi = seg >> 1;
    const int my_g = vi & 3;
    const int t_loc = 2 * (vi >> 2) + half;  // token within the wave's 8
    const bool valid = wave * kTokPerWave + t_loc < n_valid;
    sc = valid ? sc * scale_log2 : kNegBig;

    // block max per head over the wave's 8 tokens
    float mx = sc;
    mx = fmaxf(mx, shfl_xor<8>(mx));
    mx = fmaxf(mx, shfl_xor<16>(mx));
    mx = fmaxf(mx, shfl_xor<32>(mx));
    float mref_own = 0.f;
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        const float mb = readlane(mx, g << 1);
        if (mb > st.m[g] + kRescaleSlack) {
            const float c = fast_exp2(st.m[g] - mb);
            st.l[g] *= c;
#pragma unroll
            for (int j = 0; j < 4; j++) st.acc[g][j] *= c;
            st.m[g] = mb;
        }
        mref_own = (my_g == g) ? st.m[g] : mref_own;
    }
    const float p = valid ? fast_exp2(sc - mref_own) : 0.f;
    float ps = p;
    ps += shfl_xor<8>(ps);
    ps += shfl_xor<16>(ps);
    ps += shfl_xor<32>(ps);
#pragma unroll
    for (int g = 0; g < kGroup; g++) st.l[g] += readlane(ps, g << 1);

    // broadcast p[token][g] through LDS (per-wave area of 32 floats)
    wave_lds_sync();
    if ((seg & 1) == 0) lds_p[t_loc * 4 + my_g] = p;
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < kTokPerWave; j++) {
        const float4 pj = *reinterpret_cast<const float4*>(lds_p + j * 4);
        const float v0 = bf16lo(r.v[j].x), v1 = bf16hi(r.v[j].x);
        const float v2 = bf16lo(r.v[j].y), v3 = bf16hi(r.v[j].y);
        const float pg[4] = {pj.x, pj.y, pj.z, pj.w};
#pragma unroll
        for (int g = 0; g < kGroup; g++) {
            st.acc[g][0] = fmaf(pg[g], v0, st.acc[g][0]);
            st.acc[g][1] = fmaf(pg[g], v1, st.acc[g][1]);
            st.acc[g][2] = fmaf(pg[g], v2, st.acc[g][2]);
            st.acc[g][3] = fmaf(pg[g], v3, st.acc[g][3]);
        }
    }
}

__device__ __forceinline__ void load_q(uint32_t (&qv)[kGroup][4], const uint16_t* qhead0, int seg) {
#pragma unroll
    for (int g = 0; g < kGroup; g++) {
        const uint4 x = *reinterpret_cast<const uint4*>(qhead0 + g * kHeadDim + seg * 8);
        qv[g][0] = x.x;
        qv[g][1] = x.y;
        qv[g][2] = x.z;
        qv[g][3] = x.w;
    }
}

// LDS for one workgroup: per-wave p broadcast + cross-wave merge area.
struct DecodeSmem {
    float p[kWaves][32];
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

__device__ __forceinline__ float sigmoidf_exact(float x) { return 1.0f / (1.0f + __expf(-x)); }

// out row = A / L (* sigmoid(gate)), written as bf16 (RNE) or fp32.
__device__ __forceinline__ void write_out(void* out, int out_bf16, size_t row_off, int d0,
                                          const uint16_t* gate_row, float L, const float (&A)[4]) {
    const float inv = 1.0f / L;
    float o[4] = {A[0] * inv, A[1] * inv, A[2] * inv, A[3] * inv};
    if (gate_row) {
        const uint2 gw = *reinterpret_cast<const uint2*>(gate_row + d0);
        o[0] *= sigmoidf_exact(bf16lo(gw.x));
        o[1] *= sigmoidf_exact(bf16hi(gw.x));
        o[2] *= sigmoidf_exact(bf16lo(gw.y));
        o[3] *= sigmoidf_exact(bf16hi(gw.y));
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

// ---------------------------------------------------------------------------
// Split-K GQA decode.  Work item = (kv head, chunk of chunk_blocks blocks of
// one sequence); items of one (seq, head) are consecutive and are spread over
// the 8 XCDs in contiguous runs (workgroup b runs on XCD b % 8).  Each item
// writes (m, l, acc) for its 4 q heads; the last item of a (seq, head) to
// arrive (device-scope counter) combines them and writes the output.
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeArgs a) {
    __shared__ DecodeSmem sm;
    const int b = blockIdx.x;
    const int item = (b & 7) * a.per_xcd + (b >> 3);
    if (item >= a.n_items) return;
    const int h = item / a.total_chunks;
    const int chunk = item - h * a.total_chunks;
    int s = 0;
    while (s + 1 < a.n_seqs && a.chunk_begin[s + 1] <= chunk) s++;
    const int c = chunk - a.chunk_begin[s];
    const int n_chunks = a.chunk_begin[s + 1] - a.chunk_begin[s];
    const int L = a.kv_len[s];
    const int n_blocks = (L + kBlockTok - 1) / kBlockTok;
    const int blk0 = c * a.chunk_blocks;
    const int blk1 = min(blk0 + a.chunk_blocks, n_blocks);
    const int slot = a.slot[s];
    const int* trow = a.table + (size_t)slot * a.table_stride;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, seg = lane & 31;
    const int new_pos = a.k_new ? L - 1 : -1;
    const uint16_t* knew = a.k_new ? a.k_new + ((size_t)s * kKvHeads + h) * kHeadDim : nullptr;
    const uint16_t* vnew = a.v_new ? a.v_new + ((size_t)s * kKvHeads + h) * kHeadDim : nullptr;

    uint32_t qv[kGroup][4];
    load_q(qv, a.q + ((size_t)s * kQHeads + h * kGroup) * kHeadDim, seg);

    WaveState st;
    init_state(st);
    BlockRegs r0, r1;
    auto unit = [&](const uint16_t* pool, int blk) {
        return pool + ((size_t)trow[blk] * kKvHeads + h) * (kBlockTok * kHeadDim);
    };
    auto nvalid = [&](int blk) { return min(kBlockTok, L - blk * kBlockTok); };
    auto nslot = [&](int blk) {
        const int d = new_pos - blk * kBlockTok;
        return (d >= 0 && d < kBlockTok) ? d : -1;
    };
    load_block(r0, unit(a.kpool, blk0), unit(a.vpool, blk0), nvalid(blk0), nslot(blk0), knew, vnew,
               wave, lane);
    for (int blk = blk0; blk < blk1; blk += 2) {
        if (blk + 1 < blk1)
            load_block(r1, unit(a.kpool, blk + 1), unit(a.vpool, blk + 1), nvalid(blk + 1),
                       nslot(blk + 1), knew, vnew, wave, lane);
        compute_block(r0, qv, nvalid(blk), a.scale_log2, sm.p[wave], st, wave, lane);
        if (blk + 1 >= blk1) break;
        if (blk + 2 < blk1)
            load_block(r0, unit(a.kpool, blk + 2), unit(a.vpool, blk + 2), nvalid(blk + 2),
                       nslot(blk + 2), knew, vnew, wave, lane);
        compute_block(r1, qv, nvalid(blk + 1), a.scale_log2, sm.p[wave], st, wave, lane);
    }

    float M, Lsum, A[4];
    merge_waves(st, sm, wave, lane, M, Lsum, A);
    const int t = threadIdx.x, g = t >> 6, d0 = (t & 63) * 4;
    const size_t orow = ((size_t)s * kQHeads + h * kGroup + g) * kHeadDim;
    const uint16_t* grow = a.gate ? a.gate + orow : nullptr;
    if (n_chunks == 1) {
        write_out(a.out, a.out_bf16, orow, d0, grow, Lsum, A);
        return;
    }
    constexpr int kItemFloats = kGroup * kHeadDim + 2 * kGroup;
    float* part = a.part + (size_t)item * kItemFloats;
    *reinterpret_cast<float4*>(part + g * kHeadDim + d0) = make_float4(A[0], A[1], A[2], A[3]);
    if ((t & 63) == 0) {
        part[kGroup * kHeadDim + 2 * g] = M;
        part[kGroup * kHeadDim + 2 * g + 1] = Lsum;
    }
    __threadfence();
    __syncthreads();
    if (t == 0) {
        const int prev = atomicAdd(&a.counters[s * kKvHeads + h], 1);
        sm.last = (prev == n_chunks - 1);
    }
    __syncthreads();
    if (!sm.last) return;
    __threadfence();
    // combine the n_chunks partials of (s, h)
    const size_t first = (size_t)h * a.total_chunks + a.chunk_begin[s];
    float Mc = kNegBig, Lc = 0.f, Ac[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < n_chunks; k++) {
        const float* pk = a.part + (first + k) * kItemFloats;
        const float mk = pk[kGroup * kHeadDim + 2 * g];
        const float lk = pk[kGroup * kHeadDim + 2 * g + 1];
        const f32x4 ak = *reinterpret_cast<const f32x4*>(pk + g * kHeadDim + d0);
        if (mk > Mc) {
            const float cc = fast_exp2(Mc - mk);
            Lc *= cc;
            Ac[0] *= cc; Ac[1] *= cc; Ac[2] *= cc; Ac[3] *= cc;
            Mc = mk;
        }
        const float w = fast_exp2(mk - Mc);
        Lc = fmaf(w, lk, Lc);
        Ac[0] = fmaf(w, ak[0], Ac[0]);
        Ac[1] = fmaf(w, ak[1], Ac[1]);
        Ac[2] = fmaf(w, ak[2], Ac[2]);
        Ac[3] = fmaf(w, ak[3], Ac[3]);
    }
    write_out(a.out, a.out_bf16, orow, d0, grow, Lc, Ac);
    if (t == 0) a.counters[s * kKvHeads + h] = 0;
}

// ---------------------------------------------------------------------------
// Causal prefill, one workgroup per (seq, query row, kv head); row r of seq s
// sits at position q_pos0[s] + r and reads keys [0, pos].
__global__ __launch_bounds__(kThreads) void prefill_rowwise_kernel(PrefillArgs a) {
    __shared__ DecodeSmem sm;
    const int h = blockIdx.x % kKvHeads;
    const int row = (blockIdx.x / kKvHeads) % a.n_q;
    const int s = blockIdx.x / (kKvHeads * a.n_q);
    const int L = a.q_pos0[s] + row + 1;
    const int n_blocks = (L + kBlockTok - 1) / kBlockTok;
    const int* trow = a.table + (size_t)a.slot[s] * a.table_stride;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, seg = lane & 31;
    const size_t qrow = (((size_t)s * a.n_q + row) * kQHeads + h * kGroup) * kHeadDim;

    uint32_t qv[kGroup][4];
    load_q(qv, a.q + qrow, seg);
    WaveState st;
    init_state(st);
    BlockRegs r0;
    for (int blk = 0; blk < n_blocks; blk++) {
        const size_t uoff = ((size_t)trow[blk] * kKvHeads + h) * (kBlockTok * kHeadDim);
        const int nv = min(kBlockTok, L - blk * kBlockTok);
        load_block(r0, a.kpool + uoff, a.vpool + uoff, nv, -1, nullptr, nullptr, wave, lane);
        compute_block(r0, qv, nv, a.scale_log2, sm.p[wave], st, wave, lane);
    }
    float M, Lsum, A[4];
    merge_waves(st, sm, wave, lane, M, Lsum, A);
    const int t = threadIdx.x, g = t >> 6, d0 = (t & 63) * 4;
    const size_t orow = qrow + (size_t)g * kHeadDim;
    write_out(a.out, a.out_bf16, orow, d0, a.gate ? a.gate + orow : nullptr, Lsum, A);
}

// ---------------------------------------------------------------------------
// Append: one thread per 16 bytes of a (token, kv head) row of K or V.
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a, int n_units) {
    const int u = blockIdx.x * blockDim.x + threadIdx.x;  // 16-B unit
    if (u >= n_units) return;
    constexpr int kRowUnits = kHeadDim * 2 / 16;  // 32
    const int part = u % kRowUnits;
    const int row = u / kRowUnits;  // over [kv][seq][tok][head]
    const int rows_per_kv = a.n_seqs * a.n_tok * kKvHeads;
    const int kv = row / rows_per_kv;
    const int r = row - kv * rows_per_kv;
    const int h = r % kKvHeads;
    const int tok = (r / kKvHeads) % a.n_tok;
    const int s = r / (kKvHeads * a.n_tok);
    const int pos = a.pos0[s] + tok;
    const int blk = a.table[(size_t)a.slot[s] * a.table_stride + pos / kBlockTok];
    const size_t dst = (((size_t)blk * kKvHeads + h) * kBlockTok + pos % kBlockTok) * kHeadDim + part * 8;
    const size_t src = (size_t)r * kHeadDim + part * 8;
    const uint16_t* from = kv ? a.v : a.k;
    uint16_t* to = kv ? a.vpool : a.kpool;
    *reinterpret_cast<uint4*>(to + dst) = *reinterpret_cast<const uint4*>(from + src);
}

// Gather: packed output rows [tok][head][d]; one thread per 16 B of K or V.
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    constexpr int kRowUnits = kHeadDim * 2 / 16;
    const int64_t rows = (int64_t)a.total_tok * kKvHeads;
    if (u >= 2 * rows * kRowUnits) return;
    const int part = (int)(u % kRowUnits);
    const int64_t row = u / kRowUnits;
    const int kv = row >= rows;
    const int64_t r = row - (kv ? rows : 0);
    const int h = (int)(r % kKvHeads);
    const int otok = (int)(r / kKvHeads);
    int s = 0;
    while (s + 1 < a.n_seqs && a.out_begin[s + 1] <= otok) s++;
    const int pos = a.tok0 + otok - a.out_begin[s];
    const int blk = a.table[(size_t)a.slot[s] * a.table_stride + pos / kBlockTok];
    const size_t src = (((size_t)blk * kKvHeads + h) * kBlockTok + pos % kBlockTok) * kHeadDim + part * 8;
    const uint16_t* from = kv ? a.vpool : a.kpool;
    uint16_t* to = kv ? a.v_out : a.k_out;
    *reinterpret_cast<u32x4*>(to + r * kHeadDim + part * 8) =
        __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(from + src));
}

// Snapshot save/restore: per pair, the sequence's whole recurrent state then
// the K/V segment of every attention layer (either part can be skipped).
// Each thread moves kSnapUnroll x 16 B.
constexpr int kSnapUnroll = 4;
__device__ __forceinline__ int64_t snap_units_begin(const SnapshotArgs& a) {
    return a.do_state ? 0 : a.state_bytes / 16;
}
__device__ __forceinline__ int64_t snap_units_end(const SnapshotArgs& a) {
    const int64_t seg_bytes = (int64_t)a.n_layers * 2 * a.seg_blocks * (int64_t)kBlockBytes;
    return a.do_kv ? (a.state_bytes + seg_bytes) / 16 : a.state_bytes / 16;
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

int launch_decode(const DecodeArgs& a, void* stream) {
    const int grid = a.per_xcd * 8;
    hipLaunchKernelGGL(decode_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_prefill(const PrefillArgs& a, void* stream) {
    const int grid = a.n_seqs * a.n_q * kKvHeads;
    hipLaunchKernelGGL(prefill_rowwise_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

int launch_append(const AppendArgs& a, int n_units, void* stream) {
    hipLaunchKernelGGL(append_kernel, dim3((n_units + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       a, n_units);
    return (int)hipGetLastError();
}

int launch_gather(const GatherArgs& a, void* stream) {
    const int64_t units = (int64_t)a.total_tok * kKvHeads * 2 * (kHeadDim * 2 / 16);
    hipLaunchKernelGGL(gather_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, a);
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
