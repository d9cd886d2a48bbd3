// kvc_calib.hip -- measurement aid for bench.py, not part of the libkvc ABI.
//
// The bf16 MFMA rate of an MI355X depends on the operand data: with constant
// operands an MFMA-only loop of v_mfma_f32_32x32x16_bf16 runs near the
// published dense peak, with random bf16 operands of the prefill's
// distributions it runs at roughly 60% of it (the card holds its power by
// lowering the clock).  kvc_calib_mfma_bf16 times that loop for one operand
// distribution, so the prefill's MFMA throughput can be set against the rate
// the same data allows:
//   mode 0  every operand 1.0
//   mode 1  A and B ~ N(0, 1) in bf16 (the S = K Q^T product)
//   mode 2  A ~ N(0, 1), B uniform in [0, 1) (the O += V^T P^T product)
//
// kvc_calib_read_floor times a read-only launch of config b's size (16 MiB:
// the K and V of 128 blocks of 64 KiB, four 16-KiB (block, kv head) units
// each) in config b's graph and replica rotation, for one launch shape: the
// number of workgroups (1, 2 or 4 per CU), 16-B loads in flight per lane,
// and whether a workgroup reads contiguous bytes (a whole 64-KiB block at
// one workgroup per CU) or 16-KiB units spread over the launch.  bench.py
// sweeps the shapes; the fastest is the single-launch read floor that the
// decode launch is set against.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kSteps = 32;   // MFMAs per repetition, over 8 accumulators
constexpr int kFrags = 4;    // A and B operand fragments per lane (two rings)

__device__ uint32_t mix(uint32_t x) {  // 32-bit integer hash (xorshift-multiply)
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}
__device__ float uniform01(uint32_t h) { return (h >> 8) * (1.0f / 16777216.0f); }
// approximately N(0, 1): sum of 4 uniforms, centred and scaled to unit variance
__device__ float normalish(uint32_t seed) {
    float s = 0.f;
    for (int i = 0; i < 4; i++) s += uniform01(mix(seed * 4u + (uint32_t)i));
    return (s - 2.0f) * 1.7320508f;
}
__device__ uint32_t pack_bf16(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 4 waves per workgroup; the operand rings (32 registers) and the 8
// accumulators (128) leave room for 2 or more waves per SIMD
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mfma_rate_kernel(int mode, int reps,
                                                                                               float* sink) {
    const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
    bf16x8_t a[kFrags], b[kFrags];
    for (int f = 0; f < kFrags; f++) {
        u32x4_t wa, wb;
        for (int j = 0; j < 4; j++) {
            const uint32_t s = (tid * kFrags + (uint32_t)f) * 8u + 2u * (uint32_t)j;
            float a0 = 1.f, a1 = 1.f, b0 = 1.f, b1 = 1.f;
            if (mode != 0) {
                a0 = normalish(2u * s);
                a1 = normalish(2u * s + 2u);
                b0 = mode == 1 ? normalish(2u * s + 1u) : uniform01(mix(2u * s + 1u));
                b1 = mode == 1 ? normalish(2u * s + 3u) : uniform01(mix(2u * s + 3u));
            }
            wa[j] = pack_bf16(a0, a1);
            wb[j] = pack_bf16(b0, b1);
        }
        asm volatile("" : "+v"(wa), "+v"(wb));  // built one fragment at a time
        a[f] = __builtin_bit_cast(bf16x8_t, wa);
        b[f] = __builtin_bit_cast(bf16x8_t, wb);
    }
    f32x16_t acc[8];
    for (int d = 0; d < 8; d++) acc[d] = f32x16_t{};
    for (int r = 0; r < reps; r++) {
#pragma unroll
        for (int i = 0; i < kSteps; i++)
            acc[i & 7] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i & 3], b[(i + 1) & 3], acc[i & 7], 0, 0, 0);
    }
    float s = 0.f;
    for (int d = 0; d < 8; d++) s += acc[d][0] + acc[d][15];
    sink[tid] = s;
}

// ---- read floor ------------------------------------------------------------
constexpr int kFloorLayers = 8, kFloorReps = 4, kFloorSeqBlocks = 128;
constexpr int kFloorPoolBlocks = kFloorReps * (kFloorSeqBlocks + 2);  // as bench.py sizes config b's pool
constexpr size_t kPieceBytes = 65536;                                 // one block of one layer's K (or V)
constexpr size_t kRegionBytes = (size_t)kFloorPoolBlocks * kPieceBytes;
constexpr size_t kLaunchBytes = (size_t)2 * kFloorSeqBlocks * kPieceBytes;  // 16 MiB

// One launch reads pieces p = 0..255 (block p / 2, K for even p and V for odd
// p) of layer `layer`: K region 2 layer, V region 2 layer + 1, at the block
// ids of the replica.  A workgroup reads `per_wg` bytes of that 16 MiB in
// rounds of LOADS 16-B loads per lane (1 KiB per wave and load); STRIDED
// workgroups read 16-KiB units u = w, w + grid, ... instead of one
// contiguous range.
template <int LOADS, bool STRIDED, bool NT>
__global__ __launch_bounds__(256) void floor_read_kernel(const uint8_t* __restrict__ pool,
                                                         const int32_t* __restrict__ ids, int layer, int per_wg,
                                                         uint32_t* __restrict__ sink) {
    const int w = blockIdx.x, t = threadIdx.x;
    const int rounds = per_wg / (4096 * LOADS);
    u32x4_t x = {0u, 0u, 0u, 0u};
    for (int r = 0; r < rounds; r++) {
        u32x4_t v[LOADS];
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            // byte of the launch's logical 16 MiB stream
            size_t o;
            if constexpr (STRIDED) {
                static_assert(16384 % (4096 * LOADS) == 0, "a strided round stays inside one 16-KiB unit");
                constexpr int unit_bytes = 16384, per_unit = unit_bytes / (4096 * LOADS);
                const int u = w + gridDim.x * (r / per_unit);
                o = (size_t)u * unit_bytes + (size_t)(r % per_unit) * 4096 * LOADS;
            } else {
                o = (size_t)w * per_wg + (size_t)r * 4096 * LOADS;
            }
            o += (size_t)i * 4096 + (size_t)t * 16;
            const int p = (int)(o / kPieceBytes);
            const uint8_t* src = pool + (size_t)(2 * layer + (p & 1)) * kRegionBytes +
                                 (size_t)ids[p >> 1] * kPieceBytes + (o % kPieceBytes);
            if (NT)
                v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src));
            else
                v[i] = *reinterpret_cast<const u32x4_t*>(src);
        }
#pragma unroll
        for (int i = 0; i < LOADS; i++) x ^= v[i];
    }
    const uint32_t y = x[0] ^ x[1] ^ x[2] ^ x[3];
    if (y == 0x9e3779b9u) sink[w * 256 + t] = y;  // keeps the loads; data never matches
}

using FloorKernel = void (*)(const uint8_t*, const int32_t*, int, int, uint32_t*);
template <int LOADS>
FloorKernel floor_kernel(bool strided, bool nt) {
    if constexpr (LOADS <= 4) {
        if (strided) return nt ? floor_read_kernel<LOADS, true, true> : floor_read_kernel<LOADS, true, false>;
    }
    return nt ? floor_read_kernel<LOADS, false, true> : floor_read_kernel<LOADS, false, false>;
}

}  // namespace

extern "C" {

// Time one read shape: `grid` workgroups of 256 threads (a multiple of 256
// dividing 4096), `loads` 16-B loads per lane and round (2, 4, 8 or 16),
// strided (16-KiB units spread over the launch) or contiguous ranges, plain
// or non-temporal loads.  A HIP graph holds config b's 32 launches (4 replicas
// x 8 layers, 16 MiB each, 512 MiB in all, blocks drawn from a seeded
// permutation of the pool as bench.py's allocator seed does); it is replayed
// once to warm up, then `rounds` times between two events.  Writes the mean
// time per launch in microseconds.  Returns 0, or a HIP error code
// (hipErrorInvalidValue for a shape that does not tile 16 MiB).
int kvc_calib_read_floor(int grid, int loads, int strided, int nt, int rounds, double* us_per_launch) {
    if (!us_per_launch || rounds < 1 || grid < 256 || grid > 4096 || grid % 256) return (int)hipErrorInvalidValue;
    const int per_wg = (int)(kLaunchBytes / grid);
    if ((size_t)per_wg * grid != kLaunchBytes || (loads != 2 && loads != 4 && loads != 8 && loads != 16))
        return (int)hipErrorInvalidValue;
    if (per_wg % (4096 * loads) || (strided && (16384 % (4096 * loads) || per_wg % 16384)))
        return (int)hipErrorInvalidValue;
    FloorKernel k = loads == 2    ? floor_kernel<2>(strided, nt)
                    : loads == 4  ? floor_kernel<4>(strided, nt)
                    : loads == 8  ? floor_kernel<8>(strided, nt)
                                  : floor_kernel<16>(strided, nt);
    // block ids of the 4 replicas: disjoint draws from a seeded permutation
    std::vector<int32_t> perm(kFloorPoolBlocks);
    for (int i = 0; i < kFloorPoolBlocks; i++) perm[i] = i;
    uint64_t st = 0x6b76635f666c6f72ull;
    for (int i = kFloorPoolBlocks - 1; i > 0; i--) {
        st += 0x9e3779b97f4a7c15ull;
        uint64_t z = st;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const int j = (int)(z % (uint64_t)(i + 1));
        const int32_t tmp = perm[i];
        perm[i] = perm[j];
        perm[j] = tmp;
    }
    uint8_t* pool = nullptr;
    int32_t* ids = nullptr;
    uint32_t* sink = nullptr;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.f;
    hipError_t e;
    if ((e = hipMalloc(&pool, kRegionBytes * 2 * kFloorLayers)) == hipSuccess &&
        (e = hipMalloc(&ids, sizeof(int32_t) * kFloorReps * kFloorSeqBlocks)) == hipSuccess &&
        (e = hipMalloc(&sink, sizeof(uint32_t) * 4096 * 256)) == hipSuccess &&
        (e = hipMemset(pool, 0x3c, kRegionBytes * 2 * kFloorLayers)) == hipSuccess &&
        (e = hipMemcpy(ids, perm.data(), sizeof(int32_t) * kFloorReps * kFloorSeqBlocks, hipMemcpyHostToDevice)) ==
            hipSuccess &&
        (e = hipStreamCreate(&stream)) == hipSuccess && (e = hipEventCreate(&e0)) == hipSuccess &&
        (e = hipEventCreate(&e1)) == hipSuccess &&
        (e = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal)) == hipSuccess) {
        for (int r = 0; r < kFloorReps; r++)
            for (int l = 0; l < kFloorLayers; l++)
                hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, stream, pool, ids + r * kFloorSeqBlocks, l, per_wg,
                                   sink);
        hipError_t le = hipGetLastError();
        e = hipStreamEndCapture(stream, &graph);
        if (e == hipSuccess) e = le;
        if (e == hipSuccess && (e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) == hipSuccess &&
            (e = hipGraphLaunch(exec, stream)) == hipSuccess && (e = hipEventRecord(e0, stream)) == hipSuccess) {
            for (int i = 0; i < rounds && e == hipSuccess; i++) e = hipGraphLaunch(exec, stream);
            if (e == hipSuccess && (e = hipEventRecord(e1, stream)) == hipSuccess &&
                (e = hipEventSynchronize(e1)) == hipSuccess)
                e = hipEventElapsedTime(&ms, e0, e1);
        }
    }
    if (stream) (void)hipStreamSynchronize(stream);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (stream) (void)hipStreamDestroy(stream);
    if (sink) (void)hipFree(sink);
    if (ids) (void)hipFree(ids);
    if (pool) (void)hipFree(pool);
    if (e != hipSuccess) return (int)e;
    *us_per_launch = ms * 1e3 / ((double)rounds * kFloorReps * kFloorLayers);
    return 0;
}

// Time the MFMA-only loop for operand distribution `mode` (0, 1 or 2) on the
// current device: 4 workgroups of 4 waves per CU (2 resident per SIMD), `reps` x
// 32 MFMAs per wave, `launches` back-to-back launches between two events
// after one warm-up launch.  Writes the achieved dense rate in TFLOP/s.
// Returns 0, or a HIP error code.
int kvc_calib_mfma_bf16(int mode, int reps, int launches, double* tflops) {
    if (mode < 0 || mode > 2 || reps < 1 || launches < 1 || !tflops) return (int)hipErrorInvalidValue;
    int dev = 0, ncu = 0;
    hipError_t e;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return (int)e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return (int)e;
    const int grid = 4 * ncu, threads = 256;
    float* sink = nullptr;
    if ((e = hipMalloc(&sink, (size_t)grid * threads * sizeof(float))) != hipSuccess) return (int)e;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.f;
    if ((e = hipEventCreate(&e0)) == hipSuccess && (e = hipEventCreate(&e1)) == hipSuccess) {
        hipLaunchKernelGGL(mfma_rate_kernel, dim3(grid), dim3(threads), 0, nullptr, mode, reps, sink);
        (void)hipEventRecord(e0, nullptr);
        for (int i = 0; i < launches; i++)
            hipLaunchKernelGGL(mfma_rate_kernel, dim3(grid), dim3(threads), 0, nullptr, mode, reps, sink);
        (void)hipEventRecord(e1, nullptr);
        if ((e = hipGetLastError()) == hipSuccess && (e = hipEventSynchronize(e1)) == hipSuccess)
            e = hipEventElapsedTime(&ms, e0, e1);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(sink);
    if (e != hipSuccess) return (int)e;
    const double flops = (double)launches * grid * (threads / 64) * reps * kSteps * (2.0 * 32 * 32 * 16);
    *tflops = flops / (ms * 1e-3) / 1e12;
    return 0;
}

}  // extern "C"
