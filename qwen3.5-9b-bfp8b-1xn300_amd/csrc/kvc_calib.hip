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
#include <hip/hip_runtime.h>

#include <cstdint>

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

}  // namespace

extern "C" {

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
