// kvc_device.h -- device helpers for the gfx950 kernels: bf16 bit handling,
// RNE rounding, wave64 cross-lane primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvc {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (u >> 16) | 0x40u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

// Two finite floats -> packed bf16 pair, round to nearest even, branch free
// (v_cvt_pk_bf16_f32 on gfx950).  For hot loops whose inputs are never NaN.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// a.x*b.x + a.y*b.y + c on packed bf16 pairs (v_dot2_f32_bf16), fp32 result.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// xor-shuffle inside a wave64 (ds_swizzle bit mode covers xor masks < 32;
// xor 32 crosses the two 32-lane halves and uses ds_bpermute).
template <int MASK>
__device__ __forceinline__ float shfl_xor(float v) {
    if constexpr (MASK < 32) {
        constexpr int pattern = (MASK << 10) | 0x1F;  // and=0x1F, or=0, xor=MASK
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), pattern));
    } else {
        int lane = __lane_id();
        return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ MASK) << 2, __float_as_int(v)));
    }
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Orders LDS accesses of one wave against each other without a workgroup
// barrier (LDS ops of a wave execute in order; this stops compiler motion).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Schraudolph (1999) exp as the reference computes it (src/engine.cpp:2349-2356):
// clamp to [-88, 88] (min first, then max), then the fp32 bit pattern of
// (int32)(12102203 x + 1065353216), slope 2^23/ln2 and bias 127 * 2^23.  The
// reference is built with -ffast-math for an FMA host, so the multiply-add is
// one fused operation (v_fma_f32 here, correctly rounded like x86 vfmadd).
// The scalar helper converts by truncation (v_cvt_i32_f32); the AVX-512 SiLU
// (:2367-2373) converts with cvtps2dq, round to nearest even.  The two differ
// only where the sum is below 2^23, which happens only for x < -87.3; the bit
// pattern is then a denormal e and 1 + e rounds to 1 either way, so the SiLU
// (x / (1 + e)) takes this truncating helper too and gives the same bits (a
// check over every fp32 input in [-88, -80] found 28,361 that round
// differently, all with 1 + e = 1).  After the clamp the sum lies in
// (0, 2^31), so the conversion never saturates.
__device__ __forceinline__ float schraudolph_exp(float x) {
    x = fmaxf(-88.0f, fminf(88.0f, x));
    return __int_as_float((int)__builtin_fmaf(12102203.0f, x, 1065353216.0f));
}
// The reference's gate sigmoid, fast_sigmoidf (src/engine.cpp:2358-2360):
// 1 / (1 + fast_expf(-x)), correctly rounded as the reference's IEEE division
// rounds it, bit-exact with that formula for every input but NaN.  With x
// clamped, y = 1 + fast_expf(-x) lies in [1, 2^127].  Below 2^126 the quotient
// is v_rcp_f32 (within 1 ulp) followed by one Newton step on FMAs (the
// residual 1 - y r is exact), which gives the correctly rounded 1 / y for
// every y the bf16 gates produce (an exhaustive GPU test covers all of them);
// larger y, whose reciprocal is subnormal, take the full IEEE division
// sequence (two scalings, five FMAs, a fixup) that the Newton step replaces.
__device__ __forceinline__ float sigmoid_ref(float x) {
    const float y = 1.0f + schraudolph_exp(-x);
    if (__builtin_expect(y >= 0x1p126f, 0)) return 1.0f / y;
    const float r = __builtin_amdgcn_rcpf(y);
    return __builtin_fmaf(__builtin_fmaf(-y, r, 1.0f), r, r);
}

// Raw buffer access with cache-policy bits.  kCpolSC1 marks an access as
// coherent at agent (device) scope: stores write through the XCD's L2 and
// loads do not take a stale line from it, so data can pass between
// workgroups on different XCDs without a full L2 writeback (buffer_wbl2).
constexpr int kCpolSC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

}  // namespace kvc
