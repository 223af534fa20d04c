// dmoe_device.h — device helpers shared by the routing and activation kernels.
//
// Everything here is bit-deterministic: single IEEE operations in a fixed
// order (every function body disables contraction), binary64 exp built from
// add/mul/fma/rint only, correctly rounded division.
#pragma once

#include "dmoe_internal.h"

namespace dmoe {

// A load of element i of a wave-uniform array through the scalar cache
// (s_load: counted by lgkmcnt, never by the vmcnt of the vector loads, and
// not queued behind them).  For data the kernel does not write.
template <class T>
__device__ __forceinline__ T ldc(const T *p, int i)
{
    return ((const __attribute__((address_space(4))) T *)(uintptr_t)p)[i];
}

// The f32 epilogue of one Q4_K super-block product: acc + dx (d S - dmin M),
// rounded the same way in every kernel whatever its file's contraction
// setting: d S rounded, then two fused multiply-adds.  (Left to
// contraction, the compiler fused the expression differently in different
// inlining contexts, and kernels meant to give the same bits did not.)
__device__ __forceinline__ float q4k_epi(float acc, float dx, float d, float S, float dmin, float M)
{
    return __builtin_fmaf(dx, __builtin_fmaf(-dmin, M, d * S), acc);
}

// exp(x) in binary64 rounded once to binary32.  Cody-Waite reduction
// x = k ln2 + r (ln2 split into a 32-significant-bit head and a tail, so k*head
// is exact), exp(r) by its degree-13 Taylor polynomial in Horner form with
// fma, then scaling by 2^k through the exponent field.
__device__ __forceinline__ double exp_f64(double x)
{
#pragma clang fp contract(off)
    const double inv_ln2 = 1.4426950408889634;
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    double kd = rint(x * inv_ln2);
    double r = fma(-kd, ln2_hi, x);
    r = fma(-kd, ln2_lo, r);
    double p = 1.0 / 6227020800.0;
    p = fma(p, r, 1.0 / 479001600.0);
    p = fma(p, r, 1.0 / 39916800.0);
    p = fma(p, r, 1.0 / 3628800.0);
    p = fma(p, r, 1.0 / 362880.0);
    p = fma(p, r, 1.0 / 40320.0);
    p = fma(p, r, 1.0 / 5040.0);
    p = fma(p, r, 1.0 / 720.0);
    p = fma(p, r, 1.0 / 120.0);
    p = fma(p, r, 1.0 / 24.0);
    p = fma(p, r, 1.0 / 6.0);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    long long k = (long long)kd;
    double two_k = __longlong_as_double((long long)((unsigned long long)(k + 1023) << 52));
    return p * two_k;
}

__device__ __forceinline__ float exp_f32(float x)
{
#pragma clang fp contract(off)
    if (x != x) return x;
    // exp(100) overflows binary32 and exp(-110) rounds to 0: clamping keeps
    // every result and keeps k in the normal binary64 exponent range.
    x = x > 100.0f ? 100.0f : x;
    x = x < -110.0f ? -110.0f : x;
    return (float)exp_f64((double)x);
}

// ggml_sigmoid (src/diffuse-moe-graph.cpp:204)
__device__ __forceinline__ float sigmoid_f32(float x)
{
#pragma clang fp contract(off)
    return 1.0f / (1.0f + exp_f32(-x));
}

// Descending-value order with ties to the lower expert id; NaN sorts last and
// -0 equals +0.
__device__ __forceinline__ uint32_t order_key(float f)
{
    if (f != f) return 0u;
    if (f == 0.0f) f = 0.0f;
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool ranks_before(uint32_t ka, int ea, uint32_t kb, int eb)
{
    return ka > kb || (ka == kb && ea < eb);
}

// order_key and expert id in one integer: a larger value ranks first, and
// equal scores rank the lower expert id first (ids below 65536).
__device__ __forceinline__ uint64_t rank_key(uint32_t key, int e)
{
    return ((uint64_t)key << 32) | (uint32_t)(0xFFFFu - (uint32_t)e);
}

// round half to even for |v| < 2^22 (the magic-number rounding ggml uses)
__device__ __forceinline__ int nearest_int(float v)
{
#pragma clang fp contract(off)
    const float t = v + 12582912.0f;
    return (int)(__float_as_uint(t) & 0x007fffffu) - 0x00400000;
}

__device__ __forceinline__ uint16_t f2h(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// DPP reductions (results exact whatever the order: max of floats, sums of
// integers).  wave_max_f32: the maximum over the 64 lanes (lanes with NaN
// contribute nothing unless every lane holds NaN).  row_sum16_i32: lane 15
// of every 16-lane row receives the sum of its row.  half_max_f32: lanes 31
// and 63 receive the maxima of lanes 0..31 and 32..63.
#define DMOE_DPP(old, v, ctrl, rmask) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, (float)(old)), \
                                                          __builtin_bit_cast(int, (float)(v)), ctrl, rmask, 0xF, false))

__device__ __forceinline__ float row_prefix_max_f32(float v, float id)
{
    v = fmaxf(v, DMOE_DPP(id, v, 0x111, 0xF));   // row_shr:1
    v = fmaxf(v, DMOE_DPP(id, v, 0x112, 0xF));   // row_shr:2
    v = fmaxf(v, DMOE_DPP(id, v, 0x114, 0xF));   // row_shr:4
    v = fmaxf(v, DMOE_DPP(id, v, 0x118, 0xF));   // row_shr:8
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v, float id)
{
    v = row_prefix_max_f32(v, id);
    v = fmaxf(v, DMOE_DPP(id, v, 0x142, 0xA));   // row_bcast:15
    v = fmaxf(v, DMOE_DPP(id, v, 0x143, 0xC));   // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// lanes 31 and 63 hold the maxima of the two 32-lane halves
__device__ __forceinline__ float half_max_f32(float v, float id)
{
    v = row_prefix_max_f32(v, id);
    return fmaxf(v, DMOE_DPP(id, v, 0x142, 0xA));  // row_bcast:15
}

__device__ __forceinline__ int row_sum16_i32(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    return v;
}

} // namespace dmoe
