// dmoe_prep.h — conversion of one (row, 256-value super-block) of f32
// activations into the MFMA operand layout of k_expert.hip (ActMfma), by one
// wavefront.  Used by the front and conversion kernels (k_prep.hip) and by the
// expert kernel for its gate/up results.
//
// ACT_Q8K reproduces ggml's Q8_K conversion of the activations that
// ggml_mul_mat_id performs before Q4_K dots (src/diffuse-moe-graph.cpp:266-269):
// per 256 values, the value of largest magnitude (lowest index on ties) maps to
// -127, iscale = -127/max, q = min(127, nearest_even(iscale*x)), d = 1/iscale,
// plus sums of 16 quants.  The quants are small integers, exact in f16.
//
// ACT_SPLIT keeps f32 activations (the shared expert, whose weights the
// reference casts to F32, :8-12, :282-284): per super-block the values are
// scaled by 2^k into [2^9, 2^10) in magnitude and split into hi = f16(v) and
// lo = f16(v - hi), about 22 significant bits; d = 2^-k.  The lo halves are
// written as rows `rows`..2*rows-1.
#pragma once

#include "dmoe_device.h"

namespace dmoe {

// Position p (0..255) of the operand layout -> value index inside the super-block.
__device__ __forceinline__ int src_index(int p)
{
    const int g = p >> 6, s = (p >> 3) & 7, e = p & 7;
    const int perm = (e & 1) ? ((e & 2) ? 3 : 2) : ((e & 2) ? 1 : 0);   // {0,2,1,3}
    return 64 * g + 32 * (e >> 2) + 4 * s + perm;
}

// v[c] = value lane + 64 c of the super-block; sv: 256 floats of LDS owned by
// the calling wavefront.  Contraction is off: the rounding is ggml's.
__device__ __forceinline__ void prep_values(const float (&v)[4], const ActMfma &out, int mode,
                                            int row, int rows, int sb, int nsb, float *sv)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    // value of largest magnitude, lowest index on ties
    float amax = -1.0f, aval = 0.0f;
    int aidx = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float a = fabsf(v[c]);
        if (a > amax) { amax = a; aval = v[c]; aidx = lane + 64 * c; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float oa = __shfl_xor(amax, m, 64);
        const float ov = __shfl_xor(aval, m, 64);
        const int oi = __shfl_xor(aidx, m, 64);
        if (oa > amax || (oa == amax && oi < aidx)) { amax = oa; aval = ov; aidx = oi; }
    }

    const int K = nsb * 256;
    const size_t vbase = (size_t)row * K + sb * 256;
    const size_t bbase = (size_t)row * (K / 16) + sb * 16;
    if (mode == ACT_Q8K) {
        float dscale = 0.0f;
        if (amax != 0.0f) {
            const float iscale = -127.0f / aval;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int q = nearest_int(iscale * v[c]);
                sv[lane + 64 * c] = (float)(q < 127 ? q : 127);
            }
            dscale = 1.0f / iscale;
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) sv[lane + 64 * c] = 0.0f;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = f2h(sv[src_index(4 * lane + i)]);
        uint2 pk;
        pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
        pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
        *reinterpret_cast<uint2 *>(out.v + vbase + 4 * lane) = pk;
        if (lane < 16) {
            float s = 0.0f;                 // integer sum, exact
            for (int i = 0; i < 16; i++) s += sv[16 * lane + i];
            out.bs[bbase + lane] = f2h(s);
        }
        if (lane == 0) out.d[(size_t)row * nsb + sb] = dscale;
    } else {
        int ex = 0;
        float scale = 1.0f, dinv = 1.0f;
        if (amax != 0.0f) {
            (void)frexpf(amax, &ex);          // amax = f * 2^ex, f in [0.5, 1)
            scale = ldexpf(1.0f, 10 - ex);    // scaled amax in [2^9, 2^10)
            dinv = ldexpf(1.0f, ex - 10);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) sv[lane + 64 * c] = v[c] * scale;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float f = sv[src_index(4 * lane + i)];
            hi[i] = f2h(f);
            lo[i] = f2h(f - (float)__builtin_bit_cast(_Float16, hi[i]));
        }
        uint2 ph, pl;
        ph.x = (uint32_t)hi[0] | ((uint32_t)hi[1] << 16);
        ph.y = (uint32_t)hi[2] | ((uint32_t)hi[3] << 16);
        pl.x = (uint32_t)lo[0] | ((uint32_t)lo[1] << 16);
        pl.y = (uint32_t)lo[2] | ((uint32_t)lo[3] << 16);
        *reinterpret_cast<uint2 *>(out.v + vbase + 4 * lane) = ph;
        *reinterpret_cast<uint2 *>(out.v_lo + vbase + 4 * lane) = pl;
        if (lane < 16) {
            float s = 0.0f;
            for (int i = 0; i < 16; i++) s += sv[16 * lane + i];
            const uint16_t sh = f2h(s);
            out.bs[bbase + lane] = sh;
            out.bs_lo[bbase + lane] = f2h(s - (float)__builtin_bit_cast(_Float16, sh));
        }
        if (lane == 0) {
            out.d[(size_t)row * nsb + sb] = dinv;             // hi row
            out.d[(size_t)(rows + row) * nsb + sb] = dinv;    // lo row
        }
    }
    // sv is reused by the wavefront's next unit
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

} // namespace dmoe
