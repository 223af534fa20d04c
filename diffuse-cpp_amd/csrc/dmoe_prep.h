// dmoe_prep.h — conversion of one (row, 256-value super-block) of f32
// activations into the int8 operand layout of k_expert.hip (ActI8), by one
// wavefront.  Used by the front and conversion kernels (k_prep.hip).
//
// ACT_Q8K reproduces ggml's Q8_K conversion of the activations that
// ggml_mul_mat_id performs before Q4_K dots (src/diffuse-moe-graph.cpp:266-269):
// per 256 values, the value of largest magnitude (lowest index on ties) maps to
// -127, iscale = -127/max, q = min(127, nearest_even(iscale*x)), d = 1/iscale,
// plus sums of 16 quants.
//
// ACT_SPLIT keeps the shared expert's f32 activations (the reference casts its
// weights to F32, :8-12, :282-284) to 15-16 significant bits: with the
// power-of-two scale s = 2^-k that brings the largest magnitude of the
// super-block into [2^14, 2^15) (one step lower if it would round above
// 32512), X = nearest_even(v / s) = 256*a1 + a0 with a0 in [-128, 127]; the a1
// digits are row `row` (d = 256 s), the a0 digits row `rows + row` (d = s).
//
// ACT_Q80 reproduces ggml's Q8_0 conversion (the vec_dot_type of Q8_0 weights):
// per 32 values d = amax/127, q = roundf(v * (1/d)) (half away from zero), d
// kept as its fp16 rounding.  ACT_SPLIT32 is ACT_SPLIT with the scale chosen
// per 32 values.  Both write one scale per 32 values and no sums.
#pragma once

#include "dmoe_device.h"

namespace dmoe {

// Byte position p (0..255) of the operand layout -> value index inside the
// super-block: p = 64g + 8j + b holds value 32j + 8g + b.
__device__ __forceinline__ int src_index(int p)
{
    const int g = p >> 6, j = (p >> 3) & 7, b = p & 7;
    return 32 * j + 8 * g + b;
}

// v[c] = value lane + 64 c of the super-block; sv: 256 floats of LDS owned by
// the calling wavefront.  Contraction is off: the rounding is ggml's.
__device__ __forceinline__ void prep_values(const float (&v)[4], const ActI8 &out, int mode,
                                            int row, int rows, int sb, int nsb, float *sv)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    // value of largest magnitude, lowest index on ties (index lane + 64 c:
    // the first c whose ballot has a match, then its lowest lane); NaNs
    // never match, and with every value NaN amax stays -1 and aval 0
    float lmax = -1.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) lmax = fmaxf(lmax, fabsf(v[c]));
    const float amax = wave_max_f32(lmax, -1.0f);
    float aval = 0.0f;
    bool found = false;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint64_t m = __ballot(fabsf(v[c]) == amax);
        if (!found && m) {
            found = true;
            aval = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[c]),
                                                                       __builtin_ctzll(m)));
        }
    }

    const int K = nsb * 256;
    const size_t qbase = (size_t)row * K + sb * 256;
    const size_t bbase = (size_t)row * (K / 16) + sb * 16;
    if (mode == ACT_Q80 || mode == ACT_SPLIT32) {
        // per 32-value block: value lane + 64c is in block 2c + lane / 32
        float bmax[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float h = half_max_f32(fabsf(v[c]), __builtin_nanf(""));
            const float m0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, h), 31));
            const float m1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, h), 63));
            bmax[c] = lane < 32 ? m0 : m1;
        }
        const size_t dbase = (size_t)row * (K / 32) + sb * 8;
        if (mode == ACT_Q80) {
            float dq[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float d = bmax[c] / 127.0f;
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                sv[lane + 64 * c] = roundf(v[c] * id);
                dq[c] = (float)(_Float16)d;
            }
            if ((lane & 31) == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) out.d[dbase + 2 * c + (lane >> 5)] = dq[c];
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            uint32_t pk = 0;
#pragma unroll
            for (int i = 0; i < 4; i++)
                pk |= ((uint32_t)(int)sv[src_index(4 * lane + i)] & 0xffu) << (8 * i);
            *reinterpret_cast<uint32_t *>(out.q + qbase + 4 * lane) = pk;
        } else {
            int kc[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                int k = 0;
                if (bmax[c] != 0.0f) {
                    int ex = 0;
                    (void)frexpf(bmax[c], &ex);
                    k = 15 - ex;
                    if (nearest_int(ldexpf(bmax[c], k)) > 32512) k -= 1;
                }
                kc[c] = k;
                sv[lane + 64 * c] = (float)nearest_int(ldexpf(v[c], k));
            }
            if ((lane & 31) == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const size_t b = dbase + 2 * c + (lane >> 5);
                    out.d[b] = ldexpf(1.0f, 8 - kc[c]);                       // a1 row
                    out.d[(size_t)rows * (K / 32) + b] = ldexpf(1.0f, -kc[c]);  // a0 row
                }
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            uint32_t phi = 0, plo = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int X = (int)sv[src_index(4 * lane + i)];
                const int a1 = (X + 128) >> 8, a0 = X - (a1 << 8);
                phi |= ((uint32_t)a1 & 0xffu) << (8 * i);
                plo |= ((uint32_t)a0 & 0xffu) << (8 * i);
            }
            *reinterpret_cast<uint32_t *>(out.q + qbase + 4 * lane) = phi;
            *reinterpret_cast<uint32_t *>(out.q + (size_t)rows * K + qbase + 4 * lane) = plo;
        }
    } else if (mode == ACT_Q8K) {
        float dscale = 0.0f;
        int qc[4] = {0, 0, 0, 0};
        if (amax != 0.0f) {
            const float iscale = -127.0f / aval;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int q = nearest_int(iscale * v[c]);
                qc[c] = q < 127 ? q : 127;
            }
            dscale = 1.0f / iscale;
        }
#pragma unroll
        for (int c = 0; c < 4; c++) sv[lane + 64 * c] = (float)qc[c];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        uint32_t pk = 0;
#pragma unroll
        for (int i = 0; i < 4; i++)
            pk |= ((uint32_t)(int)sv[src_index(4 * lane + i)] & 0xffu) << (8 * i);
        *reinterpret_cast<uint32_t *>(out.q + qbase + 4 * lane) = pk;
        // sums of 16 quants: values 16 g .. 16 g + 15 are lanes 16 r .. 16 r + 15
        // of c = g / 4, r = g % 4 (integers, exact in any order)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int s16 = row_sum16_i32(qc[c]);
            if ((lane & 15) == 15) out.bs[bbase + 4 * c + (lane >> 4)] = f2h((float)s16);
        }
        if (lane == 0) out.d[(size_t)row * nsb + sb] = dscale;
    } else {
        int k = 0;
        if (amax != 0.0f) {
            int ex = 0;
            (void)frexpf(amax, &ex);          // amax = f * 2^ex, f in [0.5, 1)
            k = 15 - ex;                      // amax * 2^k in [2^14, 2^15)
            if (nearest_int(ldexpf(amax, k)) > 32512) k -= 1;
        }
        int xc[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            xc[c] = nearest_int(ldexpf(v[c], k));
            sv[lane + 64 * c] = (float)xc[c];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        uint32_t phi = 0, plo = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int X = (int)sv[src_index(4 * lane + i)];
            const int a1 = (X + 128) >> 8, a0 = X - (a1 << 8);
            phi |= ((uint32_t)a1 & 0xffu) << (8 * i);
            plo |= ((uint32_t)a0 & 0xffu) << (8 * i);
        }
        const size_t lo_off = (size_t)rows * K;
        *reinterpret_cast<uint32_t *>(out.q + qbase + 4 * lane) = phi;
        *reinterpret_cast<uint32_t *>(out.q + lo_off + qbase + 4 * lane) = plo;
        // digit sums of 16 values (lanes 16 r .. 16 r + 15 of c: group 4 c + r)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int a1 = (xc[c] + 128) >> 8, a0 = xc[c] - (a1 << 8);
            const int s1 = row_sum16_i32(a1), s0 = row_sum16_i32(a0);
            if ((lane & 15) == 15) {
                const int g = 4 * c + (lane >> 4);
                out.bs[bbase + g] = f2h((float)s1);
                out.bs[(size_t)rows * (K / 16) + bbase + g] = f2h((float)s0);
            }
        }
        if (lane == 0) {
            out.d[(size_t)row * nsb + sb] = ldexpf(1.0f, 8 - k);           // a1 row
            out.d[(size_t)(rows + row) * nsb + sb] = ldexpf(1.0f, -k);     // a0 row
        }
    }
    // sv is reused by the wavefront's next unit
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// One wavefront converts one (row, super-block) of a job.  sv: 256 floats of LDS.
__device__ __forceinline__ void prep_wave(const PrepJob &job, int wid, float *sv)
{
    const int lane = threadIdx.x & 63;
    const int nsb = job.K / 256;
    const int row = wid / nsb, sb = wid - row * nsb;
    const float *x = job.src + (size_t)row * job.K + sb * 256;
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = x[lane + 64 * c];
    prep_values(v, job.out, job.mode, row, job.rows, sb, nsb, sv);
}

} // namespace dmoe
