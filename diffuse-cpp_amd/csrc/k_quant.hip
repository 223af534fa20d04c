// k_quant.hip — quantisation kernels.
//
//  * activation conversion to the weight's vec_dot_type before the expert
//    products, as ggml_mul_mat_id does on the CPU (the reference's expert
//    products, src/diffuse-moe-graph.cpp:266-269):
//      Q4_K weights -> Q8_K activations, Q8_0 -> Q8_0, F16 -> F16, F32 -> F32
//  * weight quantisation into GGUF blocks (counterpart of quantize_to_type,
//    tools/quant_lib.c:16-27), used to build synthetic expert tensors in HBM.
#include "dmoe_internal.h"

#pragma clang fp contract(off)

namespace dmoe {

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);   // round to nearest even
}

// round half to even for |v| < 2^22
__device__ __forceinline__ int nearest_int(float v)
{
    const float t = v + 12582912.0f;
    return (int)(__float_as_uint(t) & 0x007fffffu) - 0x00400000;
}

// ---------------------------------------------------------------------------
// Q8_K: one wavefront per 256-value super-block; lane l holds values l,
// l+64, l+128, l+192.  The value of largest magnitude (lowest index on ties)
// maps to -127: iscale = -127/max, q = min(127, nearest(iscale*x)),
// d = 1/iscale, bsums = sums of 16 consecutive q.
__global__ __launch_bounds__(256) void k_act_q8K(const float *__restrict__ src, int rows, int n,
                                                 int8_t *__restrict__ qs, float *__restrict__ dq,
                                                 int16_t *__restrict__ bsums)
{
    const int lane = threadIdx.x & 63;
    const int nsb = n / 256;
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= rows * nsb) return;
    const int row = wid / nsb, sb = wid % nsb;
    const float *x = src + (size_t)row * n + sb * 256;

    float v[4];
    float amax = -1.0f;
    int aidx = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        v[c] = x[lane + 64 * c];
        const float a = fabsf(v[c]);
        if (a > amax) { amax = a; aidx = lane + 64 * c; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float oa = __shfl_xor(amax, m, 64);
        const int oi = __shfl_xor(aidx, m, 64);
        if (oa > amax || (oa == amax && oi < aidx)) { amax = oa; aidx = oi; }
    }
    int8_t *q = qs + (size_t)row * n + sb * 256;
    int16_t *bs = bsums + (size_t)row * (n / 16) + sb * 16;
    if (amax == 0.0f) {
#pragma unroll
        for (int c = 0; c < 4; c++) q[lane + 64 * c] = 0;
        if (lane < 16) bs[lane] = 0;
        if (lane == 0) dq[(size_t)row * nsb + sb] = 0.0f;
        return;
    }
    const float vmax = x[aidx];
    const float iscale = -127.0f / vmax;
    int qi[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int t = nearest_int(iscale * v[c]);
        qi[c] = t < 127 ? t : 127;
        q[lane + 64 * c] = (int8_t)qi[c];
    }
    // group g = 16 consecutive values = lanes 16*(g%4)..+15 of register g/4
#pragma unroll
    for (int c = 0; c < 4; c++) {
        int s = qi[c];
        s += __shfl_xor(s, 8, 64);
        s += __shfl_xor(s, 4, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 1, 64);
        if ((lane & 15) == 0) bs[4 * c + (lane >> 4)] = (int16_t)s;
    }
    if (lane == 0) dq[(size_t)row * nsb + sb] = 1.0f / iscale;
}

// Q8_0: lane = value; 32-lane halves are independent blocks.
// d = amax/127, q = roundf(x/d) (half away from zero), d kept as its fp16 value.
__global__ __launch_bounds__(256) void k_act_q8_0(const float *__restrict__ src, int rows, int n,
                                                  int8_t *__restrict__ qs, float *__restrict__ dq)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)rows * n) return;     // n % 32 == 0: whole blocks exit together
    const float v = src[i];
    float amax = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    qs[i] = (int8_t)roundf(v * id);
    if ((threadIdx.x & 31) == 0) dq[i / 32] = f16_bits_to_f32(f32_to_f16_bits(d));
}

__global__ __launch_bounds__(256) void k_act_f16(const float *__restrict__ src, size_t total,
                                                 uint16_t *__restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < total) dst[i] = f32_to_f16_bits(src[i]);
}

__global__ __launch_bounds__(256) void k_copy_f32(const float *__restrict__ src, size_t total,
                                                  float *__restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < total) dst[i] = src[i];
}

hipError_t launch_act_quant(const float *src, int rows, int n, const ActBuf &dst, hipStream_t s)
{
    const size_t total = (size_t)rows * n;
    switch (dst.type) {
    case DMOE_ACT_Q8_K: {
        const int waves = rows * (n / 256);
        hipLaunchKernelGGL(k_act_q8K, dim3((waves + 3) / 4), dim3(256), 0, s, src, rows, n,
                           (int8_t *)dst.vals, dst.d, dst.bsums);
        break;
    }
    case DMOE_TYPE_Q8_0:
        hipLaunchKernelGGL(k_act_q8_0, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           src, rows, n, (int8_t *)dst.vals, dst.d);
        break;
    case DMOE_TYPE_F16:
        hipLaunchKernelGGL(k_act_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           src, total, (uint16_t *)dst.vals);
        break;
    case DMOE_TYPE_F32:
        hipLaunchKernelGGL(k_copy_f32, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           src, total, (float *)dst.vals);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weight quantisers: one thread per block.
//   Q8_0: as the activation quantiser above.
//   Q4_K: min/max per 32-value sub-block (a plain quantiser, not ggml's
//         iterative one): scale_j = (max - min')/15, min' = min(min, 0),
//         d = max scale / 63, dmin = max(-min') / 63 (both as fp16),
//         6-bit sc_j, m_j by nearest rounding, q = nearest((x + dmin*m_j) /
//         (d*sc_j)) clamped to 0..15, packed in the GGUF Q4_K layout.
__global__ __launch_bounds__(256) void k_wq_q8_0(const float *__restrict__ src, int64_t nblk,
                                                 uint8_t *__restrict__ dst)
{
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    const float *x = src + b * 32;
    uint8_t *y = dst + b * 34;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_bits(d);
    y[0] = (uint8_t)(dh & 0xff);
    y[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

__global__ __launch_bounds__(256) void k_wq_q4K(const float *__restrict__ src, int64_t nblk,
                                                uint8_t *__restrict__ dst)
{
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    const float *x = src + b * 256;
    uint8_t *y = dst + b * 144;
    float scale[8], mn[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; l++) {
            const float v = x[32 * j + l];
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        if (lo > 0.0f) lo = 0.0f;
        scale[j] = (hi - lo) / 15.0f;
        mn[j] = -lo;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mn[j] > max_min) max_min = mn[j];
    }
    const uint16_t dh = f32_to_f16_bits(max_scale / 63.0f);
    const uint16_t mh = f32_to_f16_bits(max_min / 63.0f);
    const float d = f16_bits_to_f32(dh), dmin = f16_bits_to_f32(mh);
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const float imin = dmin > 0.0f ? 1.0f / dmin : 0.0f;
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        const int a = nearest_int(scale[j] * id);
        const int c = nearest_int(mn[j] * imin);
        sc[j] = (uint8_t)(a < 0 ? 0 : a > 63 ? 63 : a);
        m[j] = (uint8_t)(c < 0 ? 0 : c > 63 ? 63 : c);
    }
    uint8_t scales[12];
    for (int j = 0; j < 4; j++) {
        scales[j] = sc[j];
        scales[j + 4] = m[j];
    }
    for (int j = 4; j < 8; j++) {
        scales[j + 4] = (uint8_t)((sc[j] & 0x0f) | ((m[j] & 0x0f) << 4));
        scales[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
        scales[j] |= (uint8_t)((m[j] >> 4) << 6);
    }
    y[0] = (uint8_t)(dh & 0xff);
    y[1] = (uint8_t)(dh >> 8);
    y[2] = (uint8_t)(mh & 0xff);
    y[3] = (uint8_t)(mh >> 8);
    for (int j = 0; j < 12; j++) y[4 + j] = scales[j];
    for (int c = 0; c < 4; c++) {
        const float ed0 = d * (float)sc[2 * c], em0 = dmin * (float)m[2 * c];
        const float ed1 = d * (float)sc[2 * c + 1], em1 = dmin * (float)m[2 * c + 1];
        for (int l = 0; l < 32; l++) {
            int q0 = 0, q1 = 0;
            if (ed0 > 0.0f) q0 = nearest_int((x[64 * c + l] + em0) / ed0);
            if (ed1 > 0.0f) q1 = nearest_int((x[64 * c + 32 + l] + em1) / ed1);
            q0 = q0 < 0 ? 0 : q0 > 15 ? 15 : q0;
            q1 = q1 < 0 ? 0 : q1 > 15 ? 15 : q1;
            y[16 + 32 * c + l] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// Q6_K (a plain quantiser, not ggml's make_qx_quants search): per 16-value
// sub-block the value of largest magnitude v_j (first on ties) gives the
// signed scale s_j = -v_j / 32; the s of largest magnitude gives d = -s / 128
// (fp16); sc_j = nearest(s_j / d) clamped to -128..127, q = nearest(x / (d
// sc_j)) clamped to -32..31, stored as q + 32 in ggml's block_q6_K layout
// (ql: low nibbles of weights 128 h + 32 k + l at ql[64 h + 32 (k % 2) + l],
// low half for k < 2, high half for k >= 2; qh[32 h + l]: bits 2k, 2k + 1).
__device__ __forceinline__ int q6_of(const float *x, const float *ds, int v)
{
    const float s = ds[v >> 4];
    int q = 0;
    if (s != 0.0f) q = nearest_int(x[v] / s);
    q = q < -32 ? -32 : q > 31 ? 31 : q;
    return q + 32;
}

__global__ __launch_bounds__(256) void k_wq_q6K(const float *__restrict__ src, int64_t nblk,
                                                uint8_t *__restrict__ dst)
{
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    const float *x = src + b * 256;
    uint8_t *y = dst + b * Q6K_BYTES;
    float sj[16];
    float smax = 0.0f, samax = 0.0f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.0f, vmax = 0.0f;
        for (int l = 0; l < 16; l++) {
            const float a = fabsf(x[16 * j + l]);
            if (a > amax) {
                amax = a;
                vmax = x[16 * j + l];
            }
        }
        sj[j] = -vmax / 32.0f;
        if (amax / 32.0f > samax) {
            samax = amax / 32.0f;
            smax = sj[j];
        }
    }
    if (samax == 0.0f) {
        for (int i = 0; i < Q6K_BYTES; i++) y[i] = 0;
        return;
    }
    const uint16_t dh = f32_to_f16_bits(-smax / 128.0f);
    const float d = f16_bits_to_f32(dh);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    float ds[16];
    for (int j = 0; j < 16; j++) {
        int sc = nearest_int(sj[j] * id);
        sc = sc < -128 ? -128 : sc > 127 ? 127 : sc;
        y[192 + j] = (uint8_t)(int8_t)sc;
        ds[j] = d * (float)sc;
    }
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const int v = 128 * h + l;
            const int q0 = q6_of(x, ds, v), q1 = q6_of(x, ds, v + 32);
            const int q2 = q6_of(x, ds, v + 64), q3 = q6_of(x, ds, v + 96);
            y[64 * h + l] = (uint8_t)((q0 & 15) | ((q2 & 15) << 4));
            y[64 * h + 32 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            y[128 + 32 * h + l] = (uint8_t)((q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6));
        }
    y[208] = (uint8_t)(dh & 0xff);
    y[209] = (uint8_t)(dh >> 8);
}

__global__ __launch_bounds__(256) void k_wq_f16(const float *__restrict__ src, int64_t total,
                                                uint16_t *__restrict__ dst)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < total) dst[i] = f32_to_f16_bits(src[i]);
}

// ---------------------------------------------------------------------------
// Q4_K row layout -> tiled layout: per matrix, 16-row tiles; inside a tile the
// super-blocks come first, so the 16 rows' blocks of one super-block are one
// contiguous 2304-byte run starting at ((r/16) * nsb + sb) * 2304.  Inside the
// run, the repacked 144-byte block of row r % 16 is nine 16-byte pieces, piece
// k at byte (16 k + r % 16) * 16 (piece-major, so that a kernel copying the
// run to LDS as it lies reads each piece without bank conflicts).
__global__ __launch_bounds__(256) void k_tile_q4k(const uint8_t *__restrict__ src, size_t nb1,
                                                  size_t nb2, int rows, int nsb, int mats,
                                                  uint8_t *__restrict__ dst)
{
    // one thread per 144-byte block
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per_mat = (size_t)rows * nsb;
    if (i >= per_mat * mats) return;
    const int m = (int)(i / per_mat);
    const size_t j = i - (size_t)m * per_mat;
    const int sb = (int)(j % nsb);
    const int r = (int)(j / nsb);
    const uint8_t *in = src + (size_t)m * nb2 + (size_t)r * nb1 + (size_t)sb * Q4K_BYTES;
    uint8_t *out = dst + (size_t)m * rows * nsb * Q4K_BYTES +
                   ((size_t)(r / 16) * nsb + sb) * (16 * Q4K_BYTES) + (size_t)(r % 16) * 16;
    uint8_t blk[Q4K_BYTES];
#pragma unroll
    for (int p = 0; p < 9; p++)
        *reinterpret_cast<uint4 *>(blk + 16 * p) = *reinterpret_cast<const uint4 *>(in + 16 * p);
    // get_scale_min_k4 of the twelve scale bytes
    const uint8_t *q = blk + 4;
    uint32_t sc[8], mn[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (k < 4) {
            sc[k] = q[k] & 63u;
            mn[k] = q[k + 4] & 63u;
        } else {
            sc[k] = (q[k + 4] & 0xFu) | ((uint32_t)(q[k - 4] >> 6) << 4);
            mn[k] = (uint32_t)(q[k + 4] >> 4) | ((uint32_t)(q[k] >> 6) << 4);
        }
    }
    uint32_t w[9 * 4];
    w[0] = *reinterpret_cast<const uint32_t *>(blk);          // d, dmin
    w[1] = sc[0] | sc[1] << 6 | sc[2] << 12 | sc[3] << 18 | sc[4] << 24 | (mn[7] & 3u) << 30;
    w[2] = sc[5] | sc[6] << 6 | sc[7] << 12 | mn[0] << 18 | mn[1] << 24 | ((mn[7] >> 2) & 3u) << 30;
    w[3] = mn[2] | mn[3] << 6 | mn[4] << 12 | mn[5] << 18 | mn[6] << 24 | ((mn[7] >> 4) & 3u) << 30;
    // quant bytes: 16 + 32g + 8c + b  <-  32c + 8g + b (as 8-byte pieces)
    const uint64_t *qs = reinterpret_cast<const uint64_t *>(blk + 16);
    uint64_t *ws = reinterpret_cast<uint64_t *>(w + 4);
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
        for (int c = 0; c < 4; c++) ws[4 * g + c] = qs[4 * c + g];
#pragma unroll
    for (int p = 0; p < 9; p++)
        *reinterpret_cast<uint4 *>(out + 256 * p) = *reinterpret_cast<const uint4 *>(w + 4 * p);
}

hipError_t launch_tile_q4k(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s)
{
    if (rows % 16 || K % 256 || nb1 % 16 || (mats > 1 && nb2 % 16)) return hipErrorInvalidValue;
    const size_t total = (size_t)rows * (K / 256) * mats;
    hipLaunchKernelGGL(k_tile_q4k, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src,
                       nb1, nb2, rows, K / 256, mats, dst);
    return hipGetLastError();
}

// Q6_K row layout -> the tiled layout of the few-token projections
// (k_proj.hip): per matrix, 16-row tiles, super-block-major, the 16 rows of
// one super-block a contiguous 3360-byte run at ((r / 16) nsb + sb) 3360 of
// 210 16-byte pieces (the same bytes as the GGUF blocks, rearranged):
//   pieces k 64 + 16 g + r (k = 0, 1, 2): what lane (r, g) of a wavefront
//     reads for row r: twelve dwords L[0..7], H[0..3] of its 64 quants
//     32 p + 8 g + b (p = 0..7 pairs of 32 weights, b = 0..7):
//       L[p] byte i: low nibbles of quants (p, b = i) and (p, b = 4 + i)
//       H[p'] byte i: the high 2 bits of quants (2p', i), (2p', 4 + i),
//                     (2p' + 1, i), (2p' + 1, 4 + i) at bits 0, 2, 4, 6
//   pieces 192 + r: the 16 int8 scales of row r
//   pieces 208, 209: the 16 rows' f16 d (row r at byte 2 r)
__global__ __launch_bounds__(256) void k_tile_q6k(const uint8_t *__restrict__ src, size_t nb1,
                                                  size_t nb2, int rows, int nsb, int mats,
                                                  uint8_t *__restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per_mat = (size_t)rows * nsb;
    if (i >= per_mat * mats) return;
    const int m = (int)(i / per_mat);
    const size_t j = i - (size_t)m * per_mat;
    const int sb = (int)(j % nsb);
    const int r = (int)(j / nsb);
    // 210-byte blocks are 2-byte aligned
    const uint16_t *in = reinterpret_cast<const uint16_t *>(src + (size_t)m * nb2 + (size_t)r * nb1 +
                                                            (size_t)sb * Q6K_BYTES);
    uint8_t blk[Q6K_BYTES];
    for (int k = 0; k < Q6K_BYTES / 2; k++) {
        const uint16_t v = in[k];
        blk[2 * k] = (uint8_t)(v & 0xff);
        blk[2 * k + 1] = (uint8_t)(v >> 8);
    }
    uint8_t q[256];
    for (int v = 0; v < 256; v++) {
        const int h = v >> 7, rr = v & 127, k = rr >> 5, l = rr & 31;
        const uint8_t lb = blk[64 * h + l + 32 * (k & 1)];
        const int lo = (k >> 1) ? (lb >> 4) : (lb & 15);
        const int hi = (blk[128 + 32 * h + l] >> (2 * k)) & 3;
        q[v] = (uint8_t)(lo | (hi << 4));
    }
    uint8_t *run = dst + (size_t)m * rows * nsb * Q6K_BYTES + ((size_t)(r / 16) * nsb + sb) * (16 * Q6K_BYTES);
    const int r16 = r % 16;
    for (int g = 0; g < 4; g++) {
        uint32_t w[12];
        for (int p = 0; p < 8; p++) {
            uint32_t v = 0;
            for (int b = 0; b < 4; b++) {
                const uint32_t lo = q[32 * p + 8 * g + b] & 15u, hi = q[32 * p + 8 * g + 4 + b] & 15u;
                v |= (lo | (hi << 4)) << (8 * b);
            }
            w[p] = v;
        }
        for (int pp = 0; pp < 4; pp++) {
            uint32_t v = 0;
            for (int b = 0; b < 4; b++) {
                const int e0 = 64 * pp + 8 * g + b;
                const uint32_t byte = (uint32_t)(q[e0] >> 4) | ((uint32_t)(q[e0 + 4] >> 4) << 2) |
                                      ((uint32_t)(q[e0 + 32] >> 4) << 4) | ((uint32_t)(q[e0 + 36] >> 4) << 6);
                v |= byte << (8 * b);
            }
            w[8 + pp] = v;
        }
        for (int k = 0; k < 3; k++)
            *reinterpret_cast<uint4 *>(run + (size_t)(64 * k + 16 * g + r16) * 16) =
                make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
    }
    uint32_t sc[4];
    for (int k = 0; k < 4; k++)
        sc[k] = (uint32_t)blk[192 + 4 * k] | ((uint32_t)blk[193 + 4 * k] << 8) | ((uint32_t)blk[194 + 4 * k] << 16) |
                ((uint32_t)blk[195 + 4 * k] << 24);
    *reinterpret_cast<uint4 *>(run + (size_t)(192 + r16) * 16) = make_uint4(sc[0], sc[1], sc[2], sc[3]);
    *reinterpret_cast<uint16_t *>(run + 208 * 16 + 2 * r16) = (uint16_t)(blk[208] | (blk[209] << 8));
}

hipError_t launch_tile_q6k(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s)
{
    if (rows % 16 || K % 256 || nb1 % 2 || (mats > 1 && nb2 % 2)) return hipErrorInvalidValue;
    const size_t total = (size_t)rows * (K / 256) * mats;
    hipLaunchKernelGGL(k_tile_q6k, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src,
                       nb1, nb2, rows, K / 256, mats, dst);
    return hipGetLastError();
}

hipError_t launch_quantize_weights(int32_t type, const float *src, void *dst, int64_t nrows,
                                   int64_t n_per_row, hipStream_t s)
{
    const int64_t total = nrows * n_per_row;
    switch (type) {
    case DMOE_TYPE_Q4_K: {
        const int64_t nblk = total / 256;
        hipLaunchKernelGGL(k_wq_q4K, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, src,
                           nblk, (uint8_t *)dst);
        break;
    }
    case DMOE_TYPE_Q6_K: {
        const int64_t nblk = total / 256;
        hipLaunchKernelGGL(k_wq_q6K, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, src,
                           nblk, (uint8_t *)dst);
        break;
    }
    case DMOE_TYPE_Q8_0: {
        const int64_t nblk = total / 32;
        hipLaunchKernelGGL(k_wq_q8_0, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, src,
                           nblk, (uint8_t *)dst);
        break;
    }
    case DMOE_TYPE_F16:
        hipLaunchKernelGGL(k_wq_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src,
                           total, (uint16_t *)dst);
        break;
    case DMOE_TYPE_F32:
        hipLaunchKernelGGL(k_copy_f32, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src,
                           (size_t)total, (float *)dst);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace dmoe
