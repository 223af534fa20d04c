// k_gemv.hip — GEMV-style expert products (few tokens per expert).
//
// The routed products mirror ggml_mul_mat_id on the CPU
// (src/diffuse-moe-graph.cpp:266-269): activations were converted to the
// weight's vec_dot_type beforehand (k_quant.hip), so each row dot is an
// exact integer dot per block followed by the block's float scale:
//   Q4_K x Q8_K : sum_j sc_j * (q . xq)_j and sum_j m_j * bsum_j per super-block
//   Q8_0 x Q8_0 : (q . xq) * (dw * dx) per 32-block
//   F16  x F16  : exact products, fp32 accumulation
//   F32  x F32  : fp32 fma accumulation
// The shared expert (:280-286) runs on F32 activations against weights
// dequantised in registers (the reference casts them to F32, :8-12).
//
// One wavefront per output row; lanes split the row into "units" (Q4_K: 64
// weights of one super-block, Q8_0: one 32-block, F16: 8 values, F32: 4)
// and keep one partial per token for a chunk of up to TB tokens; partials are
// combined with a butterfly.  The weight unit is loaded once per token chunk.
#include "dmoe_internal.h"

namespace dmoe {

constexpr int TB = 8;   // tokens per pass over a weight row

__device__ __forceinline__ float h2f(uint32_t h16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h16); }

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ uint32_t scale_byte(const uint4 &h, int i)
{
    const uint32_t w = i < 4 ? h.y : (i < 8 ? h.z : h.w);
    return (w >> (8 * (i & 3))) & 0xffu;
}

// get_scale_min_k4 over the 12 scale bytes held in h.y, h.z, h.w
__device__ __forceinline__ void q4k_scale_min(const uint4 &h, int j, int &sc, int &m)
{
    if (j < 4) {
        sc = (int)(scale_byte(h, j) & 63u);
        m = (int)(scale_byte(h, j + 4) & 63u);
    } else {
        sc = (int)((scale_byte(h, j + 4) & 0x0fu) | ((scale_byte(h, j - 4) >> 6) << 4));
        m = (int)((scale_byte(h, j + 4) >> 4) | ((scale_byte(h, j) >> 6) << 4));
    }
}

// ---------------------------------------------------------------------------
// Weight units
template <int WT> struct WUnit;

template <> struct WUnit<DMOE_TYPE_Q4_K> {
    static constexpr int N = 64;
    float d, dmin;
    int sc0, sc1, m0, m1;
    uint32_t q[8];
    __device__ __forceinline__ void load(const uint8_t *row, int u)
    {
        const uint8_t *blk = row + (size_t)(u >> 2) * Q4K_BYTES;
        const int c = u & 3;
        const uint4 h = *reinterpret_cast<const uint4 *>(blk);
        d = h2f(h.x & 0xffffu);
        dmin = h2f(h.x >> 16);
        q4k_scale_min(h, 2 * c, sc0, m0);
        q4k_scale_min(h, 2 * c + 1, sc1, m1);
        const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * c);
        const uint4 a = qp[0], b = qp[1];
        q[0] = a.x; q[1] = a.y; q[2] = a.z; q[3] = a.w;
        q[4] = b.x; q[5] = b.y; q[6] = b.z; q[7] = b.w;
    }
    // Q8_K activation row `row` of xq
    __device__ __forceinline__ float dot(const ActBuf &xq, int row, int u) const
    {
        const int n = xq.n;
        const int b = u >> 2, c = u & 3;
        const uint4 *xp = reinterpret_cast<const uint4 *>((const int8_t *)xq.vals + (size_t)row * n +
                                                          b * 256 + 64 * c);
        const uint4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
        const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo = __builtin_amdgcn_sdot4((int)(q[i] & 0x0f0f0f0fu), (int)xl[i], lo, false);
            hi = __builtin_amdgcn_sdot4((int)((q[i] >> 4) & 0x0f0f0f0fu), (int)xh[i], hi, false);
        }
        const int16_t *bs = xq.bsums + (size_t)row * (n / 16) + b * 16 + 4 * c;
        const int sumi = sc0 * lo + sc1 * hi;
        const int summ = m0 * ((int)bs[0] + (int)bs[1]) + m1 * ((int)bs[2] + (int)bs[3]);
        const float xd = xq.d[(size_t)row * (n / 256) + b];
        return (xd * d) * (float)sumi - (xd * dmin) * (float)summ;
    }
    // f32 activations against the dequantised unit (w = d*sc*q - dmin*m)
    __device__ __forceinline__ float dotf(const float *x, int u) const
    {
        const int b = u >> 2, c = u & 3;
        const float4 *xp = reinterpret_cast<const float4 *>(x + b * 256 + 64 * c);
        const float d0 = d * (float)sc0, d1 = d * (float)sc1;
        const float n0 = dmin * (float)m0, n1 = dmin * (float)m1;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 xl = xp[i];
            const float4 xh = xp[8 + i];
            const uint32_t w = q[i];
            acc = __builtin_fmaf(d0 * (float)(w & 15u) - n0, xl.x, acc);
            acc = __builtin_fmaf(d0 * (float)((w >> 8) & 15u) - n0, xl.y, acc);
            acc = __builtin_fmaf(d0 * (float)((w >> 16) & 15u) - n0, xl.z, acc);
            acc = __builtin_fmaf(d0 * (float)((w >> 24) & 15u) - n0, xl.w, acc);
            acc = __builtin_fmaf(d1 * (float)((w >> 4) & 15u) - n1, xh.x, acc);
            acc = __builtin_fmaf(d1 * (float)((w >> 12) & 15u) - n1, xh.y, acc);
            acc = __builtin_fmaf(d1 * (float)((w >> 20) & 15u) - n1, xh.z, acc);
            acc = __builtin_fmaf(d1 * (float)((w >> 28) & 15u) - n1, xh.w, acc);
        }
        return acc;
    }
};

template <> struct WUnit<DMOE_TYPE_Q8_0> {
    static constexpr int N = 32;
    float d;
    uint32_t q[8];
    __device__ __forceinline__ void load(const uint8_t *row, int u)
    {
        // 34-byte blocks are only 2-byte aligned inside a row
        const uint16_t *p = reinterpret_cast<const uint16_t *>(row + (size_t)u * Q8_0_BYTES);
        d = h2f(p[0]);
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = (uint32_t)p[1 + 2 * i] | ((uint32_t)p[2 + 2 * i] << 16);
    }
    __device__ __forceinline__ float dot(const ActBuf &xq, int row, int u) const
    {
        const int n = xq.n;
        const uint4 *xp = reinterpret_cast<const uint4 *>((const int8_t *)xq.vals + (size_t)row * n + u * 32);
        const uint4 x0 = xp[0], x1 = xp[1];
        const uint32_t xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) s = __builtin_amdgcn_sdot4((int)q[i], (int)xv[i], s, false);
        return (float)s * (d * xq.d[(size_t)row * (n / 32) + u]);
    }
    __device__ __forceinline__ float dotf(const float *x, int u) const
    {
        const float4 *xp = reinterpret_cast<const float4 *>(x + u * 32);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 xv = xp[i];
            const uint32_t w = q[i];
            acc = __builtin_fmaf(d * (float)(int8_t)(w & 0xffu), xv.x, acc);
            acc = __builtin_fmaf(d * (float)(int8_t)((w >> 8) & 0xffu), xv.y, acc);
            acc = __builtin_fmaf(d * (float)(int8_t)((w >> 16) & 0xffu), xv.z, acc);
            acc = __builtin_fmaf(d * (float)(int8_t)(w >> 24), xv.w, acc);
        }
        return acc;
    }
};

// Q6_K (ggml's block_q6_K: ql[128], qh[64], int8 scales[16], f16 d; 210
// bytes per 256 weights).  Unit u: weights 64 c .. 64 c + 63 of super-block
// u / 4 (c = u % 4), i.e. half h = c / 2, quarters k0 = 2 (c % 2) and k0 + 1:
// weight 64 c + l (l < 32) has the low (k0 = 0) or high (k0 = 2) nibble of
// ql[64 h + l] and bits 2 k0 of qh[32 h + l]; weight 64 c + 32 + l the same
// nibble of ql[64 h + 32 + l] and bits 2 k0 + 2.  Sub-block 4 c + j (16
// weights) has scale scales[4 c + j].
template <> struct WUnit<DMOE_TYPE_Q6_K> {
    static constexpr int N = 64;
    float d;
    int sc[4];
    uint32_t q[16];     // 6-bit quants (0..63) as bytes: q[0..7] weights 0..31, q[8..15] 32..63
    // 210-byte blocks are only 2-byte aligned inside a row: dwords are read
    // as two halves
    __device__ __forceinline__ static uint32_t ld32(const uint16_t *p, int i)
    {
        return (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
    }
    __device__ __forceinline__ void load(const uint8_t *row, int u)
    {
        const uint8_t *blk = row + (size_t)(u >> 2) * Q6K_BYTES;
        const int c = u & 3, h = c >> 1, k0 = 2 * (c & 1);
        const uint16_t *ql = reinterpret_cast<const uint16_t *>(blk + 64 * h);
        const uint16_t *qh = reinterpret_cast<const uint16_t *>(blk + 128 + 32 * h);
        const int ns = 2 * k0;          // nibble shift 0 or 4
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t H = ld32(qh, i);
            q[i] = ((ld32(ql, i) >> ns) & 0x0f0f0f0fu) | (((H >> (2 * k0)) & 0x03030303u) << 4);
            q[8 + i] = ((ld32(ql, 8 + i) >> ns) & 0x0f0f0f0fu) | (((H >> (2 * k0 + 2)) & 0x03030303u) << 4);
        }
        const uint32_t s4 = ld32(reinterpret_cast<const uint16_t *>(blk + 192 + 4 * c), 0);
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = (int)(int8_t)(s4 >> (8 * j));
        d = h2f(*reinterpret_cast<const uint16_t *>(blk + 208));
    }
    // Q8_K activation row `row` of xq: per sub-block sum (q - 32) a =
    // sum q a - 32 (the row's sum of those 16 activations)
    __device__ __forceinline__ float dot(const ActBuf &xq, int row, int u) const
    {
        const int n = xq.n;
        const int b = u >> 2, c = u & 3;
        const uint4 *xp = reinterpret_cast<const uint4 *>((const int8_t *)xq.vals + (size_t)row * n +
                                                          b * 256 + 64 * c);
        const int16_t *bs = xq.bsums + (size_t)row * (n / 16) + b * 16 + 4 * c;
        int sumi = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 xv = xp[j];
            int sj = 0;
            sj = __builtin_amdgcn_sdot4((int)q[4 * j + 0], (int)xv.x, sj, false);
            sj = __builtin_amdgcn_sdot4((int)q[4 * j + 1], (int)xv.y, sj, false);
            sj = __builtin_amdgcn_sdot4((int)q[4 * j + 2], (int)xv.z, sj, false);
            sj = __builtin_amdgcn_sdot4((int)q[4 * j + 3], (int)xv.w, sj, false);
            sumi += sc[j] * (sj - 32 * (int)bs[j]);
        }
        const float xd = xq.d[(size_t)row * (n / 256) + b];
        return (xd * d) * (float)sumi;
    }
    // f32 activations against the dequantised unit (w = (d sc) (q - 32), exact)
    __device__ __forceinline__ float dotf(const float *x, int u) const
    {
        const int b = u >> 2, c = u & 3;
        const float4 *xp = reinterpret_cast<const float4 *>(x + b * 256 + 64 * c);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float ds = d * (float)sc[j];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 xv = xp[4 * j + i];
                const uint32_t w = q[4 * j + i];
                acc = __builtin_fmaf(ds * (float)((int)(w & 0xffu) - 32), xv.x, acc);
                acc = __builtin_fmaf(ds * (float)((int)((w >> 8) & 0xffu) - 32), xv.y, acc);
                acc = __builtin_fmaf(ds * (float)((int)((w >> 16) & 0xffu) - 32), xv.z, acc);
                acc = __builtin_fmaf(ds * (float)((int)(w >> 24) - 32), xv.w, acc);
            }
        }
        return acc;
    }
};

template <> struct WUnit<DMOE_TYPE_F16> {
    static constexpr int N = 8;
    uint4 w;
    __device__ __forceinline__ void load(const uint8_t *row, int u)
    {
        w = reinterpret_cast<const uint4 *>(row)[u];
    }
    __device__ __forceinline__ static float dot2(uint32_t a, uint32_t b, float acc)
    {
        acc = __builtin_fmaf(h2f(a & 0xffffu), h2f(b & 0xffffu), acc);
        return __builtin_fmaf(h2f(a >> 16), h2f(b >> 16), acc);
    }
    __device__ __forceinline__ float dot(const ActBuf &xq, int row, int u) const
    {
        const uint4 x = reinterpret_cast<const uint4 *>((const uint16_t *)xq.vals + (size_t)row * xq.n)[u];
        float acc = 0.0f;
        acc = dot2(w.x, x.x, acc);
        acc = dot2(w.y, x.y, acc);
        acc = dot2(w.z, x.z, acc);
        acc = dot2(w.w, x.w, acc);
        return acc;
    }
    __device__ __forceinline__ float dotf(const float *x, int u) const
    {
        const float4 a = reinterpret_cast<const float4 *>(x)[2 * u];
        const float4 b = reinterpret_cast<const float4 *>(x)[2 * u + 1];
        float acc = 0.0f;
        acc = __builtin_fmaf(h2f(w.x & 0xffffu), a.x, acc);
        acc = __builtin_fmaf(h2f(w.x >> 16), a.y, acc);
        acc = __builtin_fmaf(h2f(w.y & 0xffffu), a.z, acc);
        acc = __builtin_fmaf(h2f(w.y >> 16), a.w, acc);
        acc = __builtin_fmaf(h2f(w.z & 0xffffu), b.x, acc);
        acc = __builtin_fmaf(h2f(w.z >> 16), b.y, acc);
        acc = __builtin_fmaf(h2f(w.w & 0xffffu), b.z, acc);
        acc = __builtin_fmaf(h2f(w.w >> 16), b.w, acc);
        return acc;
    }
};

template <> struct WUnit<DMOE_TYPE_F32> {
    static constexpr int N = 4;
    float4 w;
    __device__ __forceinline__ void load(const uint8_t *row, int u)
    {
        w = reinterpret_cast<const float4 *>(row)[u];
    }
    __device__ __forceinline__ float dotf(const float *x, int u) const
    {
        const float4 a = reinterpret_cast<const float4 *>(x)[u];
        float acc = 0.0f;
        acc = __builtin_fmaf(w.x, a.x, acc);
        acc = __builtin_fmaf(w.y, a.y, acc);
        acc = __builtin_fmaf(w.z, a.z, acc);
        acc = __builtin_fmaf(w.w, a.w, acc);
        return acc;
    }
    __device__ __forceinline__ float dot(const ActBuf &xq, int row, int u) const
    {
        return dotf((const float *)xq.vals + (size_t)row * xq.n, u);
    }
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// ---------------------------------------------------------------------------
// Routed gate/up: grid (ceil(ff/4), E); wave = one ff row of expert e for all
// pairs routed to e.  h[pair][r] = silu(gate) * up.
template <int WT>
__global__ __launch_bounds__(256) void k_gateup_routed(WTensor wg, WTensor wu, ActBuf xq,
                                                       RouteParams rp, RouteBufs rb, int ff,
                                                       float *__restrict__ h)
{
    const int e = blockIdx.y;
    const int cnt = rb.counts[e];
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (cnt == 0 || r >= ff) return;
    const int lane = threadIdx.x & 63;
    const int off = rb.offsets[e];
    const int K = rp.top_k;
    const uint8_t *rg = wg.data + (size_t)e * wg.nb2 + (size_t)r * wg.nb1;
    const uint8_t *ru = wu.data + (size_t)e * wu.nb2 + (size_t)r * wu.nb1;
    const int nunits = xq.n / WUnit<WT>::N;
    for (int c0 = 0; c0 < cnt; c0 += TB) {
        const int nt = min(TB, cnt - c0);
        int pair[TB], tok[TB];
        float ag[TB], au[TB];
#pragma unroll
        for (int i = 0; i < TB; i++) {
            pair[i] = rb.perm[off + c0 + min(i, nt - 1)];
            tok[i] = pair[i] / K;
            ag[i] = 0.0f;
            au[i] = 0.0f;
        }
        for (int u = lane; u < nunits; u += 64) {
            WUnit<WT> a, b;
            a.load(rg, u);
            b.load(ru, u);
#pragma unroll
            for (int i = 0; i < TB; i++) {
                if (i < nt) {
                    ag[i] += a.dot(xq, tok[i], u);
                    au[i] += b.dot(xq, tok[i], u);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < TB; i++) {
            const float g = wave_sum(ag[i]);
            const float v = wave_sum(au[i]);
            if (lane == i && i < nt) h[(size_t)pair[i] * ff + r] = silu(g) * v;
        }
    }
}

// Routed down: grid (ceil(H/4), E); ye[pair][r] = Wd[e][r] . hq[pair]
template <int WT>
__global__ __launch_bounds__(256) void k_down_routed(WTensor wd, ActBuf hq, RouteBufs rb, int H,
                                                     float *__restrict__ ye)
{
    const int e = blockIdx.y;
    const int cnt = rb.counts[e];
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (cnt == 0 || r >= H) return;
    const int lane = threadIdx.x & 63;
    const int off = rb.offsets[e];
    const uint8_t *rd = wd.data + (size_t)e * wd.nb2 + (size_t)r * wd.nb1;
    const int nunits = hq.n / WUnit<WT>::N;
    for (int c0 = 0; c0 < cnt; c0 += TB) {
        const int nt = min(TB, cnt - c0);
        int pair[TB];
        float acc[TB];
#pragma unroll
        for (int i = 0; i < TB; i++) {
            pair[i] = rb.perm[off + c0 + min(i, nt - 1)];
            acc[i] = 0.0f;
        }
        for (int u = lane; u < nunits; u += 64) {
            WUnit<WT> a;
            a.load(rd, u);
#pragma unroll
            for (int i = 0; i < TB; i++)
                if (i < nt) acc[i] += a.dot(hq, pair[i], u);
        }
#pragma unroll
        for (int i = 0; i < TB; i++) {
            const float v = wave_sum(acc[i]);
            if (lane == i && i < nt) ye[(size_t)pair[i] * H + r] = v;
        }
    }
}

// Shared expert gate/up on f32 activations: grid ceil(sff/4); hs[t][r]
template <int WT>
__global__ __launch_bounds__(256) void k_gateup_shared(WTensor wg, WTensor wu,
                                                       const float *__restrict__ x, int N, int H,
                                                       int sff, float *__restrict__ hs)
{
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= sff) return;
    const int lane = threadIdx.x & 63;
    const uint8_t *rg = wg.data + (size_t)r * wg.nb1;
    const uint8_t *ru = wu.data + (size_t)r * wu.nb1;
    const int nunits = H / WUnit<WT>::N;
    for (int t0 = 0; t0 < N; t0 += TB) {
        const int nt = min(TB, N - t0);
        float ag[TB], au[TB];
#pragma unroll
        for (int i = 0; i < TB; i++) { ag[i] = 0.0f; au[i] = 0.0f; }
        for (int u = lane; u < nunits; u += 64) {
            WUnit<WT> a, b;
            a.load(rg, u);
            b.load(ru, u);
#pragma unroll
            for (int i = 0; i < TB; i++) {
                if (i < nt) {
                    const float *xr = x + (size_t)(t0 + i) * H;
                    ag[i] += a.dotf(xr, u);
                    au[i] += b.dotf(xr, u);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < TB; i++) {
            const float g = wave_sum(ag[i]);
            const float v = wave_sum(au[i]);
            if (lane == i && i < nt) hs[(size_t)(t0 + i) * sff + r] = silu(g) * v;
        }
    }
}

template <int WT>
__global__ __launch_bounds__(256) void k_down_shared(WTensor wd, const float *__restrict__ hs,
                                                     int N, int sff, int H, float *__restrict__ ys)
{
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= H) return;
    const int lane = threadIdx.x & 63;
    const uint8_t *rd = wd.data + (size_t)r * wd.nb1;
    const int nunits = sff / WUnit<WT>::N;
    for (int t0 = 0; t0 < N; t0 += TB) {
        const int nt = min(TB, N - t0);
        float acc[TB];
#pragma unroll
        for (int i = 0; i < TB; i++) acc[i] = 0.0f;
        for (int u = lane; u < nunits; u += 64) {
            WUnit<WT> a;
            a.load(rd, u);
#pragma unroll
            for (int i = 0; i < TB; i++)
                if (i < nt) acc[i] += a.dotf(hs + (size_t)(t0 + i) * sff, u);
        }
#pragma unroll
        for (int i = 0; i < TB; i++) {
            const float v = wave_sum(acc[i]);
            if (lane == i && i < nt) ys[(size_t)(t0 + i) * H + r] = v;
        }
    }
}

// ---------------------------------------------------------------------------
#define DMOE_TYPE_SWITCH(T, ...)                                                                   \
    switch (T) {                                                                                   \
    case DMOE_TYPE_Q4_K: { constexpr int WT = DMOE_TYPE_Q4_K; __VA_ARGS__; } break;                \
    case DMOE_TYPE_Q6_K: { constexpr int WT = DMOE_TYPE_Q6_K; __VA_ARGS__; } break;                \
    case DMOE_TYPE_Q8_0: { constexpr int WT = DMOE_TYPE_Q8_0; __VA_ARGS__; } break;                \
    case DMOE_TYPE_F16:  { constexpr int WT = DMOE_TYPE_F16;  __VA_ARGS__; } break;                \
    case DMOE_TYPE_F32:  { constexpr int WT = DMOE_TYPE_F32;  __VA_ARGS__; } break;                \
    default: return hipErrorInvalidValue;                                                          \
    }

hipError_t launch_gateup_routed(const WTensor &wg, const WTensor &wu, const ActBuf &xq,
                                const RouteParams &rp, const RouteBufs &rb, int ff, float *h,
                                hipStream_t s)
{
    const dim3 grid((ff + 3) / 4, rp.n_experts);
    DMOE_TYPE_SWITCH(wg.type, hipLaunchKernelGGL(k_gateup_routed<WT>, grid, dim3(256), 0, s, wg,
                                                 wu, xq, rp, rb, ff, h));
    return hipGetLastError();
}

hipError_t launch_down_routed(const WTensor &wd, const ActBuf &hq, const RouteParams &rp,
                              const RouteBufs &rb, int H, float *ye, hipStream_t s)
{
    const dim3 grid((H + 3) / 4, rp.n_experts);
    DMOE_TYPE_SWITCH(wd.type, hipLaunchKernelGGL(k_down_routed<WT>, grid, dim3(256), 0, s, wd, hq,
                                                 rb, H, ye));
    return hipGetLastError();
}

hipError_t launch_gateup_shared(const WTensor &wg, const WTensor &wu, const float *x, int N,
                                int H, int sff, float *hs, hipStream_t s)
{
    const dim3 grid((sff + 3) / 4);
    DMOE_TYPE_SWITCH(wg.type, hipLaunchKernelGGL(k_gateup_shared<WT>, grid, dim3(256), 0, s, wg,
                                                 wu, x, N, H, sff, hs));
    return hipGetLastError();
}

hipError_t launch_down_shared(const WTensor &wd, const float *hs, int N, int sff, int H,
                              float *ys, hipStream_t s)
{
    const dim3 grid((H + 3) / 4);
    DMOE_TYPE_SWITCH(wd.type, hipLaunchKernelGGL(k_down_shared<WT>, grid, dim3(256), 0, s, wd, hs,
                                                 N, sff, H, ys));
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Combine (:270-278, :285): y = ((ye_0 w_0 + ye_1 w_1) + ...) + ys, each
// product rounded before the add, slots in routing order.
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ ye,
                                                 const float *__restrict__ weights,
                                                 const float *__restrict__ ys, int N, int K, int H,
                                                 float *__restrict__ y)
{
#pragma clang fp contract(off)
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)N * H) return;
    const int t = (int)(i / H), r = (int)(i % H);
    float acc = ye[(size_t)(t * K) * H + r] * weights[t * K];
    for (int s = 1; s < K; s++) acc = acc + ye[(size_t)(t * K + s) * H + r] * weights[t * K + s];
    if (ys) acc = acc + ys[i];
    y[i] = acc;
}

// The same, four consecutive outputs per thread (H % 4 == 0, 16-byte aligned
// buffers): each output's operations and their order are those of k_combine.
__global__ __launch_bounds__(256) void k_combine4(const float4 *__restrict__ ye,
                                                  const float *__restrict__ weights,
                                                  const float4 *__restrict__ ys, int N, int K, int H4,
                                                  float4 *__restrict__ y)
{
#pragma clang fp contract(off)
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)N * H4) return;
    const int t = (int)(i / H4), r = (int)(i % H4);
    float4 v[8];
    const int kk = K < 8 ? K : 8;
#pragma unroll
    for (int s = 0; s < 8; s++)
        if (s < kk) v[s] = ye[(size_t)(t * K + s) * H4 + r];
    const float w0 = weights[t * K];
    float4 acc = make_float4(v[0].x * w0, v[0].y * w0, v[0].z * w0, v[0].w * w0);
    for (int s = 1; s < K; s++) {
        const float ws = weights[t * K + s];
        const float4 e = s < 8 ? v[s] : ye[(size_t)(t * K + s) * H4 + r];
        acc.x = acc.x + e.x * ws;
        acc.y = acc.y + e.y * ws;
        acc.z = acc.z + e.z * ws;
        acc.w = acc.w + e.w * ws;
    }
    if (ys) {
        const float4 b = ys[i];
        acc.x = acc.x + b.x;
        acc.y = acc.y + b.y;
        acc.z = acc.z + b.z;
        acc.w = acc.w + b.w;
    }
    y[i] = acc;
}

hipError_t launch_combine(const float *ye, const float *weights, const float *ys, int N, int K,
                          int H, float *y, hipStream_t s)
{
    const auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (H % 4 == 0 && al16(ye) && al16(y) && (!ys || al16(ys))) {
        const size_t total = (size_t)N * (H / 4);
        hipLaunchKernelGGL(k_combine4, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(ye), weights,
                           reinterpret_cast<const float4 *>(ys), N, K, H / 4, reinterpret_cast<float4 *>(y));
        return hipGetLastError();
    }
    const size_t total = (size_t)N * H;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, ye,
                       weights, ys, N, K, H, y);
    return hipGetLastError();
}

} // namespace dmoe
