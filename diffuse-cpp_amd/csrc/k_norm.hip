// k_norm.hip — the residual stream around the MoE segment (gfx950).
//
// src/diffuse-moe-graph.cpp:292 adds the segment's output to the residual
// stream (cur = moe_out + residual), and :175-178 form the next segment's
// input from that stream: cur = rms_norm(residual) * post_attn_norm (the
// attention half of the layer sits in between; a chain of MoE segments alone
// goes straight from one to the next).  ggml_rms_norm (ggml is not vendored in
// the reference; this is its CPU definition) per row of n values: the f32
// squares summed in double, mean = (float)(sum / n), scale =
// 1.0f / sqrtf(mean + eps), out = x * scale; the gain multiply is a separate
// ggml_mul, (x * scale) * gain.
//
// One workgroup per row: h += y (when y is given, in place), then
// x = rms_norm(h) (* gain when given).  The double sum runs in a fixed order
// (per thread over its float4s, then a xor butterfly per wavefront, then the
// wavefront partials in order), so results are reproducible; it differs from
// ggml's sequential order only inside double rounding.
#include "dmoe_prep.h"

#pragma clang fp contract(off)

namespace dmoe {

constexpr int NORM_THREADS = 256;

__global__ __launch_bounds__(NORM_THREADS) void k_residual_rmsnorm(float *__restrict__ h,
                                                                  const float *__restrict__ y,
                                                                  const float *__restrict__ gain,
                                                                  float *__restrict__ x, int H, float eps)
{
    __shared__ double s_part[NORM_THREADS / 64];
    const size_t base = (size_t)blockIdx.x * H;
    float4 *hr = reinterpret_cast<float4 *>(h + base);
    const float4 *yr = y ? reinterpret_cast<const float4 *>(y + base) : nullptr;
    const float4 *gr = reinterpret_cast<const float4 *>(gain);
    float4 *xr = reinterpret_cast<float4 *>(x + base);
    const int n4 = H / 4, tid = threadIdx.x;
    double acc = 0.0;
    for (int i = tid; i < n4; i += NORM_THREADS) {
        float4 v = hr[i];
        if (yr) {
            const float4 u = yr[i];
            v.x = v.x + u.x;
            v.y = v.y + u.y;
            v.z = v.z + u.z;
            v.w = v.w + u.w;
            hr[i] = v;
        }
        acc += (double)(v.x * v.x);
        acc += (double)(v.y * v.y);
        acc += (double)(v.z * v.z);
        acc += (double)(v.w * v.w);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if ((tid & 63) == 0) s_part[tid >> 6] = acc;
    __syncthreads();
    double sum = 0.0;
#pragma unroll
    for (int w = 0; w < NORM_THREADS / 64; w++) sum += s_part[w];
    const float mean = (float)(sum / (double)H);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = tid; i < n4; i += NORM_THREADS) {
        const float4 v = hr[i];
        float4 o = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
        if (gr) {
            const float4 g = gr[i];
            o = make_float4(o.x * g.x, o.y * g.y, o.z * g.z, o.w * g.w);
        }
        xr[i] = o;
    }
}

// The same row operation around the few-token projections (k_proj.hip),
// with their producers and consumers folded in: the residual added is the sum
// of a projection's KS reduction slices (in slice order, as k_proj_reduce
// adds them), h may be read from one buffer and written to another, and the
// normed row may leave as two int8 digit rows (ACT_SPLIT, prep_values, one
// wavefront per super-block) for the next projection instead of (or beside)
// f32.  The row is staged in LDS between the sum and the outputs.  The sum
// runs on the first NORM_THREADS threads in k_residual_rmsnorm's order; the
// outputs use all NF_THREADS.
constexpr int NF_MAXH = 8192;
constexpr int NF_THREADS = 1024;

__global__ __launch_bounds__(NF_THREADS) void k_norm_fused(NormArgs a)
{
    __shared__ double s_part[NORM_THREADS / 64];
    __shared__ float4 s_row[NF_MAXH / 4];
    __shared__ float s_v[NF_THREADS / 64][256];
    const int H = a.H, n4 = H / 4, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int row = blockIdx.x;
    const size_t base4 = (size_t)row * n4;
    const float4 *hi = reinterpret_cast<const float4 *>(a.h_in) + base4;
    float4 *ho = a.h_out ? reinterpret_cast<float4 *>(a.h_out) + base4 : nullptr;
    const float4 *gr = reinterpret_cast<const float4 *>(a.gain);
    // the row (h + the slices' sum) to LDS and h_out, every thread
    for (int i = tid; i < n4; i += NF_THREADS) {
        float4 v = hi[i];
        if (a.y) {
            const float4 *yr = reinterpret_cast<const float4 *>(a.y) + base4 + i;
            float4 u = yr[0];
            for (int k = 1; k < a.ks; k++) {
                const float4 b = yr[(size_t)k * a.kstride / 4];
                u.x = u.x + b.x;
                u.y = u.y + b.y;
                u.z = u.z + b.z;
                u.w = u.w + b.w;
            }
            v.x = v.x + u.x;
            v.y = v.y + u.y;
            v.z = v.z + u.z;
            v.w = v.w + u.w;
            if (ho) ho[i] = v;
        }
        s_row[i] = v;
    }
    __syncthreads();
    // the squares' double sum in k_residual_rmsnorm's order
    double acc = 0.0;
    if (tid < NORM_THREADS)
        for (int i = tid; i < n4; i += NORM_THREADS) {
            const float4 v = s_row[i];
            acc += (double)(v.x * v.x);
            acc += (double)(v.y * v.y);
            acc += (double)(v.z * v.z);
            acc += (double)(v.w * v.w);
        }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if (lane == 0 && tid < NORM_THREADS) s_part[w] = acc;
    __syncthreads();
    double sum = 0.0;
#pragma unroll
    for (int q = 0; q < NORM_THREADS / 64; q++) sum += s_part[q];
    const float mean = (float)(sum / (double)H);
    const float scale = 1.0f / sqrtf(mean + a.eps);
    if (a.x) {
        float4 *xr = reinterpret_cast<float4 *>(a.x) + base4;
        for (int i = tid; i < n4; i += NF_THREADS) {
            const float4 v = s_row[i];
            float4 o = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
            if (gr) {
                const float4 g = gr[i];
                o = make_float4(o.x * g.x, o.y * g.y, o.z * g.z, o.w * g.w);
            }
            xr[i] = o;
        }
    }
    if (a.act.q) {
        const float *sr = reinterpret_cast<const float *>(s_row);
        const int nsb = H / 256;
        for (int sb = w; sb < nsb; sb += NF_THREADS / 64) {
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int i = sb * 256 + lane + 64 * c;
                float o = sr[i] * scale;
                if (a.gain) o = o * a.gain[i];
                v[c] = o;
            }
            prep_values(v, a.act, ACT_SPLIT, row, a.rows, sb, nsb, s_v[w]);
        }
    }
}

hipError_t launch_norm_fused(const NormArgs &a, hipStream_t s)
{
    if (a.rows <= 0) return hipSuccess;
    if (a.H <= 0 || a.H % 256 || a.H > NF_MAXH || !a.h_in || (a.y && (a.ks < 1 || a.kstride % 4)) ||
        (a.act.q && a.act.K != a.H))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_norm_fused, dim3(a.rows), dim3(NF_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_residual_rmsnorm(float *h, const float *y, const float *gain, float *x, int rows, int H,
                                   float eps, hipStream_t s)
{
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_residual_rmsnorm, dim3(rows), dim3(NORM_THREADS), 0, s, h, y, gain, x, H, eps);
    return hipGetLastError();
}

} // namespace dmoe
