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
#include "dmoe_internal.h"

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

hipError_t launch_residual_rmsnorm(float *h, const float *y, const float *gain, float *x, int rows, int H,
                                   float eps, hipStream_t s)
{
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_residual_rmsnorm, dim3(rows), dim3(NORM_THREADS), 0, s, h, y, gain, x, H, eps);
    return hipGetLastError();
}

} // namespace dmoe
