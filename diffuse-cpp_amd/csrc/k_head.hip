// k_head.hip — per-position argmax and confidence of the LM-head logits
// (the temperature-0 branch of sample_token, src/diffuse-sampler.cpp:29-49).
//
// One workgroup per token row of V logits.  Argmax: each thread scans its
// strided indices in ascending order keeping the first of equal maxima (a NaN
// never compares greater), then the threads' (value, index) pairs combine in
// a fixed tree, larger value first, lower index on ties; a NaN at index 0 is
// the answer, as in the reference's loop which starts from logits[0].
// Confidence: 1 / sum_v exp(l_v - max) with exp the library's correctly
// rounded binary32 exp, each thread summing its terms in binary64, the
// partials added in a fixed tree (the reference adds in float, sequentially:
// the two sums differ by that float accumulation's rounding).
#include "dmoe_device.h"

namespace dmoe {

constexpr int AP_THREADS = 256;

__global__ __launch_bounds__(AP_THREADS) void k_argmax_prob(const float *__restrict__ logits, int V,
                                                            int32_t *__restrict__ tokens,
                                                            float *__restrict__ probs)
{
#pragma clang fp contract(off)
    __shared__ float s_v[AP_THREADS];
    __shared__ int s_i[AP_THREADS];
    __shared__ double s_d[AP_THREADS];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *row = logits + (size_t)t * V;
    float m = -__builtin_inff();
    int mi = V;                                  // none yet
    for (int v = tid; v < V; v += AP_THREADS) {
        const float l = row[v];
        if (l > m) {
            m = l;
            mi = v;
        }
    }
    s_v[tid] = m;
    s_i[tid] = mi;
    __syncthreads();
    for (int w = AP_THREADS / 2; w > 0; w >>= 1) {
        if (tid < w) {
            const float a = s_v[tid], b = s_v[tid + w];
            const int ia = s_i[tid], ib = s_i[tid + w];
            if (b > a || (b == a && ib < ia)) {
                s_v[tid] = b;
                s_i[tid] = ib;
            }
        }
        __syncthreads();
    }
    const float first = row[0];
    int best = s_i[0];
    float best_val = s_v[0];
    // every logit -inf, or logits[0] NaN: the reference keeps index 0
    if (best == V || first != first) {
        best = 0;
        best_val = first;
    }
    double acc = 0.0;
    for (int v = tid; v < V; v += AP_THREADS) acc += (double)exp_f32(row[v] - best_val);
    s_d[tid] = acc;
    __syncthreads();
    for (int w = AP_THREADS / 2; w > 0; w >>= 1) {
        if (tid < w) s_d[tid] = s_d[tid] + s_d[tid + w];
        __syncthreads();
    }
    if (tid == 0) {
        tokens[t] = best;
        probs[t] = 1.0f / (float)s_d[0];
    }
}

hipError_t launch_argmax_prob(const float *logits, int N, int V, int32_t *tokens, float *probs,
                              hipStream_t s)
{
    if (N <= 0 || V <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax_prob, dim3(N), dim3(AP_THREADS), 0, s, logits, V, tokens, probs);
    return hipGetLastError();
}

} // namespace dmoe
