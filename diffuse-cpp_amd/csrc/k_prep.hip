// k_prep.hip — the front of the layer and the activation conversions.
//
// Front kernel, one launch over three kinds of workgroups:
//   * router logits L = Wg x (src/diffuse-moe-graph.cpp:203) in one fixed fp32
//     summation order, with probs = sigmoid(L) (:204) and the selection score
//     sel = probs + bias (:207-210) computed by the lane that owns each logit;
//   * up to two conversions of x into the MFMA operand layout of k_expert.hip.
//
// The conversions themselves (Q8_K for the routed experts, two int8 digits
// for the shared expert) are in dmoe_prep.h.
#include "dmoe_prep.h"

#pragma clang fp contract(off)

namespace dmoe {

// One wavefront converts one (row, super-block) of a job.  sv: 256 floats of LDS.
__device__ void prep_wave(const PrepJob &job, int wid, float *sv)
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

// ---------------------------------------------------------------------------
// Router logits.  One wavefront per (LE experts, LT tokens).  For every
// (token, expert) lane l keeps one partial:  a_l = fma(W[k], x[k], a_l) for
// k = 256*i + 4*l + j, i ascending then j = 0..3; the 64 partials are then
// combined by six xor butterfly rounds (m = 32..1), after which every lane
// holds the same value (each round adds the same two operands in both
// partner lanes).  Lane t*LE + e then computes sigmoid and the score.  The
// tile shape only changes which rows a wavefront reads, not the order.
constexpr int LG_E = 2, LG_T = 4;        // up to a few hundred tokens
constexpr int LW_E = 8, LW_T = 8;        // more tokens: fewer re-reads of x

template <int LE, int LT>
__device__ void logits_wave(const float *__restrict__ W, const float *__restrict__ bias,
                            const float *__restrict__ x, int N, int H, int E, int wave,
                            const RouteBufs &rb)
{
    static_assert(LE * LT <= 64, "one lane per output");
    const int lane = threadIdx.x & 63;
    const int ne = (E + LE - 1) / LE;
    const int e0 = (wave % ne) * LE;
    const int t0 = (wave / ne) * LT;

    float acc[LT][LE];
#pragma unroll
    for (int t = 0; t < LT; t++)
#pragma unroll
        for (int e = 0; e < LE; e++) acc[t][e] = 0.0f;

    const float4 *wr[LE];
    const float4 *xr[LT];
#pragma unroll
    for (int e = 0; e < LE; e++)
        wr[e] = reinterpret_cast<const float4 *>(W + (size_t)min(e0 + e, E - 1) * H);
#pragma unroll
    for (int t = 0; t < LT; t++)
        xr[t] = reinterpret_cast<const float4 *>(x + (size_t)min(t0 + t, N - 1) * H);

    constexpr int UNR = LE * LT > 8 ? 1 : 4;
#pragma unroll UNR
    for (int i = 0; i < H / 256; i++) {
        float4 w[LE], xv[LT];
#pragma unroll
        for (int e = 0; e < LE; e++) w[e] = wr[e][i * 64 + lane];
#pragma unroll
        for (int t = 0; t < LT; t++) xv[t] = xr[t][i * 64 + lane];
#pragma unroll
        for (int t = 0; t < LT; t++)
#pragma unroll
            for (int e = 0; e < LE; e++) {
                float a = acc[t][e];
                a = __builtin_fmaf(w[e].x, xv[t].x, a);
                a = __builtin_fmaf(w[e].y, xv[t].y, a);
                a = __builtin_fmaf(w[e].z, xv[t].z, a);
                a = __builtin_fmaf(w[e].w, xv[t].w, a);
                acc[t][e] = a;
            }
    }
    float mine = 0.0f;
#pragma unroll
    for (int t = 0; t < LT; t++)
#pragma unroll
        for (int e = 0; e < LE; e++) {
            float v = acc[t][e];
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
            if (lane == t * LE + e) mine = v;
        }
    const int t = lane / LE, e = lane % LE;
    if (lane < LT * LE && t0 + t < N && e0 + e < E) {
        const size_t o = (size_t)(t0 + t) * E + e0 + e;
        const float p = sigmoid_f32(mine);
        rb.logits[o] = mine;
        rb.probs[o] = p;
        rb.sel[o] = bias ? p + bias[e0 + e] : p;
    }
}

// logit wavefronts of a launch (wide: the 8 x 8 tiles)
__host__ __device__ __forceinline__ int logit_waves(int N, int E, bool wide)
{
    return wide ? ((E + LW_E - 1) / LW_E) * ((N + LW_T - 1) / LW_T)
                : ((E + LG_E - 1) / LG_E) * ((N + LG_T - 1) / LG_T);
}

__device__ __forceinline__ int prep_blocks(const PrepJob &j)
{
    return (j.rows * (j.K / 256) + 3) / 4;
}

struct FrontArgs {
    const float *W, *bias, *x;
    int N, H, E, logit_blocks, wide;
    RouteBufs rb;
    PrepJob job[2];
    int njobs;
};

__global__ __launch_bounds__(256) void k_front(FrontArgs a)
{
    __shared__ float s_v[4][256];
    const int w = threadIdx.x >> 6;
    int b = blockIdx.x;
    if (b < a.logit_blocks) {
        const int wave = b * 4 + w;
        if (wave < logit_waves(a.N, a.E, a.wide)) {
            if (a.wide)
                logits_wave<LW_E, LW_T>(a.W, a.bias, a.x, a.N, a.H, a.E, wave, a.rb);
            else
                logits_wave<LG_E, LG_T>(a.W, a.bias, a.x, a.N, a.H, a.E, wave, a.rb);
        }
        return;
    }
    b -= a.logit_blocks;
    for (int j = 0; j < a.njobs; j++) {
        const int nb = prep_blocks(a.job[j]);
        if (b < nb) {
            const int wid = b * 4 + w;
            if (wid < a.job[j].rows * (a.job[j].K / 256)) prep_wave(a.job[j], wid, s_v[w]);
            return;
        }
        b -= nb;
    }
}

hipError_t launch_front(const float *W, const float *bias, const float *x, int N, int H, int E,
                        const RouteBufs &rb, const PrepJob *jobs, int njobs, hipStream_t s)
{
    FrontArgs a{};
    a.W = W;
    a.bias = bias;
    a.x = x;
    a.N = N;
    a.H = H;
    a.E = E;
    a.rb = rb;
    a.wide = N >= 256;
    a.logit_blocks = (logit_waves(N, E, a.wide) + 3) / 4;
    int blocks = a.logit_blocks;
    a.njobs = njobs;
    for (int j = 0; j < njobs; j++) {
        if (jobs[j].K % 256) return hipErrorInvalidValue;
        a.job[j] = jobs[j];
        blocks += (jobs[j].rows * (jobs[j].K / 256) + 3) / 4;
    }
    hipLaunchKernelGGL(k_front, dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

struct PrepArgs {
    PrepJob job[2];
    int njobs;
};

__global__ __launch_bounds__(256) void k_prep(PrepArgs a)
{
    __shared__ float s_v[4][256];
    const int w = threadIdx.x >> 6;
    int b = blockIdx.x;
    for (int j = 0; j < a.njobs; j++) {
        const int nb = prep_blocks(a.job[j]);
        if (b < nb) {
            const int wid = b * 4 + w;
            if (wid < a.job[j].rows * (a.job[j].K / 256)) prep_wave(a.job[j], wid, s_v[w]);
            return;
        }
        b -= nb;
    }
}

hipError_t launch_prep(const PrepJob *jobs, int njobs, hipStream_t s)
{
    PrepArgs a{};
    a.njobs = njobs;
    int blocks = 0;
    for (int j = 0; j < njobs; j++) {
        if (jobs[j].K % 256 || jobs[j].rows <= 0) return hipErrorInvalidValue;
        a.job[j] = jobs[j];
        blocks += (jobs[j].rows * (jobs[j].K / 256) + 3) / 4;
    }
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_prep, dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

// probs and sel from given logits
__global__ __launch_bounds__(256) void k_scores(const float *__restrict__ logits,
                                                const float *__restrict__ bias, int N, int E,
                                                RouteBufs rb)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)N * E) return;
    const float p = sigmoid_f32(logits[i]);
    rb.probs[i] = p;
    rb.sel[i] = bias ? p + bias[i % E] : p;
}

hipError_t launch_scores(const float *logits, const float *bias, int N, int E,
                         const RouteBufs &rb, hipStream_t s)
{
    const size_t total = (size_t)N * E;
    hipLaunchKernelGGL(k_scores, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, logits,
                       bias, N, E, rb);
    return hipGetLastError();
}

} // namespace dmoe
