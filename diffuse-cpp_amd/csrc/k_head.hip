// k_head.hip — per-position argmax and confidence of the LM-head logits
// (the temperature-0 branch of sample_token, src/diffuse-sampler.cpp:29-49).
//
// Two launches so that a row of a large vocabulary spreads over many
// workgroups (32 positions of 157184 logits are 1248 chunks, not 32 rows).
//
// k_argmax_part: one workgroup per chunk of AP_CHUNK logits of a row, held in
// registers.  Its argmax: each thread's values in ascending index order keep
// the first of equal maxima (a NaN never compares greater), then the
// threads' (value, index) pairs combine by xor butterflies in each
// wavefront and the wavefronts' results in wavefront order, larger value
// first, lower index on ties.  Its exp-sum s_c = sum exp(l - m_c) over the
// chunk, about the chunk's own maximum m_c (0 when the chunk holds no value
// above -inf, so that its -inf logits add 0 and a NaN still adds NaN), each
// term 2^((l - m_c) log2 e) by the hardware exp2 in binary32 (a few ulp of
// the exact value; the correctly rounded binary32 exp through binary64 made
// the launch VALU bound at twice the time), each thread adding its terms in
// binary64 and the partials in the same fixed order.
//
// k_argmax_final: one wave per row combines the chunks in the same rule (the
// first index of the largest; every logit -inf, or a NaN logits[0], gives
// index 0 and that value, as the reference's loop which starts from
// logits[0]) and rescales each chunk's sum to the row maximum M in binary64:
// sum = sum_c s_c exp(m_c - M), added in a fixed tree, confidence 1 / sum.
// Up to the rounding of the binary64 additions and of exp(m_c - M) this is
// sum_v exp(l_v - M) (the reference adds float expf terms sequentially; the
// two differ by that float accumulation's rounding), and the NaN / infinity
// cases come out as the reference's: NaN whenever one of its terms is.
#include "dmoe_device.h"

namespace dmoe {

constexpr int AP_THREADS = 256;
constexpr int AP_WAVES = AP_THREADS / 64;
constexpr int AP_PER = 16;                                 // logits per thread
constexpr int AP_CHUNK = AP_THREADS * AP_PER;              // logits per workgroup

size_t argmax_partials_bytes(int N, int V)
{
    return (size_t)N * ((V + AP_CHUNK - 1) / AP_CHUNK) * sizeof(ArgmaxPart);
}

// larger value first, lower index on ties (NaN never wins a comparison)
__device__ __forceinline__ bool ap_better(float b, int ib, float a, int ia)
{
    return b > a || (b == a && ib < ia);
}

// The chunk's reductions run in registers: xor butterflies inside each
// wavefront (rounds 32 .. 1), then the four wavefronts' results combined by
// one thread in wavefront order, so a chunk costs two barriers.
__global__ __launch_bounds__(AP_THREADS) void k_argmax_part(const float *__restrict__ logits, int V, int C,
                                                            ArgmaxPart *__restrict__ part)
{
#pragma clang fp contract(off)
    __shared__ float s_v[AP_WAVES];
    __shared__ int s_i[AP_WAVES];
    __shared__ double s_d[AP_WAVES];
    __shared__ float s_mc;
    const int c = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const float *row = logits + (size_t)t * V;
    const int v0 = c * AP_CHUNK;
    float l[AP_PER];
#pragma unroll
    for (int k = 0; k < AP_PER; k++) {
        const int v = v0 + k * AP_THREADS + tid;
        l[k] = v < V ? row[v] : -__builtin_inff();
    }
    float m = -__builtin_inff();
    int mi = V;                                            // none yet
#pragma unroll
    for (int k = 0; k < AP_PER; k++)
        if (l[k] > m) {
            m = l[k];
            mi = v0 + k * AP_THREADS + tid;
        }
#pragma unroll
    for (int r = 32; r >= 1; r >>= 1) {
        const float om = __shfl_xor(m, r, 64);
        const int oi = __shfl_xor(mi, r, 64);
        if (ap_better(om, oi, m, mi)) {
            m = om;
            mi = oi;
        }
    }
    if (lane == 0) {
        s_v[wave] = m;
        s_i[wave] = mi;
    }
    __syncthreads();
    if (tid == 0) {
        float bm = s_v[0];
        int bi = s_i[0];
        for (int w = 1; w < AP_WAVES; w++)
            if (ap_better(s_v[w], s_i[w], bm, bi)) {
                bm = s_v[w];
                bi = s_i[w];
            }
        s_mc = bm;
        s_i[0] = bi;
    }
    __syncthreads();
    const float mc = s_mc;
    const float base = mc == -__builtin_inff() ? 0.0f : mc;
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < AP_PER; k++)
        if (v0 + k * AP_THREADS + tid < V)
            acc += (double)__builtin_amdgcn_exp2f((l[k] - base) * 1.44269504088896341f);
#pragma unroll
    for (int r = 32; r >= 1; r >>= 1) acc = acc + __shfl_xor(acc, r, 64);
    if (lane == 0) s_d[wave] = acc;
    __syncthreads();
    if (tid == 0) {
        double sum = s_d[0];
        for (int w = 1; w < AP_WAVES; w++) sum = sum + s_d[w];
        ArgmaxPart p;
        p.m = mc;
        p.idx = s_i[0];
        p.sum = sum;
        part[(size_t)t * C + c] = p;
    }
}

constexpr int AF_THREADS = 64;

__global__ __launch_bounds__(AF_THREADS) void k_argmax_final(const float *__restrict__ logits, int V, int C,
                                                             const ArgmaxPart *__restrict__ part,
                                                             int32_t *__restrict__ tokens,
                                                             float *__restrict__ probs)
{
#pragma clang fp contract(off)
    __shared__ float s_v[AF_THREADS];
    __shared__ int s_i[AF_THREADS];
    __shared__ double s_d[AF_THREADS];
    const int t = blockIdx.x, tid = threadIdx.x;
    const ArgmaxPart *p = part + (size_t)t * C;
    float m = -__builtin_inff();
    int mi = V;
    for (int c = tid; c < C; c += AF_THREADS)             // ascending chunks: first index kept
        if (ap_better(p[c].m, p[c].idx, m, mi)) {
            m = p[c].m;
            mi = p[c].idx;
        }
    s_v[tid] = m;
    s_i[tid] = mi;
    __syncthreads();
    for (int w = AF_THREADS / 2; w > 0; w >>= 1) {
        if (tid < w && ap_better(s_v[tid + w], s_i[tid + w], s_v[tid], s_i[tid])) {
            s_v[tid] = s_v[tid + w];
            s_i[tid] = s_i[tid + w];
        }
        __syncthreads();
    }
    const float first = logits[(size_t)t * V];
    int best = s_i[0];
    float best_val = s_v[0];
    if (best == V || first != first) {
        best = 0;
        best_val = first;
    }
    double acc = 0.0;
    for (int c = tid; c < C; c += AF_THREADS) {
        const float mc = p[c].m;
        // exp(m_c - M): 0 for a chunk of -inf logits; below e^-700 the
        // chunk adds nothing a binary32 result can hold (M's own chunk adds
        // at least 1)
        double d = (double)mc - (double)best_val;
        d = d < -700.0 ? -700.0 : d;
        const double scale = mc == -__builtin_inff() && best_val == best_val && best_val != -__builtin_inff()
                                 ? 0.0
                                 : exp_f64(d);
        acc += p[c].sum * scale;
    }
    s_d[tid] = acc;
    __syncthreads();
    for (int w = AF_THREADS / 2; w > 0; w >>= 1) {
        if (tid < w) s_d[tid] = s_d[tid] + s_d[tid + w];
        __syncthreads();
    }
    if (tid == 0) {
        tokens[t] = best;
        probs[t] = 1.0f / (float)s_d[0];
    }
}

hipError_t launch_argmax_prob(const float *logits, int N, int V, ArgmaxPart *part, int32_t *tokens,
                              float *probs, hipStream_t s)
{
    if (N <= 0 || V <= 0 || N > 65535) return hipErrorInvalidValue;
    const int C = (V + AP_CHUNK - 1) / AP_CHUNK;
    hipLaunchKernelGGL(k_argmax_part, dim3(C, N), dim3(AP_THREADS), 0, s, logits, V, C, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3(N), dim3(AF_THREADS), 0, s, logits, V, C, part, tokens, probs);
    return hipGetLastError();
}

} // namespace dmoe
