// k_router.hip — router stages of the MoE segment on gfx950.
//
//   router_logits : L = Wg x in one fixed fp32 summation order
//                   (src/diffuse-moe-graph.cpp:203)
//   route         : sigmoid, selection bias, per-block max fold, capacity
//                   threshold, allowed mask, per-token top-k, gate weights
//                   (src/diffuse-moe-graph.cpp:204-262)
//   dispatch      : stable grouping of (token, slot) pairs by expert — the
//                   row grouping ggml_mul_mat_id performs (:266-269)
//
// Bit-exactness: every float operation here is a single IEEE operation in a
// fixed order (no contraction: see the pragma), exp is evaluated in binary64
// from add/mul/fma/rint only, and division is the correctly rounded one, so
// the results do not depend on thread scheduling.
#include "dmoe_internal.h"

#pragma clang fp contract(off)

namespace dmoe {

// ---------------------------------------------------------------------------
// exp(x) in binary64 rounded once to binary32.  Cody-Waite reduction
// x = k ln2 + r (ln2 split into a 32-significant-bit head and a tail, so k*head
// is exact), exp(r) by its degree-13 Taylor polynomial in Horner form with
// fma, then scaling by 2^k through the exponent field.
__device__ __forceinline__ double exp_f64(double x)
{
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
    if (x != x) return x;
    // exp(100) overflows binary32 and exp(-110) rounds to 0: clamping keeps
    // every result and keeps k in the normal binary64 exponent range.
    x = x > 100.0f ? 100.0f : x;
    x = x < -110.0f ? -110.0f : x;
    return (float)exp_f64((double)x);
}

// ggml_sigmoid, :204
__device__ __forceinline__ float sigmoid_f32(float x)
{
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

// ---------------------------------------------------------------------------
// Router logits.  One wavefront per (expert, chunk of 8 tokens).  Lane l keeps
// one partial per token:  a_l = fma(W[k], x[k], a_l) for k = 256*i + 4*l + j,
// i ascending then j = 0..3; the 64 partials are then combined by six xor
// butterfly rounds (m = 32..1).  Every lane ends with the same value because
// each round adds the same two operands in both partner lanes.
constexpr int LOGIT_TOK = 8;

__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ W,
                                                       const float *__restrict__ x, int N,
                                                       int H, int E, float *__restrict__ logits)
{
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nchunk = (N + LOGIT_TOK - 1) / LOGIT_TOK;
    if (wave >= E * nchunk) return;
    const int e = wave % E;
    const int t0 = (wave / E) * LOGIT_TOK;
    const int nt = min(LOGIT_TOK, N - t0);

    float acc[LOGIT_TOK];
#pragma unroll
    for (int t = 0; t < LOGIT_TOK; t++) acc[t] = 0.0f;

    const float4 *wrow = reinterpret_cast<const float4 *>(W + (size_t)e * H);
    for (int i = 0; i < H / 256; i++) {
        const float4 w = wrow[i * 64 + lane];
#pragma unroll
        for (int t = 0; t < LOGIT_TOK; t++) {
            if (t < nt) {
                const float4 xv =
                    reinterpret_cast<const float4 *>(x + (size_t)(t0 + t) * H)[i * 64 + lane];
                float a = acc[t];
                a = __builtin_fmaf(w.x, xv.x, a);
                a = __builtin_fmaf(w.y, xv.y, a);
                a = __builtin_fmaf(w.z, xv.z, a);
                a = __builtin_fmaf(w.w, xv.w, a);
                acc[t] = a;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < LOGIT_TOK; t++) {
        float v = acc[t];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
        if (lane == t && t < nt) logits[(size_t)(t0 + t) * E + e] = v;
    }
}

hipError_t launch_router_logits(const float *W, const float *x, int N, int H, int E,
                                float *logits, hipStream_t s)
{
    const int nchunk = (N + LOGIT_TOK - 1) / LOGIT_TOK;
    const int waves = E * nchunk;
    hipLaunchKernelGGL(k_router_logits, dim3((waves + 3) / 4), dim3(256), 0, s, W, x, N, H, E,
                       logits);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Routing.  One workgroup per routing group: a block of block_size tokens when
// block routing is on, otherwise a chunk of 32 tokens.  Selection scores are
// recomputed from the logits where needed (a pure function), so no thread
// reads another thread's global writes.
constexpr int MAX_E = 1024;     // experts per layer supported by this kernel
constexpr int MAX_K = 32;       // top_k supported by this kernel

__device__ __forceinline__ float sel_score(const float *logits, const float *bias, int t, int e,
                                           int E)
{
    float p = sigmoid_f32(logits[(size_t)t * E + e]);
    return bias ? p + bias[e] : p;     // :207-210
}

__global__ __launch_bounds__(256) void k_route(RouteParams rp, const float *__restrict__ logits,
                                               const float *__restrict__ bias, RouteBufs rb)
{
    __shared__ float s_bmax[MAX_E];
    __shared__ uint32_t s_key[MAX_E];
    __shared__ float s_add[MAX_E];
    __shared__ float s_thr;

    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int g = blockIdx.x;
    const int t0 = g * G;
    const int t1 = min(N, t0 + G);
    const int tid = threadIdx.x;

    // probs for the group's tokens (:204), for the caller's debug copy and the
    // gate weights
    for (int i = tid; i < (t1 - t0) * E; i += blockDim.x) {
        const int t = t0 + i / E, e = i % E;
        rb.probs[(size_t)t * E + e] = sigmoid_f32(logits[(size_t)t * E + e]);
    }

    if (rp.use_block) {
        // :223-229  bmax = s_0 folded with m <- s_j + relu(m - s_j), j = 1..blk-1
        for (int e = tid; e < E; e += blockDim.x) {
            float m = sel_score(logits, bias, t0, e, E);
            for (int j = 1; j < G; j++) {
                const float sj = sel_score(logits, bias, t0 + j, e, E);
                float r = m - sj;
                r = r > 0.0f ? r : 0.0f;          // ggml_relu
                m = sj + r;
            }
            s_bmax[e] = m;
            s_key[e] = order_key(m);
        }
        __syncthreads();
        // :232-236  thr = the cap-th largest bmax (position cap-1 of the
        // descending order); exactly one expert has that rank.
        for (int e = tid; e < E; e += blockDim.x) {
            const uint32_t ke = s_key[e];
            int rank = 0;
            for (int f = 0; f < E; f++) rank += (f != e) && ranks_before(s_key[f], f, ke, e);
            if (rank == rp.capacity - 1) s_thr = s_bmax[e];
        }
        __syncthreads();
        // :241-243  keep = step(bmax - (thr + -1e-6)); additive 0 / -1e30
        const float th = s_thr;
        const float tp = th + (-1e-6f);
        for (int e = tid; e < E; e += blockDim.x) {
            const float diff = s_bmax[e] - tp;
            const int keep = diff > 0.0f;
            s_add[e] = (float)keep * 1e30f + (-1e30f);
            rb.bmax[(size_t)g * E + e] = s_bmax[e];
            rb.allowed[(size_t)g * E + e] = (uint8_t)keep;
        }
        if (tid == 0) rb.thr[g] = th;
        __syncthreads();
    }

    // :252  per-token top-k of sel' = s + mask; one wavefront per token.
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    const int ncand = (E + 63) / 64;
    for (int t = t0 + wave; t < t1; t += nwaves) {
        uint32_t key[MAX_E / 64];
        bool taken[MAX_E / 64];
        for (int c = 0; c < ncand; c++) {
            const int e = lane + 64 * c;
            taken[c] = e >= E;
            key[c] = 0u;
            if (e < E) {
                float s = sel_score(logits, bias, t, e, E);
                if (rp.use_block) s = s + s_add[e];   // :248
                key[c] = order_key(s);
            }
        }
        int chosen[MAX_K];
        for (int slot = 0; slot < K; slot++) {
            // best candidate of this lane
            uint64_t best = 0;
            for (int c = 0; c < ncand; c++) {
                if (taken[c]) continue;
                const int e = lane + 64 * c;
                const uint64_t v = ((uint64_t)key[c] << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
                best = v > best ? v : best;
            }
            // wavefront max: larger key first, then the lower expert id
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                const uint32_t lo = __shfl_xor((uint32_t)best, m, 64);
                const uint32_t hi = __shfl_xor((uint32_t)(best >> 32), m, 64);
                const uint64_t o = ((uint64_t)hi << 32) | lo;
                best = o > best ? o : best;
            }
            const int e = (int)(0xffffffffu - (uint32_t)best);
            chosen[slot] = e;
            if ((e & 63) == lane) taken[e >> 6] = true;
        }
        if (lane == 0) {
            // :253-262  w = probs[idx]; w /= sum (binary64 row sum); w *= scale
            float w[MAX_K];
            for (int s = 0; s < K; s++) w[s] = sigmoid_f32(logits[(size_t)t * E + chosen[s]]);
            if (rp.norm_topk_prob) {
                double acc = 0.0;
                for (int s = 0; s < K; s++) acc += (double)w[s];
                const float S = (float)acc;
                for (int s = 0; s < K; s++) w[s] = w[s] / S;
            }
            if (rp.routed_scaling != 1.0f)
                for (int s = 0; s < K; s++) w[s] = w[s] * rp.routed_scaling;
            for (int s = 0; s < K; s++) {
                rb.idx[(size_t)t * K + s] = chosen[s];
                rb.weights[(size_t)t * K + s] = w[s];
            }
        }
    }
}

hipError_t launch_route(const RouteParams &rp, const float *logits, const float *bias,
                        const RouteBufs &rb, hipStream_t s)
{
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (rp.n_tokens + G - 1) / G;
    hipLaunchKernelGGL(k_route, dim3(ngroups), dim3(256), 0, s, rp, logits, bias, rb);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dispatch: counts[e], offsets[e] (exclusive scan) and perm (pair ids grouped
// by expert, ascending pair id inside each expert).  One workgroup; each
// thread owns experts e = tid, tid + blockDim, ... and scans the pair list,
// staged in LDS, in ascending order — no atomics, so the result is fixed.
constexpr int DISP_THREADS = 1024;
constexpr int DISP_CHUNK = 8192;

__global__ __launch_bounds__(DISP_THREADS) void k_dispatch(RouteParams rp, RouteBufs rb)
{
    __shared__ int32_t s_idx[DISP_CHUNK];
    __shared__ int32_t s_cnt[MAX_E];
    const int E = rp.n_experts;
    const int P = rp.n_tokens * rp.top_k;
    const int tid = threadIdx.x;

    int cnt[MAX_E / DISP_THREADS + 1];
    for (int c = 0; c * DISP_THREADS < E; c++) cnt[c] = 0;
    for (int base = 0; base < P; base += DISP_CHUNK) {
        const int n = min(DISP_CHUNK, P - base);
        __syncthreads();
        for (int i = tid; i < n; i += DISP_THREADS) s_idx[i] = rb.idx[base + i];
        __syncthreads();
        for (int c = 0; c * DISP_THREADS < E; c++) {
            const int e = tid + c * DISP_THREADS;
            if (e >= E) break;
            int k = 0;
            for (int i = 0; i < n; i++) k += s_idx[i] == e;
            cnt[c] += k;
        }
    }
    for (int c = 0; c * DISP_THREADS < E; c++) {
        const int e = tid + c * DISP_THREADS;
        if (e < E) s_cnt[e] = cnt[c];
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < E; e++) {
            const int k = s_cnt[e];
            rb.counts[e] = k;
            rb.offsets[e] = run;
            s_cnt[e] = run;
            run += k;
        }
        rb.offsets[E] = run;
    }
    __syncthreads();
    int pos[MAX_E / DISP_THREADS + 1];
    for (int c = 0; c * DISP_THREADS < E; c++) {
        const int e = tid + c * DISP_THREADS;
        pos[c] = e < E ? s_cnt[e] : 0;
    }
    for (int base = 0; base < P; base += DISP_CHUNK) {
        const int n = min(DISP_CHUNK, P - base);
        __syncthreads();
        for (int i = tid; i < n; i += DISP_THREADS) s_idx[i] = rb.idx[base + i];
        __syncthreads();
        for (int c = 0; c * DISP_THREADS < E; c++) {
            const int e = tid + c * DISP_THREADS;
            if (e >= E) break;
            int p = pos[c];
            for (int i = 0; i < n; i++)
                if (s_idx[i] == e) rb.perm[p++] = base + i;
            pos[c] = p;
        }
    }
}

hipError_t launch_dispatch(const RouteParams &rp, const RouteBufs &rb, hipStream_t s)
{
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(DISP_THREADS), 0, s, rp, rb);
    return hipGetLastError();
}

} // namespace dmoe
