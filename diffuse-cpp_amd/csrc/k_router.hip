// k_router.hip — router stages of the MoE segment on gfx950.
//
//   router_logits : L = Wg x in one fixed fp32 summation order
//                   (src/diffuse-moe-graph.cpp:203)
//   route         : sigmoid, selection bias, per-block max fold, capacity
//                   threshold, allowed mask, per-token top-k, gate weights
//                   (src/diffuse-moe-graph.cpp:204-262), plus each routing
//                   group's expert histogram and the local rank of its pairs
//   dispatch      : stable grouping of (token, slot) pairs by expert — the
//                   row grouping ggml_mul_mat_id performs (:266-269) — and the
//                   work list of the expert kernels
//
// Bit-exactness: every float operation here is a single IEEE operation in a
// fixed order (no contraction: see the pragma), exp is evaluated in binary64
// from add/mul/fma/rint only, and division is the correctly rounded one, so
// the results do not depend on thread scheduling.  Counts and ranks are
// computed without atomics.
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
// Router logits.  One wavefront per (4 experts, 4 tokens).  For every
// (token, expert) lane l keeps one partial:  a_l = fma(W[k], x[k], a_l) for
// k = 256*i + 4*l + j, i ascending then j = 0..3; the 64 partials are then
// combined by six xor butterfly rounds (m = 32..1).  Every lane ends with the
// same value because each round adds the same two operands in both partners.
constexpr int LG_E = 4, LG_T = 4;

__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ W,
                                                       const float *__restrict__ x, int N,
                                                       int H, int E, float *__restrict__ logits)
{
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ne = (E + LG_E - 1) / LG_E;
    const int nt = (N + LG_T - 1) / LG_T;
    if (wave >= ne * nt) return;
    const int e0 = (wave % ne) * LG_E;
    const int t0 = (wave / ne) * LG_T;

    float acc[LG_T][LG_E];
#pragma unroll
    for (int t = 0; t < LG_T; t++)
#pragma unroll
        for (int e = 0; e < LG_E; e++) acc[t][e] = 0.0f;

    const float4 *wr[LG_E];
    const float4 *xr[LG_T];
#pragma unroll
    for (int e = 0; e < LG_E; e++)
        wr[e] = reinterpret_cast<const float4 *>(W + (size_t)min(e0 + e, E - 1) * H);
#pragma unroll
    for (int t = 0; t < LG_T; t++)
        xr[t] = reinterpret_cast<const float4 *>(x + (size_t)min(t0 + t, N - 1) * H);

    for (int i = 0; i < H / 256; i++) {
        float4 w[LG_E], xv[LG_T];
#pragma unroll
        for (int e = 0; e < LG_E; e++) w[e] = wr[e][i * 64 + lane];
#pragma unroll
        for (int t = 0; t < LG_T; t++) xv[t] = xr[t][i * 64 + lane];
#pragma unroll
        for (int t = 0; t < LG_T; t++)
#pragma unroll
            for (int e = 0; e < LG_E; e++) {
                float a = acc[t][e];
                a = __builtin_fmaf(w[e].x, xv[t].x, a);
                a = __builtin_fmaf(w[e].y, xv[t].y, a);
                a = __builtin_fmaf(w[e].z, xv[t].z, a);
                a = __builtin_fmaf(w[e].w, xv[t].w, a);
                acc[t][e] = a;
            }
    }
#pragma unroll
    for (int t = 0; t < LG_T; t++)
#pragma unroll
        for (int e = 0; e < LG_E; e++) {
            float v = acc[t][e];
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
            if (lane == t * LG_E + e && t0 + t < N && e0 + e < E)
                logits[(size_t)(t0 + t) * E + e0 + e] = v;
        }
}

hipError_t launch_router_logits(const float *W, const float *x, int N, int H, int E,
                                float *logits, hipStream_t s)
{
    const int waves = ((E + LG_E - 1) / LG_E) * ((N + LG_T - 1) / LG_T);
    hipLaunchKernelGGL(k_router_logits, dim3((waves + 3) / 4), dim3(256), 0, s, W, x, N, H, E,
                       logits);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Routing.  One workgroup per routing group: a block of block_size tokens when
// block routing is on, otherwise a chunk of 32 tokens.  The group's selection
// scores live in LDS (group tokens x experts <= ROUTE_LDS floats).
constexpr int MAX_E = 1024;     // experts per layer supported by these kernels
constexpr int MAX_K = 32;       // top_k supported by these kernels
constexpr int ROUTE_THREADS = 512;
constexpr int NCAND = MAX_E / 64;

__global__ __launch_bounds__(ROUTE_THREADS) void k_route(RouteParams rp,
                                                         const float *__restrict__ logits,
                                                         const float *__restrict__ bias,
                                                         RouteBufs rb)
{
    __shared__ float s_sel[ROUTE_LDS];
    __shared__ float s_bmax[MAX_E];
    __shared__ uint32_t s_key[MAX_E];
    __shared__ float s_add[MAX_E];
    __shared__ int32_t s_idx[ROUTE_LDS / 8];      // group pairs (tokens x slots)
    __shared__ float s_thr;

    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int g = blockIdx.x;
    const int t0 = g * G;
    const int nt = min(N, t0 + G) - t0;
    const int tid = threadIdx.x;

    // :204 probs (written for the debug copy), :207-210 sel = probs + bias
    for (int i = tid; i < nt * E; i += ROUTE_THREADS) {
        const int t = i / E, e = i - t * E;
        const float p = sigmoid_f32(logits[(size_t)(t0 + t) * E + e]);
        rb.probs[(size_t)(t0 + t) * E + e] = p;
        s_sel[i] = bias ? p + bias[e] : p;
    }
    __syncthreads();

    if (rp.use_block) {
        // :223-229  bmax = s_0 folded with m <- s_j + relu(m - s_j), j = 1..blk-1
        for (int e = tid; e < E; e += ROUTE_THREADS) {
            float m = s_sel[e];
            for (int j = 1; j < G; j++) {
                const float sj = s_sel[j * E + e];
                float r = m - sj;
                r = r > 0.0f ? r : 0.0f;          // ggml_relu
                m = sj + r;
            }
            s_bmax[e] = m;
            s_key[e] = order_key(m);
        }
        __syncthreads();
        // :232-236  thr = the cap-th largest bmax (position cap-1 of the
        // descending order); exactly one expert has that rank
        for (int e = tid; e < E; e += ROUTE_THREADS) {
            const uint32_t ke = s_key[e];
            int rank = 0;
            for (int f = 0; f < E; f++) rank += ranks_before(s_key[f], f, ke, e);
            if (rank == rp.capacity - 1) s_thr = s_bmax[e];
        }
        __syncthreads();
        // :241-243  keep = step(bmax - (thr + -1e-6)); additive 0 / -1e30
        const float th = s_thr;
        const float tp = th + (-1e-6f);
        for (int e = tid; e < E; e += ROUTE_THREADS) {
            const float diff = s_bmax[e] - tp;
            const int keep = diff > 0.0f;
            s_add[e] = (float)keep * 1e30f + (-1e30f);
            rb.bmax[(size_t)g * E + e] = s_bmax[e];
            rb.allowed[(size_t)g * E + e] = (uint8_t)keep;
        }
        if (tid == 0) rb.thr[g] = th;
        __syncthreads();
    }

    // :252  per-token top-k of sel' = s + mask; one wavefront per token
    const int lane = tid & 63;
    const int wave = tid >> 6;
    for (int t = wave; t < nt; t += ROUTE_THREADS / 64) {
        uint32_t key[NCAND];
#pragma unroll
        for (int c = 0; c < NCAND; c++) {
            const int e = lane + 64 * c;
            key[c] = 0u;
            if (e < E) {
                float s = s_sel[t * E + e];
                if (rp.use_block) s = s + s_add[e];       // :248
                key[c] = order_key(s) | 0u;
            }
        }
        uint32_t taken = 0;        // bit c: candidate lane + 64c already chosen
        int mine = -1;             // expert chosen for slot `lane`
        for (int slot = 0; slot < K; slot++) {
            uint64_t best = 0;
#pragma unroll
            for (int c = 0; c < NCAND; c++) {
                const int e = lane + 64 * c;
                if (e >= E || (taken >> c) & 1u) continue;
                const uint64_t v = ((uint64_t)key[c] << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
                best = v > best ? v : best;
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                const uint32_t lo = __shfl_xor((uint32_t)best, m, 64);
                const uint32_t hi = __shfl_xor((uint32_t)(best >> 32), m, 64);
                const uint64_t o = ((uint64_t)hi << 32) | lo;
                best = o > best ? o : best;
            }
            const int e = (int)(0xffffffffu - (uint32_t)best);
            if ((e & 63) == lane) taken |= 1u << (e >> 6);
            if (lane == slot) mine = e;
        }
        // :253-262  w = probs[idx]; w /= sum (binary64 row sum); w *= scale
        float w = 0.0f;
        if (lane < K) w = sigmoid_f32(logits[(size_t)(t0 + t) * E + mine]);
        double acc = 0.0;
        for (int s = 0; s < K; s++) acc += (double)__shfl(w, s, 64);
        if (lane < K) {
            if (rp.norm_topk_prob) w = w / (float)acc;
            if (rp.routed_scaling != 1.0f) w = w * rp.routed_scaling;
            rb.idx[(size_t)(t0 + t) * K + lane] = mine;
            rb.weights[(size_t)(t0 + t) * K + lane] = w;
            s_idx[t * K + lane] = mine;
        }
    }
    __syncthreads();

    // group histogram and the rank of each pair among the group's pairs of the
    // same expert (pairs in t-major, slot-minor order)
    const int np = nt * K;
    for (int e = tid; e < E; e += ROUTE_THREADS) {
        int c = 0;
        for (int j = 0; j < np; j++) c += s_idx[j] == e;
        rb.hist[(size_t)g * E + e] = c;
    }
    for (int j = tid; j < np; j += ROUTE_THREADS) {
        const int e = s_idx[j];
        int r = 0;
        for (int i = 0; i < j; i++) r += s_idx[i] == e;
        rb.lrank[(size_t)t0 * K + j] = r;
    }
}

// General-shape routing (groups too large for LDS): selection scores are
// recomputed from the logits where needed; each token's top-k is serial.
__global__ __launch_bounds__(256) void k_route_general(RouteParams rp,
                                                       const float *__restrict__ logits,
                                                       const float *__restrict__ bias,
                                                       RouteBufs rb)
{
    __shared__ float s_bmax[MAX_E];
    __shared__ uint32_t s_key[MAX_E];
    __shared__ float s_add[MAX_E];
    __shared__ float s_thr;
    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int g = blockIdx.x, t0 = g * G, t1 = min(N, t0 + G), tid = threadIdx.x;
    auto sel = [&](int t, int e) {
        const float p = sigmoid_f32(logits[(size_t)t * E + e]);
        return bias ? p + bias[e] : p;
    };
    for (int i = tid; i < (t1 - t0) * E; i += blockDim.x) {
        const int t = t0 + i / E, e = i % E;
        rb.probs[(size_t)t * E + e] = sigmoid_f32(logits[(size_t)t * E + e]);
    }
    if (rp.use_block) {
        for (int e = tid; e < E; e += blockDim.x) {
            float m = sel(t0, e);
            for (int j = 1; j < G; j++) {
                const float sj = sel(t0 + j, e);
                float r = m - sj;
                r = r > 0.0f ? r : 0.0f;
                m = sj + r;
            }
            s_bmax[e] = m;
            s_key[e] = order_key(m);
        }
        __syncthreads();
        for (int e = tid; e < E; e += blockDim.x) {
            int rank = 0;
            for (int f = 0; f < E; f++) rank += ranks_before(s_key[f], f, s_key[e], e);
            if (rank == rp.capacity - 1) s_thr = s_bmax[e];
        }
        __syncthreads();
        const float th = s_thr, tp = th + (-1e-6f);
        for (int e = tid; e < E; e += blockDim.x) {
            const int keep = (s_bmax[e] - tp) > 0.0f;
            s_add[e] = (float)keep * 1e30f + (-1e30f);
            rb.bmax[(size_t)g * E + e] = s_bmax[e];
            rb.allowed[(size_t)g * E + e] = (uint8_t)keep;
        }
        if (tid == 0) rb.thr[g] = th;
        __syncthreads();
    }
    for (int t = t0 + tid; t < t1; t += blockDim.x) {
        int chosen[MAX_K];
        for (int s = 0; s < K; s++) {
            int best = -1;
            uint32_t bk = 0;
            for (int e = 0; e < E; e++) {
                bool taken = false;
                for (int q = 0; q < s; q++) taken |= chosen[q] == e;
                if (taken) continue;
                float v = sel(t, e);
                if (rp.use_block) v = v + s_add[e];
                const uint32_t k = order_key(v);
                if (best < 0 || ranks_before(k, e, bk, best)) { best = e; bk = k; }
            }
            chosen[s] = best;
        }
        float w[MAX_K];
        double acc = 0.0;
        for (int s = 0; s < K; s++) {
            w[s] = sigmoid_f32(logits[(size_t)t * E + chosen[s]]);
            acc += (double)w[s];
        }
        for (int s = 0; s < K; s++) {
            float v = w[s];
            if (rp.norm_topk_prob) v = v / (float)acc;
            if (rp.routed_scaling != 1.0f) v = v * rp.routed_scaling;
            rb.idx[(size_t)t * K + s] = chosen[s];
            rb.weights[(size_t)t * K + s] = v;
        }
    }
}

bool route_fits_lds(const RouteParams &rp)
{
    const int G = rp.use_block ? rp.block_size : 32;
    return (size_t)G * rp.n_experts <= ROUTE_LDS && (size_t)G * rp.top_k <= ROUTE_LDS / 8;
}

hipError_t launch_route(const RouteParams &rp, const float *logits, const float *bias,
                        const RouteBufs &rb, hipStream_t s)
{
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (rp.n_tokens + G - 1) / G;
    if (route_fits_lds(rp))
        hipLaunchKernelGGL(k_route, dim3(ngroups), dim3(ROUTE_THREADS), 0, s, rp, logits, bias,
                           rb);
    else
        hipLaunchKernelGGL(k_route_general, dim3(ngroups), dim3(256), 0, s, rp, logits, bias, rb);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dispatch.  counts[e] = sum of the group histograms, offsets = exclusive scan,
// perm[offsets[e] + (pairs of e in earlier groups) + local rank] = pair id,
// which is the stable grouping of the t-major pair list.  Also the work list:
// (expert, token chunk) entries for every expert with pairs.
constexpr int DISP_THREADS = 1024;

__global__ __launch_bounds__(DISP_THREADS) void k_dispatch(RouteParams rp, RouteBufs rb,
                                                           WorkList wl)
{
    __shared__ int32_t s_scan[MAX_E];
    __shared__ int32_t s_chunks[MAX_E];
    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (N + G - 1) / G;
    const int tid = threadIdx.x;

    for (int e = tid; e < E; e += DISP_THREADS) {
        int run = 0;
        for (int g = 0; g < ngroups; g++) run += rb.hist[(size_t)g * E + e];
        s_scan[e] = run;
        s_chunks[e] = (run + wl.chunk - 1) / wl.chunk;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0, nec = 0;
        for (int e = 0; e < E; e++) {
            const int c = s_scan[e];
            rb.counts[e] = c;
            rb.offsets[e] = run;
            s_scan[e] = run;
            run += c;
            for (int k = 0; k < s_chunks[e]; k++) {
                wl.ec_expert[nec] = e;
                wl.ec_chunk[nec] = k;
                nec++;
            }
        }
        rb.offsets[E] = run;
        wl.n_ec[0] = nec;
    }
    __syncthreads();
    // hist and lrank were written by the routing launch
    const int P = N * K;
    for (int p = tid; p < P; p += DISP_THREADS) {
        const int g = (p / K) / G;
        const int e = rb.idx[p];
        int base = s_scan[e];
        for (int h = 0; h < g; h++) base += rb.hist[(size_t)h * E + e];
        rb.perm[base + rb.lrank[p]] = p;
    }
}

// General shapes: one thread per expert scans the pair list.
__global__ __launch_bounds__(DISP_THREADS) void k_dispatch_general(RouteParams rp, RouteBufs rb,
                                                                   WorkList wl)
{
    __shared__ int32_t s_cnt[MAX_E];
    const int E = rp.n_experts, P = rp.n_tokens * rp.top_k, tid = threadIdx.x;
    for (int e = tid; e < E; e += DISP_THREADS) {
        int k = 0;
        for (int i = 0; i < P; i++) k += rb.idx[i] == e;
        s_cnt[e] = k;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0, nec = 0;
        for (int e = 0; e < E; e++) {
            const int k = s_cnt[e];
            rb.counts[e] = k;
            rb.offsets[e] = run;
            s_cnt[e] = run;
            run += k;
            for (int c = 0; c < (k + wl.chunk - 1) / wl.chunk; c++) {
                wl.ec_expert[nec] = e;
                wl.ec_chunk[nec] = c;
                nec++;
            }
        }
        rb.offsets[E] = run;
        wl.n_ec[0] = nec;
    }
    __syncthreads();
    for (int e = tid; e < E; e += DISP_THREADS) {
        int p = s_cnt[e];
        for (int i = 0; i < P; i++)
            if (rb.idx[i] == e) rb.perm[p++] = i;
    }
}

hipError_t launch_dispatch(const RouteParams &rp, const RouteBufs &rb, const WorkList &wl,
                           hipStream_t s)
{
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (rp.n_tokens + G - 1) / G;
    (void)ngroups;
    if (route_fits_lds(rp))
        hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(DISP_THREADS), 0, s, rp, rb, wl);
    else
        hipLaunchKernelGGL(k_dispatch_general, dim3(1), dim3(DISP_THREADS), 0, s, rp, rb, wl);
    return hipGetLastError();
}

} // namespace dmoe
