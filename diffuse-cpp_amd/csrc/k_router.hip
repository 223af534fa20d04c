// k_router.hip — routing stages of the MoE segment on gfx950 (after the
// router logits, which k_prep.hip's front kernel computes together with
// probs = sigmoid(logits) and sel = probs + bias, src/diffuse-moe-graph.cpp:203-210).
//
//   route    : per routing group (a block of block_size tokens with block
//              routing, else 32 tokens): block max fold, capacity threshold,
//              allowed mask, per-token top-k and gate weights (:212-262), the
//              group's expert histogram and the local rank of its pairs; the
//              last group to finish then runs the dispatch: counts, offsets,
//              the stable grouping of (token, slot) pairs by expert (the row
//              grouping ggml_mul_mat_id performs, :266-269) and the work list
//              of the expert kernels.
//
// Bit-exactness: single IEEE operations in a fixed order (no contraction),
// order decisions on exact integer keys, counts and ranks without atomics on
// the results (one atomic counter only elects the group that dispatches).
#include "dmoe_device.h"

#pragma clang fp contract(off)

namespace dmoe {

constexpr int MAX_E = 1024;     // experts per layer supported by these kernels
constexpr int MAX_K = 32;       // top_k supported by these kernels
constexpr int RT_THREADS = 1024;
constexpr int RT_WAVES = RT_THREADS / 64;

// Block-wide exclusive scan of one int per thread (blockDim.x == 1024).
// Returns the exclusive prefix; *total receives the sum.
__device__ __forceinline__ int block_scan(int v, int *s_tmp, int *total)
{
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int x = v;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const int o = __shfl_up(x, m, 64);
        if (lane >= m) x += o;
    }
    if (lane == 63) s_tmp[w] = x;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int i = 0; i < RT_WAVES; i++) {
            const int t = s_tmp[i];
            s_tmp[i] = run;
            run += t;
        }
        s_tmp[RT_WAVES] = run;
    }
    __syncthreads();
    const int excl = s_tmp[w] + x - v;
    *total = s_tmp[RT_WAVES];
    __syncthreads();
    return excl;
}

// Dispatch of one forward, run by the last routing group (all 1024 threads).
__device__ void dispatch_all(const RouteParams &rp, const RouteBufs &rb, const WorkList &wl,
                             int *s_tmp, int *s_off)
{
    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (N + G - 1) / G;
    const int tid = threadIdx.x;
    int c = 0;
    if (tid < E)
        for (int g = 0; g < ngroups; g++) c += rb.hist[(size_t)g * E + tid];
    int total;
    const int off = block_scan(c, s_tmp, &total);
    const int nch = (c + wl.chunk - 1) / wl.chunk;
    int nec;
    const int ecb = block_scan(nch, s_tmp, &nec);
    if (tid < E) {
        rb.counts[tid] = c;
        rb.offsets[tid] = off;
        s_off[tid] = off;
        for (int k = 0; k < nch; k++) {
            wl.ec_expert[ecb + k] = tid;
            wl.ec_chunk[ecb + k] = k;
        }
    }
    if (tid == 0) {
        rb.offsets[E] = total;
        wl.n_ec[0] = nec;
    }
    __syncthreads();
    const int P = N * K;
    for (int p = tid; p < P; p += RT_THREADS) {
        const int g = (p / K) / G;
        const int e = rb.idx[p];
        int base = s_off[e];
        for (int h = 0; h < g; h++) base += rb.hist[(size_t)h * E + e];
        rb.perm[base + rb.lrank[p]] = p;
    }
}

__global__ __launch_bounds__(RT_THREADS) void k_route(RouteParams rp, RouteBufs rb, WorkList wl,
                                                      int32_t *counter)
{
    __shared__ uint32_t s_key[ROUTE_LDS];         // group scores, then sel' keys
    __shared__ float s_bmax[MAX_E];
    __shared__ uint32_t s_bkey[MAX_E];
    __shared__ int32_t s_cand[MAX_E];
    __shared__ int32_t s_slot[RT_WAVES][MAX_K];
    __shared__ int32_t s_idx[ROUTE_LDS / 8];      // group pairs (tokens x slots)
    __shared__ int s_tmp[RT_WAVES + 1];
    __shared__ float s_thr;
    __shared__ int s_nan, s_nc, s_last;

    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int g = blockIdx.x;
    const int t0 = g * G;
    const int nt = min(N, t0 + G) - t0;
    const int tid = threadIdx.x;
    float *s_sel = reinterpret_cast<float *>(s_key);

    if (tid == 0) s_nan = 0;
    __syncthreads();
    // selection scores of the group (sel = probs + bias, :207-210)
    for (int i = tid; i < nt * E; i += RT_THREADS) {
        const float v = rb.sel[(size_t)t0 * E + i];
        s_sel[i] = v;
        if (v != v) s_nan = 1;
    }
    __syncthreads();

    bool restrict_cand = false;
    if (rp.use_block) {
        // :223-229  bmax = s_0 folded with m <- s_j + relu(m - s_j), j = 1..blk-1
        for (int e = tid; e < E; e += RT_THREADS) {
            float m = s_sel[e];
            for (int j = 1; j < G; j++) {
                const float sj = s_sel[j * E + e];
                float r = m - sj;
                r = r > 0.0f ? r : 0.0f;          // ggml_relu
                m = sj + r;
            }
            s_bmax[e] = m;
            s_bkey[e] = order_key(m);
        }
        __syncthreads();
        // :232-236  thr = the cap-th largest bmax (position cap-1 of the
        // descending order); exactly one expert has that rank
        for (int e = tid; e < E; e += RT_THREADS) {
            const uint32_t ke = s_bkey[e];
            int rank = 0;
            for (int f = 0; f < E; f++) rank += ranks_before(s_bkey[f], f, ke, e);
            if (rank == rp.capacity - 1) s_thr = s_bmax[e];
        }
        __syncthreads();
        // :241-248  keep = step(bmax - (thr + -1e-6)); sel' = sel + (0 | -1e30)
        const float tp = s_thr + (-1e-6f);
        const int keep = tid < E ? (s_bmax[tid] - tp) > 0.0f : 0;
        if (tid < E) {
            rb.bmax[(size_t)g * E + tid] = s_bmax[tid];
            rb.allowed[(size_t)g * E + tid] = (uint8_t)keep;
        }
        if (tid == 0) rb.thr[g] = s_thr;
        int nallowed;
        const int pos = block_scan(keep, s_tmp, &nallowed);
        // Every allowed score (finite, |sel| < 1e20) ranks above every masked
        // one (sel - 1e30 < -9e29), so the top-k can be taken among the
        // allowed experts alone when there are at least k of them.
        restrict_cand = rp.bias_small && !s_nan && nallowed >= K;
        if (restrict_cand && keep) s_cand[pos] = tid;
        const float add = (float)keep * 1e30f + (-1e30f);
        for (int t = 0; t < nt; t++)
            if (tid < E) s_key[t * E + tid] = order_key(s_sel[t * E + tid] + add);
        if (tid == 0) s_nc = restrict_cand ? nallowed : E;
    } else {
        for (int i = tid; i < nt * E; i += RT_THREADS) s_key[i] = order_key(s_sel[i]);
        if (tid == 0) s_nc = E;
    }
    if (!restrict_cand)
        for (int e = tid; e < E; e += RT_THREADS) s_cand[e] = e;
    __syncthreads();

    // :252  top-k: a candidate's slot is its rank among the token's candidates
    // (descending sel', ties to the lower expert id)
    const int lane = tid & 63, wave = tid >> 6;
    const int nc = s_nc;
    for (int t = wave; t < nt; t += RT_WAVES) {
        const uint32_t *kt = s_key + t * E;
        for (int c = lane; c < nc; c += 64) {
            const int e = s_cand[c];
            const uint32_t k = kt[e];
            int rank = 0;
            for (int c2 = 0; c2 < nc; c2++) {
                const int e2 = s_cand[c2];
                rank += ranks_before(kt[e2], e2, k, e);
            }
            if (rank < K) s_slot[wave][rank] = e;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // :253-262  w = probs[idx]; w /= sum (binary64 row sum); w *= scale
        const int mine = lane < K ? s_slot[wave][lane] : 0;
        float w = lane < K ? rb.probs[(size_t)(t0 + t) * E + mine] : 0.0f;
        double acc = 0.0;
        for (int s = 0; s < K; s++) acc += (double)__shfl(w, s, 64);
        if (lane < K) {
            if (rp.norm_topk_prob) w = w / (float)acc;
            if (rp.routed_scaling != 1.0f) w = w * rp.routed_scaling;
            rb.idx[(size_t)(t0 + t) * K + lane] = mine;
            rb.weights[(size_t)(t0 + t) * K + lane] = w;
            s_idx[t * K + lane] = mine;
        }
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();

    // group histogram and the rank of each pair among the group's pairs of the
    // same expert (pairs in t-major, slot-minor order)
    const int np = nt * K;
    for (int e = tid; e < E; e += RT_THREADS) {
        int c = 0;
        for (int j = 0; j < np; j++) c += s_idx[j] == e;
        rb.hist[(size_t)g * E + e] = c;
    }
    for (int j = tid; j < np; j += RT_THREADS) {
        const int e = s_idx[j];
        int r = 0;
        for (int i = 0; i < j; i++) r += s_idx[i] == e;
        rb.lrank[(size_t)t0 * K + j] = r;
    }

    // the last group to finish runs the dispatch
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const int ngroups = (N + G - 1) / G;
        s_last = atomicAdd(counter, 1) == ngroups - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    dispatch_all(rp, rb, wl, s_tmp, reinterpret_cast<int *>(s_bkey));
    if (tid == 0) *counter = 0;
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

// General shapes: one thread per expert scans the pair list.
constexpr int DISP_THREADS = 1024;

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

bool route_fits_lds(const RouteParams &rp)
{
    const int G = rp.use_block ? rp.block_size : 32;
    return (size_t)G * rp.n_experts <= ROUTE_LDS && (size_t)G * rp.top_k <= ROUTE_LDS / 8 &&
           rp.top_k <= MAX_K && rp.n_experts <= RT_THREADS;
}

hipError_t launch_route(const RouteParams &rp, const RouteBufs &rb, const WorkList &wl,
                        int32_t *counter, hipStream_t s)
{
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (rp.n_tokens + G - 1) / G;
    if (route_fits_lds(rp)) {
        hipLaunchKernelGGL(k_route, dim3(ngroups), dim3(RT_THREADS), 0, s, rp, rb, wl, counter);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_route_general, dim3(ngroups), dim3(256), 0, s, rp, rb.logits,
                       rp.bias, rb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_dispatch_general, dim3(1), dim3(1024), 0, s, rp, rb, wl);
    return hipGetLastError();
}

} // namespace dmoe
