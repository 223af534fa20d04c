// k_router.hip — routing stages of the MoE segment on gfx950 (after the
// router logits, which k_prep.hip's front kernel computes together with
// probs = sigmoid(logits) and sel = probs + bias, src/diffuse-moe-graph.cpp:203-210).
//
//   route    : per routing group (a block of block_size tokens with block
//              routing, else 32 tokens): block max fold, capacity threshold,
//              allowed mask, per-token top-k and gate weights (:212-262), the
//              group's expert histogram and the local rank of its pairs
//   dispatch : counts, offsets, the stable grouping of (token, slot) pairs by
//              expert (the row grouping ggml_mul_mat_id performs, :266-269)
//              and the work list of the expert kernels; in the route kernel
//              itself when the forward is one group, else in one workgroup
//              launched after it (the launch boundary makes every group's
//              results visible to it without a device-scope fence per group)
//
// Bit-exactness: single IEEE operations in a fixed order (no contraction),
// order decisions on exact integer keys, counts and ranks without atomics on
// the results.
#include "dmoe_prep.h"

#pragma clang fp contract(off)

namespace dmoe {

constexpr int MAX_E = 1024;     // experts per layer supported by these kernels
constexpr int MAX_K = 32;       // top_k supported by these kernels
constexpr int RT_THREADS = 1024;
constexpr int RT_WAVES = RT_THREADS / 64;
// token bitmasks per expert: E * ceil(G/32) words, with G*E <= ROUTE_LDS and E <= 1024
constexpr int RT_BITS = ROUTE_LDS / 32 + MAX_E;
// per-(group, expert) prefix table of the dispatch (64 x 256 at 2048 tokens)
constexpr int ROUTE_PREF = 16384;
// a group has at most ROUTE_LDS / 8 pairs, one per thread
static_assert(ROUTE_LDS / 8 <= RT_THREADS, "one thread per pair of a routing group");

// Block-wide exclusive scan of one int per thread (blockDim.x == 1024).
// Returns the exclusive prefix; *total receives the sum.
__device__ __forceinline__ int block_scan(int v, int *s_tmp, int *total)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const int o = __shfl_up(x, m, 64);
        if (lane >= m) x += o;
    }
    if (lane == 63) s_tmp[w] = x;
    __syncthreads();
    // every thread adds the wavefront totals itself (independent LDS reads)
    int before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < RT_WAVES; i++) {
        const int t = s_tmp[i];
        before += i < w ? t : 0;
        all += t;
    }
    *total = all;
    __syncthreads();            // s_tmp is reused by the next scan
    return before + x - v;
}

// Counts, offsets and the expert-chunk work list from each thread's pair
// count c (threads tid < E), all 1024 threads.  s_off receives the offsets;
// the global outputs are written when publish is set.
__device__ void dispatch_lists(int c, const RouteParams &rp, const RouteBufs &rb,
                               const WorkList &wl, int *s_tmp, int *s_off, bool publish)
{
    const int E = rp.n_experts, tid = threadIdx.x;
    int total, nec, off, ecb;
    const int nch = (c + wl.chunk - 1) / wl.chunk;
    if (rp.n_tokens * rp.top_k < 32768 && E + rp.n_tokens * rp.top_k / wl.chunk + 1 < 32768) {
        // both prefixes in one scan (pair counts in the low 16 bits, chunk
        // counts in the high ones): every partial sum of either is below 2^15
        int both;
        const int p = block_scan(c | (nch << 16), s_tmp, &both);
        off = p & 0xFFFF;
        ecb = p >> 16;
        total = both & 0xFFFF;
        nec = both >> 16;
    } else {
        off = block_scan(c, s_tmp, &total);
        ecb = block_scan(nch, s_tmp, &nec);
    }
    if (tid < E) s_off[tid] = off;
    if (publish && tid < E) {
        rb.counts[tid] = c;
        rb.offsets[tid] = off;
        for (int k = 0; k < nch; k++) {
            wl.ec_expert[ecb + k] = tid;
            wl.ec_chunk[ecb + k] = k;
        }
    }
    if (publish && tid == 0) {
        rb.offsets[E] = total;
        wl.n_ec[0] = nec;
    }
    __syncthreads();
}

// Dispatch of one forward over several routing groups, from the groups'
// histograms (pairs per expert) and the pairs' local ranks, by one workgroup
// of 1024 threads for the pairs of groups g_lo .. g_hi - 1 (every workgroup
// derives the offsets from all histograms; the one with publish set writes
// counts, offsets and the work list).  The groups are taken in chunks of
// ROUTE_PREF / E: a chunk's histograms are copied to LDS by all threads
// (eight loads in flight each), scanned over its groups by thread e (the
// exclusive prefix, carried from chunk to chunk), and the pairs of the
// workgroup's groups in the chunk are then scattered to their slots, eight per
// thread at a time.  One chunk holds every group up to ROUTE_PREF / E groups;
// beyond that the totals take one more pass.
__device__ void dispatch_all(const RouteParams &rp, const RouteBufs &rb, const WorkList &wl,
                             int *s_tmp, int *s_off, int *s_pref, int g_lo, int g_hi, bool publish)
{
    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (N + G - 1) / G;
    const int gchunk = ROUTE_PREF / E;
    const int tid = threadIdx.x;
    auto load_chunk = [&](int gb, int ng) {
        const int n = ng * E;
        const int *src = rb.hist + (size_t)gb * E;
        for (int i0 = 0; i0 < n; i0 += 8 * RT_THREADS) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * RT_THREADS + tid;
                v[j] = i < n ? src[i] : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * RT_THREADS + tid;
                if (i < n) s_pref[i] = v[j];
            }
        }
        __syncthreads();
    };
    // thread e: s_pref[g][e] <- pairs of expert e in earlier groups (from
    // *run on), *run advanced past the chunk
    auto scan_chunk = [&](int ng, int *run) {
        if (tid >= E) return;
        int c = *run, g = 0;
        for (; g + 8 <= ng; g += 8) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = s_pref[(g + j) * E + tid];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                s_pref[(g + j) * E + tid] = c;
                c += v[j];
            }
        }
        for (; g < ng; g++) {
            const int v = s_pref[g * E + tid];
            s_pref[g * E + tid] = c;
            c += v;
        }
        *run = c;
    };

    int c = 0;                         // pairs of expert tid
    if (ngroups <= gchunk) {
        load_chunk(0, ngroups);
        scan_chunk(ngroups, &c);
    } else {
        // totals first: all threads add histogram entries into LDS counters
        int *s_cnt = s_pref;
        for (int e = tid; e < E; e += RT_THREADS) s_cnt[e] = 0;
        __syncthreads();
        const int n = ngroups * E;
        for (int i0 = 0; i0 < n; i0 += 8 * RT_THREADS) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * RT_THREADS + tid;
                v[j] = i < n ? rb.hist[i] : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * RT_THREADS + tid;
                if (i < n && v[j]) atomicAdd(&s_cnt[i % E], v[j]);
            }
        }
        __syncthreads();
        if (tid < E) c = s_cnt[tid];
        __syncthreads();               // s_pref is reused by the chunks below
    }
    dispatch_lists(c, rp, rb, wl, s_tmp, s_off, publish);

    // a pair's group p / (K G) by a float reciprocal, made exact by one
    // correction each way (pair indices below 2^24)
    const int KG = K * G;
    const float rkg = 1.0f / (float)KG;
    int run = 0;                       // thread e: pairs of expert e before the chunk
    for (int gb = 0; gb < g_hi; gb += gchunk) {
        const int ng = min(gchunk, ngroups - gb);
        if (ngroups > gchunk) {
            load_chunk(gb, ng);
            scan_chunk(ng, &run);
        }
        __syncthreads();
        // this workgroup's pairs in the chunk: tokens lo * G .. hi * G, K slots each
        const int lo = max(gb, g_lo), hi = min(gb + ng, g_hi);
        const int p_lo = lo * KG, p_hi = lo < hi ? min(N, hi * G) * K : p_lo;
        for (int p0 = p_lo; p0 < p_hi; p0 += 8 * RT_THREADS) {
            int ev[8], lv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int p = p0 + j * RT_THREADS + tid;
                ev[j] = p < p_hi ? rb.idx[p] : 0;
                lv[j] = p < p_hi ? rb.lrank[p] : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int p = p0 + j * RT_THREADS + tid;
                if (p >= p_hi) continue;
                int q = (int)((float)p * rkg);
                q -= q * KG > p ? 1 : 0;
                q += (q + 1) * KG <= p ? 1 : 0;
                const int g = q - gb, e = ev[j];
                rb.perm[s_off[e] + s_pref[g * E + e] + lv[j]] = p;
            }
        }
        __syncthreads();               // before the next chunk overwrites s_pref
    }
}

// Wavefront reductions of unsigned ints over 64 lanes (DPP row shifts and
// broadcasts; the result is read from lane 63).
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v)
{
    const int id = MAX ? 0 : -1;
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x111, 0xF, 0xF, false));   // row_shr:1
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x112, 0xF, 0xF, false));   // row_shr:2
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x114, 0xF, 0xF, false));   // row_shr:4
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x118, 0xF, 0xF, false));   // row_shr:8
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xA, 0xF, false));   // row_bcast:15
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xC, 0xF, false));   // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ int wave_sum_i32(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return __builtin_amdgcn_readlane(v, 63);
}

// One wavefront: the bmax at position cap-1 of the descending order (ties to
// the lower expert id).  Lane l keeps the order keys of experts l + 64 r.  A
// most-significant-bit-first radix select finds the cap-th largest key P
// (counts by ballot), starting below the bits that every key shares; the
// expert at position cap-1 is then the (cap - 1 - #{keys > P})-th lowest id
// among the experts whose key is P.
template <int R, bool FULL>
__device__ void find_threshold(int E, int cap, const uint64_t *s_rk, const float *s_bmax,
                               float *s_thr)
{
    const int lane = threadIdx.x & 63;
    uint32_t k[R];
    uint64_t valid[R];
    uint32_t hi = 0u, lo = ~0u;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int f = lane + 64 * r;
        k[r] = f < E ? (uint32_t)(s_rk[f] >> 32) : 0u;
        valid[r] = __ballot(f < E);
        if (f < E) {
            hi = k[r] > hi ? k[r] : hi;
            lo = k[r] < lo ? k[r] : lo;
        }
    }
    hi = wave_reduce_u32<true>(hi);
    lo = wave_reduce_u32<false>(lo);
    // every key lies in [lo, hi]: they share the bits above the highest bit
    // where lo and hi differ, so P starts as that prefix (all keys >= P)
    const uint32_t diff = hi ^ lo;
    const int top = diff ? 31 - __builtin_clz(diff) : -1;
    uint32_t P = top >= 0 ? (hi & ~((2u << top) - 1u)) : hi;
    for (uint32_t bit = top >= 0 ? 1u << top : 0u; bit; bit >>= 1) {
        const uint32_t cand = P | bit;
        int cnt = 0;
#pragma unroll
        for (int r = 0; r < R; r++)
            cnt += __popcll(FULL ? __ballot(k[r] >= cand) : __ballot(k[r] >= cand) & valid[r]);
        P = cnt >= cap ? cand : P;
    }
    int n = cap - 1;
#pragma unroll
    for (int r = 0; r < R; r++) n -= __popcll(__ballot(k[r] > P) & valid[r]);
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint64_t m = __ballot(k[r] == P) & valid[r];
        const int c = __popcll(m);
        if (n >= 0 && n < c) {
            for (int i = 0; i < n; i++) m &= m - 1;
            const int f = __builtin_ctzll(m) + 64 * r;
            if (lane == 0) *s_thr = s_bmax[f];
        }
        n -= c;
    }
}

// Exclusive prefix of a 0/1 flag over threads tid < 256 (any block size):
// ballots and lane counts, four wavefront totals through LDS (s_w4: 4 ints).
__device__ __forceinline__ int flag_scan256(int flag, int *s_w4, int *total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t b = __ballot(flag);
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
    if (lane == 0 && wave < 4) s_w4[wave] = __popcll(b);
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const int t = s_w4[w];
        before += w < wave ? t : 0;
        all += t;
    }
    *total = all;
    return before + below;
}

// Activation conversions that ride along with a one-group route: job list
// and the conversion workgroups after the routing one.
struct RoutePrep {
    PrepJob job[2];
    int njobs;
};

// SINGLE: the forward is one routing group (the dispatch needs nothing
// beyond this block; the token probabilities are staged in LDS).  Blocks
// after the first then convert activations (pp), one (row, super-block) per
// wavefront, and touch nothing of the routing.
template <bool SINGLE>
__global__ __launch_bounds__(RT_THREADS) void k_route(RouteParams rp, RouteBufs rb, WorkList wl, RoutePrep pp)
{
    __shared__ uint32_t s_key[ROUTE_LDS];         // group scores, then sel' keys
    __shared__ float s_bmax[MAX_E];
    __shared__ uint64_t s_rk[MAX_E];              // rank keys of the block maxima
    __shared__ int32_t s_cand[MAX_E];
    __shared__ int32_t s_idx[ROUTE_LDS / 8];      // group pairs (tokens x slots)
    __shared__ float s_w[ROUTE_LDS / 8];          // their probs
    __shared__ __align__(16) uint32_t s_k32[RT_WAVES][2][64];   // per wavefront: order keys of two tokens
    __shared__ uint32_t s_bits[RT_BITS];          // [e][word]: tokens of the group that chose e
    __shared__ int s_tmp[RT_WAVES + 1];
    __shared__ float s_probs[SINGLE ? ROUTE_LDS : 1];   // the group's probs (one group)
    __shared__ float s_thr;
    __shared__ int s_nan, s_nc;

    const int E = rp.n_experts, K = rp.top_k, N = rp.n_tokens;
    const int G = rp.use_block ? rp.block_size : 32;
    const int g = blockIdx.x;
    const int t0 = g * G;
    const int nt = min(N, t0 + G) - t0;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int words = (G + 31) / 32;
    float *s_sel = reinterpret_cast<float *>(s_key);

    if constexpr (SINGLE) {
        if (g > 0) {
            int wid = (g - 1) * RT_WAVES + wave;
            float *sv = s_sel + wave * 256;
            for (int j = 0; j < pp.njobs; j++) {
                const int n = pp.job[j].rows * (pp.job[j].K / 256);
                if (wid < n) {
                    prep_wave(pp.job[j], wid, sv);
                    return;
                }
                wid -= n;
            }
            return;
        }
    }

    // one forward = one group: the group's probs go to LDS, loaded with the scores
    constexpr int R = ROUTE_LDS / RT_THREADS;
    float pv[R];
    if constexpr (SINGLE) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = tid + r * RT_THREADS;
            pv[r] = i < nt * E ? rb.probs[(size_t)t0 * E + i] : 0.0f;
        }
    }
    if (tid == 0) s_nan = 0;
    for (int i = tid; i < E * words; i += RT_THREADS) s_bits[i] = 0u;

    // selection scores of the group (sel = probs + bias, :207-210); every
    // load is issued before the first is used.  Blocks of 32 tokens: thread
    // e loads the 32 scores of expert e and folds them in registers.
    const bool fold32 = rp.use_block && G == 32 && nt == 32;
    bool nan = false;
    if (fold32) {
        if (tid < E) {
            const float *src = rb.sel + (size_t)t0 * E + tid;
            float v[32];
#pragma unroll
            for (int t = 0; t < 32; t++) v[t] = src[(size_t)t * E];
            // :223-229  bmax = s_0 folded with m <- s_j + relu(m - s_j), j = 1..blk-1
            float m = v[0];
            nan = v[0] != v[0];
#pragma unroll
            for (int j = 1; j < 32; j++) {
                s_sel[j * E + tid] = v[j];
                nan |= v[j] != v[j];
                float r = m - v[j];
                r = r > 0.0f ? r : 0.0f;          // ggml_relu
                m = v[j] + r;
            }
            s_sel[tid] = v[0];
            s_bmax[tid] = m;
            s_rk[tid] = rank_key(order_key(m), tid);
        }
    } else {
        const int n = nt * E;
        const float *src = rb.sel + (size_t)t0 * E;
        float v[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = tid + r * RT_THREADS;
            v[r] = i < n ? src[i] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = tid + r * RT_THREADS;
            if (i < n) s_sel[i] = v[r];
            nan |= v[r] != v[r];
        }
    }
    if constexpr (SINGLE) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = tid + r * RT_THREADS;
            if (i < nt * E) s_probs[i] = pv[r];
        }
    }
    __syncthreads();
    if (nan) s_nan = 1;

    bool restrict_cand = false;
    if (rp.use_block) {
        if (!fold32) {
            for (int e = tid; e < E; e += RT_THREADS) {
                float m = s_sel[e];
                for (int j = 1; j < G; j++) {
                    const float sj = s_sel[j * E + e];
                    float r = m - sj;
                    r = r > 0.0f ? r : 0.0f;      // ggml_relu
                    m = sj + r;
                }
                s_bmax[e] = m;
                s_rk[e] = rank_key(order_key(m), e);
            }
            __syncthreads();
        }
        // :232-236  thr = the cap-th largest bmax (position cap-1 of the
        // descending order, ties to the lower expert id)
        if (E == 256) {
            // rank counting on all 1,024 threads: thread (part q, expert e)
            // counts the experts of part q (64 of them, read as LDS
            // broadcasts) whose rank key is above e's; the expert whose four
            // counts sum to cap - 1 holds the threshold (rank keys are unique)
            int *s_cnt4 = s_idx;                      // [4][256], free until the top-k
            const int e = tid & 255, q = tid >> 8;
            const uint64_t my = s_rk[e];
            int cnt = 0;
#pragma unroll 16
            for (int i = 0; i < 64; i++) cnt += s_rk[64 * q + i] > my ? 1 : 0;
            s_cnt4[q * 256 + e] = cnt;
            __syncthreads();
            if (tid < 256 &&
                s_cnt4[tid] + s_cnt4[256 + tid] + s_cnt4[512 + tid] + s_cnt4[768 + tid] == rp.capacity - 1)
                s_thr = s_bmax[tid];
        } else if (wave == 0) {
            if (E < 256)
                find_threshold<4, false>(E, rp.capacity, s_rk, s_bmax, &s_thr);
            else
                find_threshold<MAX_E / 64, false>(E, rp.capacity, s_rk, s_bmax, &s_thr);
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
        const int pos = E <= 256 ? flag_scan256(keep, s_tmp, &nallowed) : block_scan(keep, s_tmp, &nallowed);
        // Every allowed score (finite, |sel| < 1e20) ranks above every masked
        // one (sel - 1e30 < -9e29), so the top-k can be taken among the
        // allowed experts alone when there are at least k of them; their
        // sel' = sel + 0 has the order key of sel.
        restrict_cand = rp.bias_small && !s_nan && nallowed >= K;
        if (restrict_cand && keep) s_cand[pos] = tid;
        if (!restrict_cand) {
            if (RT_THREADS % E == 0) {
                // every thread converts the scores of one expert
                const int e = tid % E;
                const float add = (float)((s_bmax[e] - tp) > 0.0f) * 1e30f + (-1e30f);
                for (int t = tid / E; t < nt; t += RT_THREADS / E)
                    s_key[t * E + e] = order_key(s_sel[t * E + e] + add);
            } else {
                const float add = (float)keep * 1e30f + (-1e30f);
                for (int t = 0; t < nt; t++)
                    if (tid < E) s_key[t * E + tid] = order_key(s_sel[t * E + tid] + add);
            }
        }
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
    const int nc = s_nc;
    if (nc <= 64) {
        // lane c holds candidate c's order key for two tokens of the
        // wavefront at a time; a candidate's slot is the number of keys
        // above its own (LDS broadcasts, four keys per read) plus, when keys
        // tie, the tied candidates of lower id (lower lane).  Without ties
        // the counts are a permutation of 0 .. nc-1, which their sum tests.
        const bool act = lane < nc;
        const int my_e = act ? s_cand[lane] : 0;
        auto okey = [&](int t) -> uint32_t {
            if (!act || t >= nt) return 0u;
            return restrict_cand ? order_key(s_sel[t * E + my_e]) : s_key[t * E + my_e];
        };
        const int nc4 = (nc + 3) & ~3;
        const int perm_sum = nc * (nc - 1) / 2;
        for (int t = wave; t < nt; t += 2 * RT_WAVES) {
            const int t2 = t + RT_WAVES;
            const uint32_t k0 = okey(t), k1 = okey(t2);
            s_k32[wave][0][lane] = k0;
            s_k32[wave][1][lane] = k1;
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            int r0 = 0, r1 = 0;
            // keys past nc are 0 and never above a candidate's
#pragma unroll 4
            for (int c2 = 0; c2 < nc4; c2 += 4) {
                const uint4 a = *reinterpret_cast<const uint4 *>(&s_k32[wave][0][c2]);
                const uint4 b = *reinterpret_cast<const uint4 *>(&s_k32[wave][1][c2]);
                r0 += (a.x > k0 ? 1 : 0) + (a.y > k0 ? 1 : 0) + (a.z > k0 ? 1 : 0) + (a.w > k0 ? 1 : 0);
                r1 += (b.x > k1 ? 1 : 0) + (b.y > k1 ? 1 : 0) + (b.z > k1 ? 1 : 0) + (b.w > k1 ? 1 : 0);
            }
            if (wave_sum_i32(act ? r0 : 0) != perm_sum)
                for (int c2 = 0; c2 < lane; c2++) r0 += s_k32[wave][0][c2] == k0 ? 1 : 0;
            if (t2 < nt && wave_sum_i32(act ? r1 : 0) != perm_sum)
                for (int c2 = 0; c2 < lane; c2++) r1 += s_k32[wave][1][c2] == k1 ? 1 : 0;
            if (act && r0 < K) s_idx[t * K + r0] = my_e;
            if (act && t2 < nt && r1 < K) s_idx[t2 * K + r1] = my_e;
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        }
    } else {
        // keys: the sel' keys, or with restricted candidates the keys of sel
        auto key = [&](int t, int e) -> uint32_t {
            return restrict_cand ? order_key(s_sel[t * E + e]) : s_key[t * E + e];
        };
        for (int t = wave; t < nt; t += RT_WAVES) {
            for (int c = lane; c < nc; c += 64) {
                const int e = s_cand[c];
                const uint32_t k = key(t, e);
                int rank = 0;
#pragma unroll 8
                for (int c2 = 0; c2 < nc; c2++) {
                    const int e2 = s_cand[c2];
                    rank += ranks_before(key(t, e2), e2, k, e);
                }
                if (rank < K) s_idx[t * K + rank] = e;
            }
        }
    }
    __syncthreads();

    // :253-262  w = probs[idx]; w /= the token's sum (binary64, slot order);
    // w *= scale.  Thread j owns pair j (token j / K, slot j % K).
    const int np = nt * K;
    const int pt = tid / K;
    int mine = 0;
    float w = 0.0f;
    if (tid < np) {
        mine = s_idx[tid];
        if constexpr (SINGLE)
            w = s_probs[pt * E + mine];
        else
            w = rb.probs[(size_t)(t0 + pt) * E + mine];
        s_w[tid] = w;
        atomicOr(&s_bits[mine * words + (pt >> 5)], 1u << (pt & 31));
    }
    __syncthreads();
    int lr = 0;
    if (tid < np) {
        double acc = 0.0;
        for (int q = 0; q < K; q++) acc += (double)s_w[pt * K + q];
        if (rp.norm_topk_prob) w = w / (float)acc;
        if (rp.routed_scaling != 1.0f) w = w * rp.routed_scaling;
        rb.idx[(size_t)t0 * K + tid] = mine;
        rb.weights[(size_t)t0 * K + tid] = w;
        // rank of the pair among the group's pairs of the same expert (pairs
        // in t-major, slot-minor order).  A token picks an expert at most
        // once, so that rank counts the earlier tokens whose bit is set.
        const uint32_t *bits = s_bits + mine * words;
        lr = __popc(bits[pt >> 5] & ((1u << (pt & 31)) - 1u));
        for (int wd = 0; wd < (pt >> 5); wd++) lr += __popc(bits[wd]);
    }
    int c = 0;                               // pairs of expert tid in this group
    if (tid < E)
        for (int wd = 0; wd < words; wd++) c += __popc(s_bits[tid * words + wd]);

    int *s_off = reinterpret_cast<int *>(s_rk);
    if constexpr (SINGLE) {
        // one routing group: the dispatch needs nothing beyond this block
        dispatch_lists(c, rp, rb, wl, s_tmp, s_off, true);
        if (tid < np) rb.perm[s_off[mine] + lr] = tid;
        return;
    } else {
        // several groups: k_dispatch_groups, the next launch, dispatches them
        if (tid < E) rb.hist[(size_t)g * E + tid] = c;
        if (tid < np) rb.lrank[(size_t)t0 * K + tid] = lr;
    }
}

// The dispatch of a forward of several routing groups, after their k_route
// launch (which leaves hist and lrank for it): workgroup b scatters the pairs
// of groups DISP_GROUPS b .. DISP_GROUPS (b + 1) - 1, workgroup 0 also writes
// counts, offsets and the work list.
constexpr int DISP_GROUPS = 4;
__global__ __launch_bounds__(RT_THREADS) void k_dispatch_groups(RouteParams rp, RouteBufs rb, WorkList wl)
{
    __shared__ int s_tmp[RT_WAVES + 1];
    __shared__ int s_off[MAX_E];
    __shared__ int s_pref[ROUTE_PREF];
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (rp.n_tokens + G - 1) / G;
    const int g_lo = blockIdx.x * DISP_GROUPS, g_hi = min(ngroups, g_lo + DISP_GROUPS);
    dispatch_all(rp, rb, wl, s_tmp, s_off, s_pref, g_lo, g_hi, blockIdx.x == 0);
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
    // (pair indices below 2^24: the dispatch's float reciprocal is exact there)
    return (size_t)G * rp.n_experts <= ROUTE_LDS && (size_t)G * rp.top_k <= ROUTE_LDS / 8 &&
           rp.top_k <= MAX_K && rp.n_experts <= RT_THREADS && (size_t)rp.n_tokens * rp.top_k < (1u << 24);
}

bool route_single(const RouteParams &rp)
{
    const int G = rp.use_block ? rp.block_size : 32;
    return route_fits_lds(rp) && (rp.n_tokens + G - 1) / G == 1;
}

hipError_t launch_route(const RouteParams &rp, const RouteBufs &rb, const WorkList &wl, hipStream_t s,
                        const PrepJob *jobs, int njobs)
{
    const int G = rp.use_block ? rp.block_size : 32;
    const int ngroups = (rp.n_tokens + G - 1) / G;
    RoutePrep pp{};
    if (njobs < 0 || njobs > 2 || (njobs > 0 && !route_single(rp))) return hipErrorInvalidValue;
    int ptasks = 0;
    for (int j = 0; j < njobs; j++) {
        if (jobs[j].K <= 0 || jobs[j].K % 256 || jobs[j].rows <= 0) return hipErrorInvalidValue;
        pp.job[j] = jobs[j];
        ptasks += jobs[j].rows * (jobs[j].K / 256);
    }
    pp.njobs = njobs;
    if (route_fits_lds(rp)) {
        if (ngroups == 1) {
            const int blocks = 1 + (ptasks + RT_WAVES - 1) / RT_WAVES;
            hipLaunchKernelGGL(k_route<true>, dim3(blocks), dim3(RT_THREADS), 0, s, rp, rb, wl, pp);
            return hipGetLastError();
        }
        hipLaunchKernelGGL(k_route<false>, dim3(ngroups), dim3(RT_THREADS), 0, s, rp, rb, wl, pp);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_dispatch_groups, dim3((ngroups + DISP_GROUPS - 1) / DISP_GROUPS), dim3(RT_THREADS),
                           0, s, rp, rb, wl);
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
