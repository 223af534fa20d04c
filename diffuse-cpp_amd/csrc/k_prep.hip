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

// ---------------------------------------------------------------------------
// Router logits.  One wavefront per (LE experts, LT tokens).  For every
// (token, expert) lane l keeps one partial:  a_l = fma(W[k], x[k], a_l) for
// k = 256*i + 4*l + j, i ascending then j = 0..3; the 64 partials are then
// combined by six xor butterfly rounds (m = 32..1): round m adds lane l's
// value and lane l ^ m's (the same two operands in both partner lanes).  The
// lane holding output t*LE + e computes sigmoid and the score.  The tile
// shape only changes which rows a wavefront reads, not the order.
//
// The butterfly of NV partial vectors runs transposed (butterfly_sum): in
// round m a lane keeps half of its values and sends the other half to lane
// l ^ m, which keeps the opposite half, so both lanes of a pair still add
// the same two operands (own value first) as the plain butterfly, for one
// output instead of all.  After log2(NV) such rounds a lane holds one
// output, index (l >> (6 - log2 NV)) & (NV - 1); the remaining rounds are
// the plain butterfly on that value.

// N values v[0..N-1] left per lane, round distance M (N a power of two,
// N * M == 32 on the first call, or N == 64 and M == 0 after the last
// transposed round).  Returns this lane's output.
template <int N, int M>
__device__ __forceinline__ float butterfly_rounds(float *v, int lane)
{
    if constexpr (N == 1) {
        float r = v[0];
#pragma unroll
        for (int m = M; m >= 1; m >>= 1) r = r + __shfl_xor(r, m, 64);
        return r;
    } else {
        const bool hi = (lane & M) != 0;
#pragma unroll
        for (int j = 0; j < N / 2; j++) {
            const float send = hi ? v[j] : v[j + N / 2];
            const float keep = hi ? v[j + N / 2] : v[j];
            v[j] = keep + __shfl_xor(send, M, 64);
        }
        return butterfly_rounds<N / 2, M / 2>(v, lane);
    }
}

// NV: a power of two up to 64; v[j] = partial of output j.  Returns this
// lane's output (index (lane >> (6 - log2 NV)) & (NV - 1)).
template <int NV>
__device__ __forceinline__ float butterfly_sum(float (&v)[NV])
{
    static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "power of two <= 64");
    return butterfly_rounds<NV, 32>(v, threadIdx.x & 63);
}

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
    // Few outputs: the transposed butterfly (fewer shuffles).  Many (the
    // 64 of the wide tile): the plain one, whose 64 independent chains hide
    // the shuffle latency better (measured faster).  Same sums either way.
    constexpr int NV = LT * LE;
    static_assert((NV & (NV - 1)) == 0, "a power-of-two tile");
    float mine = 0.0f;
    int j;
    bool writer;
    if constexpr (NV <= 8) {
        constexpr int SH = 6 - __builtin_ctz(NV);
        float v[NV];
#pragma unroll
        for (int t = 0; t < LT; t++)
#pragma unroll
            for (int e = 0; e < LE; e++) v[t * LE + e] = acc[t][e];
        mine = butterfly_sum<NV>(v);
        j = lane >> SH;
        writer = (lane & ((1 << SH) - 1)) == 0;
    } else {
#pragma unroll
        for (int t = 0; t < LT; t++)
#pragma unroll
            for (int e = 0; e < LE; e++) {
                float v = acc[t][e];
#pragma unroll
                for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
                if (lane == t * LE + e) mine = v;
            }
        j = lane;
        writer = lane < NV;
    }
    const int t = j / LE, e = j % LE;
    if (writer && t0 + t < N && e0 + e < E) {
        const size_t o = (size_t)(t0 + t) * E + e0 + e;
        const float p = sigmoid_f32(mine);
        rb.logits[o] = mine;
        rb.probs[o] = p;
        rb.sel[o] = bias ? p + bias[e0 + e] : p;
    }
}

// Few tokens: one workgroup (4 wavefronts) per tile of LS_T tokens x LS_E
// experts.  The tile's x rows are staged in LDS once (every wavefront of the
// workgroup reads them there, not from L2); wavefront w keeps the rows of
// experts 2w, 2w + 1 of the tile in registers, every load issued up front.
// Lane l's partials and the butterfly rounds are those of logits_wave.
constexpr int LS_T = 4, LS_E = 8, LS_MAXK = 16;  // LS_MAXK * 256 = the largest n_embd

// NK = H / 256 (a power of two up to LS_MAXK)
// The activation conversions of the tile's rows run here too (the rows are in
// LDS): task (job j, row r, super-block sb) = (j * LS_T + r) * NK + sb goes
// to wavefront g = 4 * (expert group) + w of the token group and every
// 4 * (expert groups) after it, between the x staging and the first use of
// the expert rows.
template <int NK>
__device__ void logits_tile_small(const float *__restrict__ W, const float *__restrict__ bias,
                                  const float *__restrict__ x, int N, int E, int tile,
                                  const RouteBufs &rb, float4 *s_x, const PrepJob *jobs,
                                  int njobs, float *sv)
{
    constexpr int H = NK * 256;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ne = (E + LS_E - 1) / LS_E;
    const int e0 = (tile % ne) * LS_E + 2 * wave;
    const int t0 = (tile / ne) * LS_T;
    constexpr int h4 = H / 4;
    // the lane that writes output (ot, oe) of the tile (butterfly_sum's
    // index: lane >> 3), and its bias, loaded first
    const int oj = lane >> 3, ot = oj / 2, oe = oj % 2;
    const bool out_lane = (lane & 7) == 0;
    const float bsel = bias && out_lane ? bias[min(e0 + oe, E - 1)] : 0.0f;
    // x rows t0 .. t0+3 (clamped) -> LDS by LDS-direct loads (no registers
    // held), issued before the expert rows' loads; the wait before the
    // barrier covers them (loads complete in issue order), the expert rows
    // are awaited at their first use.
    {
        const uint32_t sx = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)s_x;
#pragma unroll
        for (int t = 0; t < LS_T; t++) {
            const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)min(t0 + t, N - 1) * H);
#pragma unroll
            for (int q = 0; q < (h4 + 255) / 256; q++) {
                const int c = q * 256 + wave * 64;         // the wavefront's first piece
                if (c < h4)
                    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                                 : : "v"(xr + c + lane),
                                     "s"(__builtin_amdgcn_readfirstlane(sx + (uint32_t)(t * h4 + c) * 16u))
                                 : "memory", "m0");
            }
        }
        // expert rows in k order (the empty asm keeps the issue order), so
        // that the first steps' operands arrive first
        float4 w[2][NK];
        const float4 *wr0 = reinterpret_cast<const float4 *>(W + (size_t)min(e0, E - 1) * H);
        const float4 *wr1 = reinterpret_cast<const float4 *>(W + (size_t)min(e0 + 1, E - 1) * H);
#pragma unroll
        for (int i = 0; i < NK; i++) {
            w[0][i] = wr0[i * 64 + lane];
            w[1][i] = wr1[i * 64 + lane];
            asm volatile("" ::: "memory");
        }
        // at most the 2 * NK expert-row loads still in flight
        __builtin_amdgcn_s_waitcnt(((2 * NK) & 15) | (((2 * NK) >> 4) << 14) | 0xF70);
        __syncthreads();

        {
            const float *sxf = reinterpret_cast<const float *>(s_x);
            const int g = (tile % ne) * 4 + wave, gstep = ne * 4;
            const int ntasks = njobs * LS_T * NK;
            for (int task = g; task < ntasks; task += gstep) {
                const int sb = task % NK, r = (task / NK) % LS_T, j = task / (NK * LS_T);
                if (t0 + r >= N) continue;
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = sxf[r * H + sb * 256 + lane + 64 * c];
                prep_values(v, jobs[j].out, jobs[j].mode, t0 + r, jobs[j].rows, sb, NK, sv);
            }
        }

        float acc[LS_T][2];
#pragma unroll
        for (int t = 0; t < LS_T; t++) acc[t][0] = acc[t][1] = 0.0f;
#pragma unroll
        for (int i = 0; i < NK; i++) {
            {
                float4 xv[LS_T];
#pragma unroll
                for (int t = 0; t < LS_T; t++) xv[t] = s_x[t * h4 + i * 64 + lane];
#pragma unroll
                for (int t = 0; t < LS_T; t++)
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        float a = acc[t][e];
                        a = __builtin_fmaf(w[e][i].x, xv[t].x, a);
                        a = __builtin_fmaf(w[e][i].y, xv[t].y, a);
                        a = __builtin_fmaf(w[e][i].z, xv[t].z, a);
                        a = __builtin_fmaf(w[e][i].w, xv[t].w, a);
                        acc[t][e] = a;
                    }
            }
        }
        float v2[LS_T * 2];
#pragma unroll
        for (int t = 0; t < LS_T; t++)
#pragma unroll
            for (int e = 0; e < 2; e++) v2[t * 2 + e] = acc[t][e];
        const float mine = butterfly_sum<LS_T * 2>(v2);
        if (out_lane && t0 + ot < N && e0 + oe < E) {
            const size_t o = (size_t)(t0 + ot) * E + e0 + oe;
            const float p = sigmoid_f32(mine);
            rb.logits[o] = mine;
            rb.probs[o] = p;
            rb.sel[o] = bias ? p + bsel : p;
        }
    }
}

__host__ __device__ __forceinline__ int small_tiles(int N, int E)
{
    return ((N + LS_T - 1) / LS_T) * ((E + LS_E - 1) / LS_E);
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
    int N, H, E, logit_blocks, wide, small;
    RouteBufs rb;
    PrepJob job[2];
    int njobs;
};

// SMALL: the logits of few tokens (logits_tile_small); else logits_wave tiles
template <bool SMALL>
__global__ __launch_bounds__(256) void k_front(FrontArgs a)
{
    __shared__ float s_v[4][256];
    const int w = threadIdx.x >> 6;
    int b = blockIdx.x;
    if constexpr (SMALL) {
        __shared__ float4 s_x[LS_T * LS_MAXK * 64];     // 64 KB: x rows of a small tile
        if (b < a.logit_blocks) {
            float *sv = s_v[w];
            switch (a.H) {
            case 256: logits_tile_small<1>(a.W, a.bias, a.x, a.N, a.E, b, a.rb, s_x, a.job, a.njobs, sv); break;
            case 512: logits_tile_small<2>(a.W, a.bias, a.x, a.N, a.E, b, a.rb, s_x, a.job, a.njobs, sv); break;
            case 1024: logits_tile_small<4>(a.W, a.bias, a.x, a.N, a.E, b, a.rb, s_x, a.job, a.njobs, sv); break;
            case 2048: logits_tile_small<8>(a.W, a.bias, a.x, a.N, a.E, b, a.rb, s_x, a.job, a.njobs, sv); break;
            default: logits_tile_small<16>(a.W, a.bias, a.x, a.N, a.E, b, a.rb, s_x, a.job, a.njobs, sv); break;
            }
        }
        return;
    } else if (b < a.logit_blocks) {
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
    a.small = !a.wide && (H == 256 || H == 512 || H == 1024 || H == 2048 || H == LS_MAXK * 256);
    a.logit_blocks = a.small ? small_tiles(N, E) : (logit_waves(N, E, a.wide) + 3) / 4;
    int blocks = a.logit_blocks;
    a.njobs = njobs;
    for (int j = 0; j < njobs; j++) {
        if (jobs[j].K % 256) return hipErrorInvalidValue;
        // small tiles convert their own rows (the jobs convert x: rows N, K H)
        if (a.small && (jobs[j].src != x || jobs[j].rows != N || jobs[j].K != H))
            return hipErrorInvalidValue;
        a.job[j] = jobs[j];
        if (!a.small) blocks += (jobs[j].rows * (jobs[j].K / 256) + 3) / 4;
    }
    if (a.small)
        hipLaunchKernelGGL(k_front<true>, dim3(blocks), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(k_front<false>, dim3(blocks), dim3(256), 0, s, a);
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

// p[0 .. n) = v (a kernel, not a memset, so that a caller's graph capture
// records no memset node)
__global__ __launch_bounds__(256) void k_fill_i32(int32_t *__restrict__ p, int32_t v, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

hipError_t launch_fill_i32(int32_t *p, int32_t v, int n, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_i32, dim3((n + 255) / 256), dim3(256), 0, s, p, v, n);
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
