// k_proj.hip — Q4_K projections of few tokens (at most PROJ_MAX_TOKENS) with
// F32 weight semantics: the attention half's fused QKV and output
// projections (src/diffuse-moe-graph.cpp:124, :172), the dense layer-0 MLP
// (:181-187) and the LM head (:299).  x arrives as two int8 digit rows per
// token (ACT_SPLIT, dmoe_prep.h: a1 rows 0..N-1, a0 rows N..2N-1, each digit
// row with its own scale per super-block), so a token's product is the sum of
// its two digit rows' products.
//
// Work division.  Workgroup (b, s, m) takes 128 T output rows of matrix m --
// wavefront w the 16-row tiles 8 (T b + k) + w, k < T, whose accumulators it
// keeps for the whole launch -- the super-blocks s S .. s S + S - 1 of the
// reduction (slice s), and every token: column block c holds tokens
// 8 c .. 8 c + 7 as 16 rows (each token's a1 and a0 interleaved).  Per
// super-block the column blocks are loaded once into LDS (k_expert.hip's
// activation layout, two stages) and shared by the eight wavefronts, which
// each run through their T tiles of that super-block; so the activations are
// read once per 128 T rows (T = 5 for the 157,184-row LM head: a fifth of the
// weight bytes).  Each tile step's operands are formed once for all blocks
// (fold_tile / compute_folded).  Weights go to a per-wavefront LDS ring of
// PJ_WST stages, PJ_WST - 1 tile steps ahead; a barrier per super-block
// publishes its activations.  A few thousand rows make too few workgroups of
// whole reductions, so the reduction may be split into KS slices (proj_plan
// weighs workgroup rounds, steps and the slices' reduction): the slices' sums go to
// part [m][s][t][row] and k_proj_reduce (or k_proj_swiglu for the MLP's gate
// and up) adds them in slice order.
#include "dmoe_q4k.h"

namespace dmoe {

constexpr int PJ_WAVES = 8;                       // wavefronts of a workgroup
constexpr int PJ_BLOCKS = PROJ_MAX_TOKENS / 8;    // column blocks of 8 tokens
constexpr int PJ_WST = 5;                         // weight ring stages per wavefront
constexpr int PJ_AHEAD = PJ_WST - 1;              // tile steps in flight
constexpr int PJ_TMAX = 6;                        // tiles per wavefront at most

// s_waitcnt vmcnt(n), lgkmcnt(0) for a wave-uniform n below 32 (the counter
// field is an immediate: one case per value; vmcnt bits 5:4 at 15:14)
#define PJ_WAIT_CASE(n)                                                              \
    case n: __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x70); break;
__device__ __forceinline__ void pj_wait_vm(int n)
{
    switch (n) {
        PJ_WAIT_CASE(0) PJ_WAIT_CASE(1) PJ_WAIT_CASE(2) PJ_WAIT_CASE(3) PJ_WAIT_CASE(4) PJ_WAIT_CASE(5)
        PJ_WAIT_CASE(6) PJ_WAIT_CASE(7) PJ_WAIT_CASE(8) PJ_WAIT_CASE(9) PJ_WAIT_CASE(10) PJ_WAIT_CASE(11)
        PJ_WAIT_CASE(12) PJ_WAIT_CASE(13) PJ_WAIT_CASE(14) PJ_WAIT_CASE(15) PJ_WAIT_CASE(16) PJ_WAIT_CASE(17)
        PJ_WAIT_CASE(18) PJ_WAIT_CASE(19) PJ_WAIT_CASE(20) PJ_WAIT_CASE(21) PJ_WAIT_CASE(22) PJ_WAIT_CASE(23)
        PJ_WAIT_CASE(24) PJ_WAIT_CASE(25) PJ_WAIT_CASE(26) PJ_WAIT_CASE(27) PJ_WAIT_CASE(28) PJ_WAIT_CASE(29)
        PJ_WAIT_CASE(30) PJ_WAIT_CASE(31)
    default: __builtin_amdgcn_s_waitcnt(0x70); break;
    }
}
#undef PJ_WAIT_CASE

template <int T>
__global__ __launch_bounds__(PJ_WAVES * 64) void k_proj_q4k(ProjJob j)
{
    __shared__ __align__(16) uint8_t s_act[2][PJ_BLOCKS][ASTEP_BYTES];
    __shared__ __align__(16) uint8_t s_w[PJ_WAVES][PJ_WST][TILE_BYTES];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = j.N, K = j.K, R = j.R, KS = j.KS;
    const int nsb = K / 256, S = nsb / KS;
    const int m = blockIdx.z, sl = blockIdx.y;
    const int ntile = R / 16;
    const int tile0 = blockIdx.x * PJ_WAVES * T + wave;      // tile k: tile0 + 8 k
    // this wavefront's tiles: a prefix k < ntw of the T
    const int ntw = tile0 >= ntile ? 0 : min(T, (ntile - 1 - tile0) / PJ_WAVES + 1);
    const int Q = S * ntw;                                   // its tile steps
    const int sb0 = sl * S;
    const int NB = (N + 7) / 8;
    const uint8_t *wm = j.w[m];
    // this lane's activation load (k_expert.hip's roles): block row ar and its
    // 16-byte unit; wavefronts 0..3 load the q rows, 4 the sums of 16, 5 the
    // scales
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);
    const bool loader = wave < ADMA_WAVES;
    const uint32_t loff = lane * 16;

    // activations of super-block s to stage s % 2 (NB loads in a loader wavefront)
    auto issue_a = [&](int s) {
        const int sb = sb0 + s;
#pragma unroll
        for (int c = 0; c < PJ_BLOCKS; c++) {
            if (c >= NB) break;
            // block row ar: token 8 c + ar / 2 (the last one repeated past N), digit ar % 2
            const int row = min(8 * c + (ar >> 1), N - 1) + (ar & 1) * N;
            uint8_t *st8 = &s_act[s & 1][c][0];
            if (wave < 4)
                lds_load16(j.x.q + (size_t)row * K + sb * 256 + aunit * 16, st8 + 1024 * wave);
            else if (wave == 4 && aload)
                lds_load16(j.x.bs + (size_t)row * (K / 16) + sb * 16 + (lane & 1) * 8, st8 + ABS_OFF);
            else if (wave == 5 && aload)
                lds_load4(j.x.d + (size_t)row * nsb + sb, st8 + AD_OFF);
        }
    };
    // weights of tile step q (super-block q / ntw of tile q % ntw) to ring stage q % PJ_WST
    auto issue_w = [&](int q) {
        const int s = q / ntw, k = q - s * ntw;
        const uint8_t *t = wm + ((size_t)(tile0 + PJ_WAVES * k) * nsb + sb0 + s) * TILE_BYTES;
        const uint8_t *d = &s_w[wave][q % PJ_WST][0];
        lds_load16_sa(t, loff, d);
        lds_load16_sa(t, loff + 1024, d + 1024);
        if (lane < TPIECES - 128) lds_load16_sa(t, loff + 2048, d + 2048);
    };

    float acc[T][PJ_BLOCKS][4];
#pragma unroll
    for (int k = 0; k < T; k++)
#pragma unroll
        for (int c = 0; c < PJ_BLOCKS; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[k][c][i] = 0.0f;

    // Issue order: A(0), W(0 .. PJ_AHEAD - 1); then per super-block s: wait
    // for A(s) (loaders), barrier, A(s + 1), and per tile step q of s: W(q +
    // PJ_AHEAD), wait for W(q), products.  Loads complete in issue order, so
    // each wait allows exactly the loads issued after the one awaited (3 per
    // weight step, NB per activation step of a loader).
    issue_a(0);
    for (int q = 0; q < min(PJ_AHEAD, Q); q++) issue_w(q);
    for (int s = 0; s < S; s++) {
        if (loader) {
            const int cnt = s == 0 ? min(PJ_AHEAD, Q)
                                   : max(0, min(Q, s * ntw + PJ_AHEAD) - ((s - 1) * ntw + PJ_AHEAD));
            pj_wait_vm(3 * cnt);
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 1 < S) issue_a(s + 1);
#pragma unroll
        for (int k = 0; k < T; k++) {
            if (k >= ntw) break;
            const int q = s * ntw + k;
            if (q + PJ_AHEAD < Q) issue_w(q + PJ_AHEAD);
            // loads issued after W(q): the weight steps ahead of it and the
            // activation steps issued since (super-blocks past the one W(q)
            // was issued in)
            const int iss = q < PJ_AHEAD ? -1 : (q - PJ_AHEAD) / ntw;
            const int a_lo = max(1, iss + 2), a_hi = min(s + 1, S - 1);
            const int cnt_a = loader ? max(0, a_hi - a_lo + 1) : 0;
            pj_wait_vm(3 * min(PJ_AHEAD, Q - 1 - q) + NB * cnt_a);
            asm volatile("" ::: "memory");
            Q4KTile t;
            read_tile(t, &s_w[wave][q % PJ_WST][0], r16, g);
            Q4KFolded f;
            fold_tile(t, g, f);
#pragma unroll
            for (int c = 0; c < PJ_BLOCKS; c++)
                if (c < NB) compute_folded(f, &s_act[s & 1][c][0], r16, g, acc[k][c]);
        }
    }
    // lane (r16, g): outputs of block rows 4 g + i = token 8 c + 2 g + i / 2,
    // digit i % 2; the token's value is the sum of its two digits' products
#pragma unroll
    for (int k = 0; k < T; k++) {
        if (k >= ntw) break;
        const int row = (tile0 + PJ_WAVES * k) * 16 + r16;
#pragma unroll
        for (int c = 0; c < PJ_BLOCKS; c++) {
            if (c >= NB) break;
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const int t = 8 * c + 2 * g + (i >> 1);
                if (t >= N) continue;
                const float v = acc[k][c][i] + acc[k][c][i + 1];
                if (j.partial)
                    j.out[((size_t)(m * KS + sl) * N + t) * R + row] = v;
                else
                    j.out[(size_t)t * j.ldo + row] = v;
            }
        }
    }
}

// y [N][ldy] = the slices' sums, added in slice order (four rows' values per
// thread)
__global__ __launch_bounds__(256) void k_proj_reduce(const float4 *__restrict__ part, int KS, int N, int R4,
                                                     float4 *__restrict__ y, int ldy4)
{
#pragma clang fp contract(off)
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N * R4) return;
    const int t = i / R4, r = i - t * R4;
    float4 a = part[(size_t)t * R4 + r];
    for (int k = 1; k < KS; k++) {
        const float4 b = part[((size_t)k * N + t) * R4 + r];
        a.x = a.x + b.x;
        a.y = a.y + b.y;
        a.z = a.z + b.z;
        a.w = a.w + b.w;
    }
    y[(size_t)t * ldy4 + r] = a;
}

// The dense MLP's h = silu(gate) up from the gate (matrix 0) and up (matrix
// 1) slices, each added in slice order, converted to two int8 digit rows per
// token for the down projection (prep_values, ACT_SPLIT); one wavefront per
// (token, super-block of h).
__global__ __launch_bounds__(256) void k_proj_swiglu(const float *__restrict__ part, int KS, int N, int R,
                                                     ActI8 ah)
{
#pragma clang fp contract(off)
    __shared__ float s_v[4][256];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nsb = R / 256;
    const int task = blockIdx.x * 4 + w;
    if (task >= N * nsb) return;
    const int t = task / nsb, sb = task - t * nsb;
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int f = sb * 256 + lane + 64 * c;
        float gsum = part[(size_t)t * R + f];
        float usum = part[((size_t)KS * N + t) * R + f];
        for (int k = 1; k < KS; k++) {
            gsum = gsum + part[((size_t)k * N + t) * R + f];
            usum = usum + part[((size_t)(KS + k) * N + t) * R + f];
        }
        v[c] = silu(gsum) * usum;
    }
    prep_values(v, ah, ACT_SPLIT, t, N, sb, nsb, s_v[w]);
}

// Tiles per wavefront (T) and reduction slices (KS, a divisor of K / 256)
// for a shape, by a cost model fitted to measured launches on the 256-CU
// part this is built for (at 32 tokens): a launch takes about 8 us plus
// 1.9 us per tile step of a wavefront (T S) and round of workgroups over the
// CUs, and the slices' sums, when there are several, about 2 us plus 0.6 us
// per MB to add (k_proj_reduce / k_proj_swiglu); the activation steps every
// workgroup reads from L2 (4.7 KB per 8 tokens and super-block) count 0.1 us
// per MB.  Ties go to more tiles per wavefront.
ProjPlan proj_plan(int R, int K, int M, int N)
{
    const int tiles = R / 16, nsb = K / 256;
    const int nb = (N + 7) / 8;
    ProjPlan best{1, nsb};
    double best_us = -1.0;
    for (int t = PJ_TMAX; t >= 1; t--)
        for (int ks = 1; ks <= nsb; ks++) {
            if (nsb % ks) continue;
            const long wgs = (long)((tiles + PJ_WAVES * t - 1) / (PJ_WAVES * t)) * M * ks;
            const long rounds = (wgs + 255) / 256;
            double us = 8.0 + 1.9 * t * (nsb / ks) * rounds;
            if (ks > 1) us += 2.0 + 0.6 * ((double)M * ks * N * R * 4 / 1e6);
            us += 0.1 * ((double)wgs * (nsb / ks) * nb * ASTEP_BYTES / 1e6);
            if (best_us < 0.0 || us < best_us) {
                best_us = us;
                best = ProjPlan{t, ks};
            }
        }
    return best;
}

bool proj_ok(int R, int K, int N)
{
    return R > 0 && R % 16 == 0 && K > 0 && K % 256 == 0 && N > 0 && N <= PROJ_MAX_TOKENS;
}

size_t proj_partial_floats(int R, int K, int M, int N)
{
    return (size_t)M * proj_plan(R, K, M, N).KS * N * R;
}

hipError_t launch_proj_q4k(const ProjJob &j, hipStream_t s)
{
    const ProjPlan pl = proj_plan(j.R, j.K, j.M, j.N);
    if (!proj_ok(j.R, j.K, j.N) || j.M < 1 || j.M > 2 || j.KS != pl.KS || j.x.K != j.K ||
        (!j.partial && (j.M != 1 || j.KS != 1 || j.ldo < j.R)))
        return hipErrorInvalidValue;
    const dim3 grid((j.R / 16 + PJ_WAVES * pl.T - 1) / (PJ_WAVES * pl.T), j.KS, j.M);
    switch (pl.T) {
    case 1: hipLaunchKernelGGL(k_proj_q4k<1>, grid, dim3(PJ_WAVES * 64), 0, s, j); break;
    case 2: hipLaunchKernelGGL(k_proj_q4k<2>, grid, dim3(PJ_WAVES * 64), 0, s, j); break;
    case 3: hipLaunchKernelGGL(k_proj_q4k<3>, grid, dim3(PJ_WAVES * 64), 0, s, j); break;
    case 4: hipLaunchKernelGGL(k_proj_q4k<4>, grid, dim3(PJ_WAVES * 64), 0, s, j); break;
    case 5: hipLaunchKernelGGL(k_proj_q4k<5>, grid, dim3(PJ_WAVES * 64), 0, s, j); break;
    default: hipLaunchKernelGGL(k_proj_q4k<6>, grid, dim3(PJ_WAVES * 64), 0, s, j); break;
    }
    return hipGetLastError();
}

hipError_t launch_proj_reduce(const float *part, int KS, int N, int R, float *y, int ldy, hipStream_t s)
{
    if (R % 4 || ldy % 4 || KS < 1 || N < 1) return hipErrorInvalidValue;
    const int n = N * (R / 4);
    hipLaunchKernelGGL(k_proj_reduce, dim3((n + 255) / 256), dim3(256), 0, s,
                       reinterpret_cast<const float4 *>(part), KS, N, R / 4, reinterpret_cast<float4 *>(y), ldy / 4);
    return hipGetLastError();
}

hipError_t launch_proj_swiglu(const float *part, int KS, int N, int R, const ActI8 &ah, hipStream_t s)
{
    if (R % 256 || ah.K != R || KS < 1 || N < 1) return hipErrorInvalidValue;
    const int tasks = N * (R / 256);
    hipLaunchKernelGGL(k_proj_swiglu, dim3((tasks + 3) / 4), dim3(256), 0, s, part, KS, N, R, ah);
    return hipGetLastError();
}

} // namespace dmoe
