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
// weight bytes).  Each wavefront reads the super-block's activation operands
// from LDS into registers once for its T tiles; each tile step's weight
// operands are formed once for all blocks (fold_tile), and a token's two
// digit rows share one scale epilogue (their scales differ by exactly 256).
// Weights go to a per-wavefront LDS ring of PJ_WST stages, PJ_WST - 1 tile
// steps ahead; a barrier per super-block publishes its activations.  The
// step counts are fixed at compile time (T, the column blocks NB), so every
// wait on the loads is a constant.  A few thousand rows make too few workgroups of
// whole reductions, so the reduction may be split into KS slices (proj_plan
// weighs workgroup rounds, steps and the slices' reduction): the slices' sums go to
// part [m][s][t][row] and k_proj_reduce (or k_proj_swiglu for the MLP's gate
// and up) adds them in slice order.
#include "dmoe_q4k.h"

#include <type_traits>

namespace dmoe {

constexpr int PJ_WAVES = 8;                       // wavefronts of a workgroup
constexpr int PJ_BLOCKS = PROJ_MAX_TOKENS / 8;    // column blocks of 8 tokens
constexpr int PJ_WST = 5;                         // weight ring stages per wavefront
constexpr int PJ_AHEAD = PJ_WST - 1;              // tile steps in flight
constexpr int PJ_TMAX = 6;                        // tiles per wavefront at most

// s_waitcnt vmcnt(n), lgkmcnt(0) for a compile-time n below 64 (vmcnt bits
// 5:4 at 15:14)
template <int n>
__device__ __forceinline__ void pj_wait()
{
    static_assert(n >= 0 && n < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | 0x70);
}

template <int J0, int J1, class F>
__device__ __forceinline__ void pj_unroll(F &&f)
{
    if constexpr (J0 < J1) {
        f(std::integral_constant<int, J0>());
        pj_unroll<J0 + 1, J1>(f);
    }
}

// A column block's operands of one step, read from LDS ahead of use: the
// four 16-byte activation units, the sums of 16 and the row scales
// (compute_folded's reads).
struct PjOps {
    v4i a[4];
    h4 ab;
    float4 dx;
};

__device__ __forceinline__ void pj_read_ops(PjOps &o, const uint8_t *ast, int r16, int g)
{
    const uint4 *ap = reinterpret_cast<const uint4 *>(ast + r16 * 256);
#pragma unroll
    for (int c = 0; c < 4; c++) o.a[c] = __builtin_bit_cast(v4i, ap[(4 * g + c) ^ (r16 & 11)]);
    o.ab = __builtin_bit_cast(h4, *reinterpret_cast<const uint2 *>(ast + ABS_OFF + r16 * 32 + 8 * g));
    o.dx = *reinterpret_cast<const float4 *>(ast + AD_OFF + 16 * g);
}

// A block's MFMAs (compute_folded's) and, separately, its scale epilogue,
// so that a block's epilogue can follow the next block's MFMAs
struct PjSums {
    v4i sh, sl;
    f4 s2;
    float4 dx;
};

__device__ __forceinline__ void pj_mfma(const Q4KFolded &f, const PjOps &o, PjSums &r)
{
    v4i sh = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[c], f.bh[c], sh, 0, 0, 0);
        sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a[c], f.bl[c], sl, 0, 0, 0);
    }
    f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
    r.s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(o.ab, f.bm, s2, 0, 0, 0);
    r.sh = sh;
    r.sl = sl;
    r.dx = o.dx;
}

// Lane (r16, g) holds block rows 4 g .. 4 g + 3 = the a1 and a0 digit rows
// of tokens 2 g and 2 g + 1 (rows 4 g + 2 u, 4 g + 2 u + 1).  The a0 row's
// scale is the a1 row's / 256 exactly (ACT_SPLIT), so a token's step is
//   dx1 (d (S1 + S0 / 256) - dmin (M1 + M0 / 256))
// with S the integer sums and M the min-term sums of its two rows: one scale
// epilogue per token instead of one per digit row.
__device__ __forceinline__ void pj_epilogue(const Q4KFolded &f, const PjSums &r, float (&acc)[2])
{
    const float dx1[2] = {r.dx.x, r.dx.z};
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int s1 = 8 * r.sh[2 * u] + r.sl[2 * u];
        const int s0 = 8 * r.sh[2 * u + 1] + r.sl[2 * u + 1];
        const float sv = __builtin_fmaf((float)s0, 0.00390625f, (float)s1);
        const float mv = __builtin_fmaf(r.s2[2 * u + 1], 0.00390625f, r.s2[2 * u]);
        acc[u] = __builtin_fmaf(dx1[u], f.d * sv - f.dmin * mv, acc[u]);
    }
}

// T tiles per wavefront, NB column blocks of 8 tokens (N in 8 NB - 7 .. 8 NB).
// Every wavefront runs T tiles (tile indices past the matrix clamped to its
// last tile, their results not stored) and every step count is fixed: the
// weight loads run PJ_AHEAD steps ahead to the end (the last steps load the
// last step's tile again, into ring stages no step reads), and every
// super-block issues an activation step (the last super-block's again at the
// end, into the stage its predecessor used, which every wavefront has
// passed).  So each wait below is a compile-time count and the step body has
// no branch.
template <int T, int NB>
__global__ __launch_bounds__(PJ_WAVES * 64) void k_proj_q4k(ProjJob j)
{
    __shared__ __align__(16) uint8_t s_act[2][NB][ASTEP_BYTES];
    __shared__ __align__(16) uint8_t s_w[PJ_WAVES][PJ_WST][TILE_BYTES];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = j.N, K = j.K, R = j.R, KS = j.KS;
    const int nsb = K / 256, S = nsb / KS;
    const int m = blockIdx.z, sl = blockIdx.y;
    const int ntile = R / 16;
    const int tile0 = blockIdx.x * PJ_WAVES * T + wave;      // tile k: tile0 + 8 k
    const int Q = S * T;                                     // tile steps of every wavefront
    const int nbr = (N + 7) / 8;                             // NB
    const int sb0 = sl * S;
    const uint8_t *wm = j.w[m];
    // this lane's activation load (k_expert.hip's roles): block row ar and its
    // 16-byte unit; wavefronts 0..3 load the q rows, 4 the sums of 16, 5 the
    // scales.  Per block one source pointer at the slice's first super-block
    // and one stride per super-block, fixed for the launch.
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);
    const bool loader = wave < ADMA_WAVES;
    const uint32_t loff = lane * 16;
    const int astride = wave < 4 ? 256 : (wave == 4 ? 32 : 4);
    const int adst = wave < 4 ? 1024 * wave : (wave == 4 ? ABS_OFF : AD_OFF);
    const uint8_t *asrc[NB];
#pragma unroll
    for (int c = 0; c < NB; c++) {
        // block row ar: token 8 c + ar / 2 (the last one repeated past N), digit ar % 2
        const int row = min(8 * c + (ar >> 1), N - 1) + (ar & 1) * N;
        asrc[c] = wave < 4 ? reinterpret_cast<const uint8_t *>(j.x.q + (size_t)row * K + sb0 * 256 + aunit * 16)
                : wave == 4 ? reinterpret_cast<const uint8_t *>(j.x.bs + (size_t)row * (K / 16) + sb0 * 16) +
                                  (lane & 1) * 16
                            : reinterpret_cast<const uint8_t *>(j.x.d + (size_t)row * nsb + sb0);
    }

    // activations of super-block s (clamped to the slice) to stage st (NB
    // loads in a loader wavefront)
    auto issue_a = [&](int s, int st) __attribute__((always_inline)) {
        const int off = min(s, S - 1) * astride;
#pragma unroll
        for (int c = 0; c < NB; c++) {
            const uint8_t *st8 = &s_act[st][c][0] + adst;
            if (wave < 5) {
                if (aload) lds_load16(asrc[c] + off, st8);
            } else if (wave == 5 && aload) {
                lds_load4(asrc[c] + off, st8);
            }
        }
    };
    // weights of tile step q (clamped to the last) to ring stage q % PJ_WST
    auto issue_w = [&](int q) __attribute__((always_inline)) {
        const int qc = min(q, Q - 1);
        const int s = qc / T, k = qc - s * T;
        const int tile = min(tile0 + PJ_WAVES * k, ntile - 1);
        const uint8_t *t = wm + ((size_t)tile * nsb + sb0 + s) * TILE_BYTES;
        const uint8_t *d = &s_w[wave][q % PJ_WST][0];
        lds_load16_sa(t, loff, d);
        lds_load16_sa(t, loff + 1024, d + 1024);
        if (lane < TPIECES - 128) lds_load16_sa(t, loff + 2048, d + 2048);
    };

    float acc[T][NB][2];
#pragma unroll
    for (int k = 0; k < T; k++)
#pragma unroll
        for (int c = 0; c < NB; c++) acc[k][c][0] = acc[k][c][1] = 0.0f;

    // Issue order: A(0), W(0 .. PJ_AHEAD - 1); then per super-block s: wait
    // for A(s) (loaders), barrier, A(s + 1), and per tile step q of s: W(q +
    // PJ_AHEAD), wait for W(q), products.  Loads complete in issue order, so
    // each wait allows exactly the loads issued after the one awaited: 3 per
    // weight step (the third, of lanes 0..15, is one instruction of the
    // wavefront), NB per activation step of a loader.  Before the barrier of
    // super-block s, A(s) has the weight steps issued since after it: PJ_AHEAD
    // at s = 0, T after (one per step of s - 1).  W(q) of step k of s has the
    // PJ_AHEAD weight steps after it and, when k < PJ_AHEAD, A(s + 1), which
    // was issued at the start of s; activation steps of earlier super-blocks
    // that may also follow it (T < PJ_AHEAD) are left out of the count, so
    // the wait is then longer than it need be, never shorter.
    issue_a(0, 0);
    for (int q = 0; q < PJ_AHEAD; q++) issue_w(q);
    for (int s = 0; s < S; s++) {
        if (loader) {
            if (s == 0)
                pj_wait<3 * PJ_AHEAD>();
            else
                pj_wait<3 * T>();
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_a(s + 1, (s + 1) & 1);
        const uint8_t *ast = &s_act[s & 1][0][0];
        // the super-block's activation operands, read once for its T tiles
        PjOps o[NB];
#pragma unroll
        for (int c = 0; c < NB; c++) pj_read_ops(o[c], ast + c * ASTEP_BYTES, r16, g);
#pragma unroll
        for (int k = 0; k < T; k++) {
            const int q = s * T + k;
            issue_w(q + PJ_AHEAD);
            constexpr int nw = 3 * PJ_AHEAD;
            if (k < PJ_AHEAD && loader)
                pj_wait<nw + NB>();
            else
                pj_wait<nw>();
            asm volatile("" ::: "memory");
            // block c + 1's MFMAs are issued before block c's epilogue, which
            // then finds block c's sums ready (two sum sets live at a time)
            Q4KTile t;
            read_tile(t, &s_w[wave][q % PJ_WST][0], r16, g);
            PjSums r[2];
            Q4KFolded f;
            fold_tile(t, g, f);
            pj_mfma(f, o[0], r[0]);
#pragma unroll
            for (int c = 0; c < NB; c++) {
                // (nbr == NB; a run-time test keeps each block's work in a
                // region of its own: merged, the blocks' and steps' products
                // are interleaved past the register file)
                if (c < nbr) {
                    if (c + 1 < NB) pj_mfma(f, o[c + 1], r[(c + 1) & 1]);
                    pj_epilogue(f, r[c & 1], acc[k][c]);
                }
            }
        }
    }
    // the last loads (repeats, never read) have landed before the workgroup
    // ends
    pj_wait<0>();
    // lane (r16, g): outputs of tokens 8 c + 2 g + u (u = 0, 1), weight row
    // r16 of each tile
#pragma unroll
    for (int k = 0; k < T; k++) {
        const int tile = tile0 + PJ_WAVES * k;
        if (tile >= ntile) break;
        const int row = tile * 16 + r16;
#pragma unroll
        for (int c = 0; c < NB; c++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = 8 * c + 2 * g + u;
                if (t >= N) continue;
                const float v = acc[k][c][u];
                if (j.partial)
                    j.out[((size_t)(m * KS + sl) * N + t) * R + row] = v;
                else
                    j.out[(size_t)t * j.ldo + row] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q6_K projections of few tokens (F32 weight semantics: the weights
// d sc_j (q - 32) are exact in binary32; ggml's block_q6_K, tiled by
// k_tile_q6k: a tile step is 16 rows x one super-block, 3360 bytes).
// Per 16-weight sub-block j of weight row r and activation digit row t the
// integer sum M_j = sum q a (q = 0..63, int8 a) comes from one
// v_mfma_i32_16x16x32_i8: the A operand holds a 32-weight pair of sub-blocks
// (k = 8 g + b: lane groups 0, 1 sub-block 2p, groups 2, 3 sub-block 2p + 1),
// the B operand the quants of the lanes of one sub-block and zeros in the
// others, so each MFMA sums exactly one sub-block.  Then
//   S = sum_j sc_j M_j - 32 sum_j sc_j bs_j
// with bs_j the activation row's sum of those 16 digits (the f16 sums of 16 of
// the operand layout): the second sum is one v_mfma_f32_16x16x16f16 of the
// sums against the scales, exact (|terms| < 2^24), so S is the exact integer
// sum_j sc_j sum (q - 32) a.  A token's two digit rows then give
//   d dx1 (S1 + S0 / 256)
// as for Q4_K.  The weight ring holds PJ6_WST stages (3360-byte steps leave
// room for four next to the activation stages).
constexpr int TILE6_BYTES = 16 * Q6K_BYTES;       // 3360
constexpr int PJ6_WST = 4;
constexpr int PJ6_AHEAD = PJ6_WST - 1;
constexpr int PJ6_LOADS = 4;                      // 16-byte LDS-direct loads per weight step

struct Q6Tile {                                   // a lane's share of one tile step
    uint32_t L[8], H[4];                          // its 64 quants (k_tile_q6k's packing)
    uint4 sc;                                     // the row's 16 int8 scales
    float d;
};

__device__ __forceinline__ void read_tile6(Q6Tile &t, const uint8_t *tile, int lane, int r16)
{
    const uint4 *p = reinterpret_cast<const uint4 *>(tile);
    const uint4 a = p[lane], b = p[64 + lane], c = p[128 + lane];
    t.L[0] = a.x; t.L[1] = a.y; t.L[2] = a.z; t.L[3] = a.w;
    t.L[4] = b.x; t.L[5] = b.y; t.L[6] = b.z; t.L[7] = b.w;
    t.H[0] = c.x; t.H[1] = c.y; t.H[2] = c.z; t.H[3] = c.w;
    t.sc = p[192 + r16];
    t.d = h16f(reinterpret_cast<const uint16_t *>(tile + 208 * 16)[r16]);
}

// The tile's B operands (quants of pair p as 8 bytes, k = 8 g + b), masked to
// the lane groups of sub-block 2p (be) and 2p + 1 (bo); the 16 scales as
// integers; the f16 scales of sub-blocks 4 g .. 4 g + 3 (the offset MFMA's B).
struct Q6Folded {
    long be[8], bo[8];
    int sc[16];
    h4 bsc;
    float d;
};

// int -> float with v_cvt_f32_i32 as written: left to the compiler, the
// conversion of a sign-extended byte (sbfe x, 8 k, 8) was folded into
// v_cvt_f32_u32 of an SDWA sign-extended byte, which reads a negative scale
// as 2^32 + sc.
__device__ __forceinline__ float cvt_f32_i32(int v)
{
    float f;
    asm volatile("v_cvt_f32_i32 %0, %1" : "=v"(f) : "v"(v));
    return f;
}

__device__ __forceinline__ void fold_tile6(const Q6Tile &t, int g, Q6Folded &f)
{
    const uint32_t keep = g < 2 ? 0xffffffffu : 0u;
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const uint32_t L = t.L[p], H = t.H[p >> 1];
        uint32_t qa, qb;
        if (p & 1) {
            qa = (L & 0x0f0f0f0fu) | (H & 0x30303030u);
            qb = ((L >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
        } else {
            qa = (L & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
            qb = ((L >> 4) & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
        }
        f.be[p] = (long)(((uint64_t)(qb & keep) << 32) | (qa & keep));
        f.bo[p] = (long)(((uint64_t)(qb & ~keep) << 32) | (qa & ~keep));
    }
    const uint32_t sw[4] = {t.sc.x, t.sc.y, t.sc.z, t.sc.w};
#pragma unroll
    for (int j = 0; j < 16; j++) f.sc[j] = __builtin_amdgcn_sbfe(sw[j >> 2], 8 * (j & 3), 8);
    const uint32_t sg = sw[g];
    f.bsc = (h4){(_Float16)cvt_f32_i32(__builtin_amdgcn_sbfe(sg, 0, 8)),
                 (_Float16)cvt_f32_i32(__builtin_amdgcn_sbfe(sg, 8, 8)),
                 (_Float16)cvt_f32_i32(__builtin_amdgcn_sbfe(sg, 16, 8)),
                 (_Float16)cvt_f32_i32(__builtin_amdgcn_sbfe(sg, 24, 8))};
    f.d = t.d;
}

// One column block: S for the lane's four digit rows, then the two tokens'
// epilogue (as pj_epilogue: the a0 row's scale is the a1 row's / 256).
__device__ __forceinline__ void pj6_block(const Q6Folded &f, const PjOps &o, float (&acc)[2])
{
    const long a[8] = {(long)((uint64_t)(uint32_t)o.a[0][1] << 32 | (uint32_t)o.a[0][0]),
                       (long)((uint64_t)(uint32_t)o.a[0][3] << 32 | (uint32_t)o.a[0][2]),
                       (long)((uint64_t)(uint32_t)o.a[1][1] << 32 | (uint32_t)o.a[1][0]),
                       (long)((uint64_t)(uint32_t)o.a[1][3] << 32 | (uint32_t)o.a[1][2]),
                       (long)((uint64_t)(uint32_t)o.a[2][1] << 32 | (uint32_t)o.a[2][0]),
                       (long)((uint64_t)(uint32_t)o.a[2][3] << 32 | (uint32_t)o.a[2][2]),
                       (long)((uint64_t)(uint32_t)o.a[3][1] << 32 | (uint32_t)o.a[3][0]),
                       (long)((uint64_t)(uint32_t)o.a[3][3] << 32 | (uint32_t)o.a[3][2])};
    f4 c2 = {0.0f, 0.0f, 0.0f, 0.0f};
    c2 = __builtin_amdgcn_mfma_f32_16x16x16f16(o.ab, f.bsc, c2, 0, 0, 0);
    // sum_j sc_j bs_j is an integer below 2^23 in magnitude: exact in the f32
    // accumulator and as a 24-bit multiplicand
    int S[4];
#pragma unroll
    for (int i = 0; i < 4; i++) S[i] = __mul24((int)c2[i], -32);
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const v4i m0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[p], f.be[p], z, 0, 0, 0);
        const v4i m1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[p], f.bo[p], z, 0, 0, 0);
        // |M_j| <= 16 * 63 * 128 and |sc_j| <= 128: 24-bit multiplicands
#pragma unroll
        for (int i = 0; i < 4; i++) {
            S[i] = __mul24(f.sc[2 * p], m0[i]) + S[i];
            asm volatile("" : "+v"(S[i]));
            S[i] = __mul24(f.sc[2 * p + 1], m1[i]) + S[i];
            asm volatile("" : "+v"(S[i]));
        }
    }
    const float dx1[2] = {o.dx.x, o.dx.z};
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const float sv = __builtin_fmaf((float)S[2 * u + 1], 0.00390625f, (float)S[2 * u]);
        acc[u] = __builtin_fmaf(dx1[u], f.d * sv, acc[u]);
    }
}

// The launch structure of k_proj_q4k (work division, activation staging,
// compile-time waits; see there) with Q6_K tile steps: PJ6_LOADS loads per
// weight step (the fourth of lanes 0..17: 3360 = 3 x 1024 + 288 bytes).
template <int T, int NB>
__global__ __launch_bounds__(PJ_WAVES * 64) void k_proj_q6k(ProjJob j)
{
    __shared__ __align__(16) uint8_t s_act[2][NB][ASTEP_BYTES];
    __shared__ __align__(16) uint8_t s_w[PJ_WAVES][PJ6_WST][TILE6_BYTES];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = j.N, K = j.K, R = j.R, KS = j.KS;
    const int nsb = K / 256, S = nsb / KS;
    const int m = blockIdx.z, sl = blockIdx.y;
    const int ntile = R / 16;
    const int tile0 = blockIdx.x * PJ_WAVES * T + wave;
    const int Q = S * T;
    const int nbr = (N + 7) / 8;
    const int sb0 = sl * S;
    const uint8_t *wm = j.w[m];
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);
    const bool loader = wave < ADMA_WAVES;
    const uint32_t loff = lane * 16;
    const int astride = wave < 4 ? 256 : (wave == 4 ? 32 : 4);
    const int adst = wave < 4 ? 1024 * wave : (wave == 4 ? ABS_OFF : AD_OFF);
    const uint8_t *asrc[NB];
#pragma unroll
    for (int c = 0; c < NB; c++) {
        const int row = min(8 * c + (ar >> 1), N - 1) + (ar & 1) * N;
        asrc[c] = wave < 4 ? reinterpret_cast<const uint8_t *>(j.x.q + (size_t)row * K + sb0 * 256 + aunit * 16)
                : wave == 4 ? reinterpret_cast<const uint8_t *>(j.x.bs + (size_t)row * (K / 16) + sb0 * 16) +
                                  (lane & 1) * 16
                            : reinterpret_cast<const uint8_t *>(j.x.d + (size_t)row * nsb + sb0);
    }
    auto issue_a = [&](int s, int st) __attribute__((always_inline)) {
        const int off = min(s, S - 1) * astride;
#pragma unroll
        for (int c = 0; c < NB; c++) {
            const uint8_t *st8 = &s_act[st][c][0] + adst;
            if (wave < 5) {
                if (aload) lds_load16(asrc[c] + off, st8);
            } else if (wave == 5 && aload) {
                lds_load4(asrc[c] + off, st8);
            }
        }
    };
    auto issue_w = [&](int q) __attribute__((always_inline)) {
        const int qc = min(q, Q - 1);
        const int s = qc / T, k = qc - s * T;
        const int tile = min(tile0 + PJ_WAVES * k, ntile - 1);
        const uint8_t *t = wm + ((size_t)tile * nsb + sb0 + s) * TILE6_BYTES;
        const uint8_t *d = &s_w[wave][q % PJ6_WST][0];
        lds_load16_sa(t, loff, d);
        lds_load16_sa(t, loff + 1024, d + 1024);
        lds_load16_sa(t, loff + 2048, d + 2048);
        if (lane < (TILE6_BYTES - 3072) / 16) lds_load16_sa(t, loff + 3072, d + 3072);
    };

    float acc[T][NB][2];
#pragma unroll
    for (int k = 0; k < T; k++)
#pragma unroll
        for (int c = 0; c < NB; c++) acc[k][c][0] = acc[k][c][1] = 0.0f;

    issue_a(0, 0);
    for (int q = 0; q < PJ6_AHEAD; q++) issue_w(q);
    for (int s = 0; s < S; s++) {
        if (loader) {
            if (s == 0)
                pj_wait<PJ6_LOADS * PJ6_AHEAD>();
            else
                pj_wait<PJ6_LOADS * T>();
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_a(s + 1, (s + 1) & 1);
        const uint8_t *ast = &s_act[s & 1][0][0];
        PjOps o[NB];
#pragma unroll
        for (int c = 0; c < NB; c++) pj_read_ops(o[c], ast + c * ASTEP_BYTES, r16, g);
#pragma unroll
        for (int k = 0; k < T; k++) {
            const int q = s * T + k;
            issue_w(q + PJ6_AHEAD);
            constexpr int nw = PJ6_LOADS * PJ6_AHEAD;
            if (k < PJ6_AHEAD && loader)
                pj_wait<nw + NB>();
            else
                pj_wait<nw>();
            asm volatile("" ::: "memory");
            Q6Tile t;
            read_tile6(t, &s_w[wave][q % PJ6_WST][0], lane, r16);
            Q6Folded f;
            fold_tile6(t, g, f);
#pragma unroll
            for (int c = 0; c < NB; c++)
                if (c < nbr) pj6_block(f, o[c], acc[k][c]);
        }
    }
    pj_wait<0>();
#pragma unroll
    for (int k = 0; k < T; k++) {
        const int tile = tile0 + PJ_WAVES * k;
        if (tile >= ntile) break;
        const int row = tile * 16 + r16;
#pragma unroll
        for (int c = 0; c < NB; c++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = 8 * c + 2 * g + u;
                if (t >= N) continue;
                const float v = acc[k][c][u];
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

template <bool Q6, int T, int NB>
static hipError_t proj_launch_nb(int nb, dim3 grid, const ProjJob &j, hipStream_t s)
{
    if constexpr (NB > PJ_BLOCKS) {
        return hipErrorInvalidValue;
    } else {
        if (nb != NB) return proj_launch_nb<Q6, T, NB + 1>(nb, grid, j, s);
        if constexpr (Q6)
            hipLaunchKernelGGL((k_proj_q6k<T, NB>), grid, dim3(PJ_WAVES * 64), 0, s, j);
        else
            hipLaunchKernelGGL((k_proj_q4k<T, NB>), grid, dim3(PJ_WAVES * 64), 0, s, j);
        return hipGetLastError();
    }
}

template <bool Q6, int T>
static hipError_t proj_launch_t(int t, int nb, dim3 grid, const ProjJob &j, hipStream_t s)
{
    if constexpr (T < 1) {
        return hipErrorInvalidValue;
    } else {
        if (t != T) return proj_launch_t<Q6, T - 1>(t, nb, grid, j, s);
        return proj_launch_nb<Q6, T, 1>(nb, grid, j, s);
    }
}

template <bool Q6>
static hipError_t launch_proj(const ProjJob &j, hipStream_t s)
{
    const ProjPlan pl = proj_plan(j.R, j.K, j.M, j.N);
    if (!proj_ok(j.R, j.K, j.N) || j.M < 1 || j.M > 2 || j.KS != pl.KS || j.x.K != j.K ||
        (!j.partial && (j.M != 1 || j.KS != 1 || j.ldo < j.R)))
        return hipErrorInvalidValue;
    const dim3 grid((j.R / 16 + PJ_WAVES * pl.T - 1) / (PJ_WAVES * pl.T), j.KS, j.M);
    const int nb = (j.N + 7) / 8;
    return proj_launch_t<Q6, PJ_TMAX>(pl.T, nb, grid, j, s);
}

hipError_t launch_proj_q4k(const ProjJob &j, hipStream_t s) { return launch_proj<false>(j, s); }

hipError_t launch_proj_q6k(const ProjJob &j, hipStream_t s) { return launch_proj<true>(j, s); }

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
