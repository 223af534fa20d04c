// k_expert_tile.hip — grouped Q4_K expert products when many tokens reach each
// expert (the sampler's later windows, N = 32 (blk + 1) of several hundred to
// thousands of tokens, and prompt prefill): src/diffuse-moe-graph.cpp:264-269
// (ggml's mul_mat_id over Q4_K weights with Q8_K activations) and the shared
// expert of :280-286 (F32 activations as two int8 digits), on int8 MFMA.
//
// Units: work-list entries of up to 32 pairs of one expert (two column
// blocks of 16) and chunks of 16 tokens of the shared expert (their a1 / a0
// digit rows interleaved, two blocks of 16 rows).  Items: (unit, row group);
// workgroup b of G runs items b, b + G, b + 2 G, ... (one workgroup per CU,
// each walking its own part of the schedule: no counters).
//   gate/up: 128 h rows; h = silu(g) u goes to HBM as f32 ([pair][moe_ff],
//            [token][shared_ff]) and one conversion launch (k_prep) writes
//            the down products' int8 layout.
//   down:    512 n_embd rows in two passes; products to ye [pair][H] /
//            ys [token][H] for the combine launch.
//
// Memory.  A CU returns vector-memory data in the order it was requested, so
// an activation load issued between the weight loads of later steps waits
// for those HBM reads (measured: a ring of activations one step ahead ran
// ~2 us per step whatever the compute).  Both kernels therefore hold an
// item's activations for the whole reduction in LDS, loaded before its
// steps, and the step loops issue weight loads only: each wavefront streams
// its tiles to two register sets one step ahead (the compiler's own loads:
// its waits are exact), continuing into the next item's first step.  The
// down kernel double-buffers its activations (37 KB per item) and loads the
// next item's at the start of the current one, ahead of its weight loads.
//
// Row groups are multiples of 8 per unit and G is a multiple of 8, so one
// row group of every unit runs on one XCD (workgroup b is placed on XCD
// b % 8), consecutive units together: the chunks of one expert read its
// weights once from HBM and then from that XCD's L2.
//
// Arithmetic: compute_sb, k_expert_q4k's products (the integers of every
// sub-block exact, one f32 epilogue per super-block in super-block order,
// rounded by q4k_epi), so the results equal the column-block kernels' bit
// for bit.
#include "dmoe_q4k.h"
#include "dmoe_q80.h"

#include <type_traits>

namespace dmoe {

constexpr int XT_WAVES = 8;

typedef unsigned int xt_u4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) xt_u4v *xt_gu4v_ptr;

__device__ __forceinline__ uint4 xt_ld_nt16(const void *p)
{
    const xt_u4v v = __builtin_nontemporal_load((xt_gu4v_ptr)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Item k is row group k % rg_n of unit k / rg_n; a unit is work-list entry
// u < n_ec (up to 16 NC pairs), else shared chunk u - n_ec (8 NC tokens).
// Every field is wave-uniform.
constexpr int XR_MAX_NC = 2;
constexpr int XR_MAX_CHUNK = EXPERT_CHUNK * XR_MAX_NC;   // 32
constexpr int XR_ROWS = XT_WAVES * 16;                   // h rows of an item (128)
constexpr int XR_MAX_K = 4096;                           // n_embd the gate/up LDS holds

struct XrItem {
    int rg, e, t_first, nt, nblk;
    bool shared, valid;
};

template <int NC>
__device__ __forceinline__ XrItem xr_decode(const MoeJob &job, int k, int rg_n, int n_ec, int nch)
{
    constexpr int XR_CHUNK = EXPERT_CHUNK * NC, XR_SCHUNK = SHARED_CHUNK * NC;
    XrItem I{};
    const int unit = k / rg_n;
    I.rg = k - unit * rg_n;
    I.valid = unit < n_ec + nch;
    if (!I.valid) return I;
    I.shared = unit >= n_ec;
    if (!I.shared) {
        I.e = ldc(job.wl.ec_expert, unit);
        const int c0 = ldc(job.wl.ec_chunk, unit) * XR_CHUNK;
        I.t_first = ldc(job.offsets, I.e) + c0;
        I.nt = min(XR_CHUNK, ldc(job.counts, I.e) - c0);
        I.nblk = (I.nt + EXPERT_CHUNK - 1) / EXPERT_CHUNK;
    } else {
        I.e = 0;
        I.t_first = (unit - n_ec) * XR_SCHUNK;
        I.nt = min(XR_SCHUNK, job.n_tokens - I.t_first);
        I.nblk = (I.nt + SHARED_CHUNK - 1) / SHARED_CHUNK;
    }
    return I;
}

// Activation row of block row r (0..15) of block c of item I: routed rows
// from the item's staged pair ids (x by token, pid / K, for gate/up; h by
// pair for down); shared items interleave the a1 / a0 digit rows (a0 rows
// start at N).  Rows past the item's last repeat it.
template <bool DOWN>
__device__ __forceinline__ int xr_arow(const XrItem &I, const int32_t *s_pids, int N, int K, int c, int r)
{
    if (I.shared) return I.t_first + min(SHARED_CHUNK * c + (r >> 1), I.nt - 1) + (r & 1) * N;
    const int p = s_pids[min(EXPERT_CHUNK * c + r, I.nt - 1)];
    return DOWN ? p : p / K;
}

// ---------------------------------------------------------------------------
// Weight formats.  Each gives:
//   NC, STEP      column blocks of 16 rows per unit; values of the reduction
//                 per step
//   TILE          bytes of one 16-row tile and step (its stride in HBM for
//                 the tiled int8 layouts)
//   ASTEP         LDS bytes of one block's activation step
//   tile, step    the first step of 16-row tile t16 of a matrix (Kin values
//                 per row) and the byte offset of step s from it
//   Tile, load    a lane's share of a tile step
//   compute2      the products of two tiles against one activation block
//   NR, row       the block rows whose activations a lane loads (NR lookups)
//   Src, src      the activation arrays (x or h; routed or shared)
//   load_act      the loads of one block's activation step into LDS
struct FmtQ4K {
    static constexpr int NC = 2, STEP = 256, TILE = TILE_BYTES, ASTEP = ASTEP_BYTES, NR = 6;
    typedef Q4KTile Tile;
    typedef ActI8 Src;
    __device__ static const uint8_t *tile(const uint8_t *m, int t16, int Kin)
    {
        return m + (size_t)t16 * (Kin / STEP) * TILE;
    }
    __device__ static size_t step(int s) { return (size_t)s * TILE; }
    __device__ static void load(Tile &t, const uint8_t *run, int r16, int g)
    {
        const uint4 *p = reinterpret_cast<const uint4 *>(run);
        t.h = xt_ld_nt16(p + r16);
        t.q0 = xt_ld_nt16(p + (1 + 2 * g) * 16 + r16);
        t.q1 = xt_ld_nt16(p + (2 + 2 * g) * 16 + r16);
    }
    __device__ static void compute2(const Tile (&t)[2], const uint8_t *ast, int r16, int g, float (&acc)[2][4])
    {
        compute_sb<2>(t, ast, r16, g, acc);
    }
    // quants: rows 4j + lane / 16; bs: lanes 0..31, row lane / 2; d: lanes 0..15
    __device__ static int row(int lane, int i)
    {
        return i < 4 ? 4 * i + (lane >> 4) : i == 4 ? (lane >> 1) & 15 : lane & 15;
    }
    __device__ static const Src &src(const MoeJob &j, bool down, bool shared)
    {
        return down ? (shared ? j.ahs : j.ah) : (shared ? j.axs : j.ax);
    }
    __device__ static void load_act(const Src &act, int Kin, int sb, const int (&rows)[NR], uint8_t *st, int lane)
    {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = 4 * j + (lane >> 4);
            lds_load16(act.q + (size_t)rows[j] * Kin + sb * 256 + (((lane & 15) ^ (r & 11)) * 16), st + 1024 * j);
        }
        if (lane < 32) lds_load16(act.bs + (size_t)rows[4] * (Kin / 16) + sb * 16 + (lane & 1) * 8, st + ABS_OFF);
        if (lane < 16) lds_load4(act.d + (size_t)rows[5] * (Kin / 256) + sb, st + AD_OFF);
    }
};

struct FmtQ80 {
    static constexpr int NC = 2, STEP = 256, TILE = Q80_TILE, ASTEP = Q80_ASTEP, NR = 5;
    struct Tile {
        uint4 d, q[4];          // piece 0 of row r16; lane group g's quant pieces
    };
    typedef ActI8 Src;
    __device__ static const uint8_t *tile(const uint8_t *m, int t16, int Kin)
    {
        return m + (size_t)t16 * (Kin / STEP) * TILE;
    }
    __device__ static size_t step(int s) { return (size_t)s * TILE; }
    __device__ static void load(Tile &t, const uint8_t *run, int r16, int g)
    {
        const uint4 *p = reinterpret_cast<const uint4 *>(run);
        t.d = xt_ld_nt16(p + r16);
#pragma unroll
        for (int j = 0; j < 4; j++) t.q[j] = xt_ld_nt16(p + (1 + 4 * g + j) * 16 + r16);
    }
    __device__ static void compute2(const Tile (&t)[2], const uint8_t *ast, int r16, int g, float (&acc)[2][4])
    {
        long a[8];
        q80_act_ops(ast, r16, g, a);
#pragma unroll
        for (int r = 0; r < 2; r++) {
            long w[8];
            q80_w_ops(t[r].q[0], t[r].q[1], t[r].q[2], t[r].q[3], w);
            q80_products(a, w, t[r].d, ast, g, acc[r]);
        }
    }
    // quants: rows 4j + lane / 16; scales: two loads of 64 lanes, lane ->
    // (block 4 h + lane / 16, row lane % 16)
    __device__ static int row(int lane, int i) { return i < 4 ? 4 * i + (lane >> 4) : lane & 15; }
    __device__ static const Src &src(const MoeJob &j, bool down, bool shared)
    {
        return down ? (shared ? j.ahs : j.ah) : (shared ? j.axs : j.ax);
    }
    __device__ static void load_act(const Src &act, int Kin, int sb, const int (&rows)[NR], uint8_t *st, int lane)
    {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = 4 * j + (lane >> 4);
            lds_load16(act.q + (size_t)rows[j] * Kin + sb * 256 + (((lane & 15) ^ (r & 11)) * 16), st + 1024 * j);
        }
#pragma unroll
        for (int h = 0; h < 2; h++)
            lds_load4(act.d + (size_t)rows[4] * (Kin / 32) + sb * 8 + 4 * h + (lane >> 4), st + Q80_AD_OFF + 256 * h);
    }
};

// F16 (ggml's F16 products: activations rounded to f16, products accumulated
// in f32; the shared expert's f32 activations as an f16 hi and lo row): the
// tiled layout of k_gemm.hip (128-row blocks, k-step-major: the 128 rows x 32
// values of k step ks of block b are the 8 KB at (b Kin / 32 + ks) 8192, row
// r at r 64 with its 16-byte chunk q at slot q ^ swz(r), swz(r) = (r >> 1) &
// 3), steps of 128 values = four k steps, one column block per unit (an
// item's activations, 16 rows x 4096 f16, fill 128 KB of LDS).  Activation
// steps in LDS: four 1 KB k steps, row r at r 64, chunk q at slot q ^ swz(r)
// (the operand reads conflict-free, as in k_gemm.hip).
typedef _Float16 xt_h8 __attribute__((ext_vector_type(8)));
typedef float xt_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int xt_swz(int r) { return (r >> 1) & 3; }

struct FmtF16 {
    static constexpr int NC = 1, STEP = 128, TILE = 4 * 1024, ASTEP = 4 * 1024, NR = 1;
    struct Tile {
        uint4 w[4];             // row r16, k chunk g of the step's four k steps
    };
    typedef const uint16_t *Src;
    __device__ static const uint8_t *tile(const uint8_t *m, int t16, int Kin)
    {
        return m + (size_t)(t16 >> 3) * (Kin / 32) * 8192 + (size_t)(t16 & 7) * 1024;
    }
    __device__ static size_t step(int s) { return (size_t)s * 4 * 8192; }
    __device__ static void load(Tile &t, const uint8_t *run, int r16, int g)
    {
        const uint8_t *p = run + r16 * 64 + ((g ^ xt_swz(r16)) * 16);
#pragma unroll
        for (int j = 0; j < 4; j++) t.w[j] = xt_ld_nt16(p + j * 8192);
    }
    __device__ static void compute2(const Tile (&t)[2], const uint8_t *ast, int r16, int g, float (&acc)[2][4])
    {
        const uint8_t *ap = ast + r16 * 64 + ((g ^ xt_swz(r16)) * 16);
#pragma unroll
        for (int r = 0; r < 2; r++) {
            xt_f4 c = {acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const xt_h8 a = *reinterpret_cast<const xt_h8 *>(ap + j * 1024);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(xt_h8, t[r].w[j]), c, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) acc[r][i] = c[i];
        }
    }
    // a k step of 16 rows x 64 bytes is one 64-lane load: lane -> row lane / 4,
    // slot lane % 4 (holding chunk (lane % 4) ^ swz(row))
    __device__ static int row(int lane, int) { return lane >> 2; }
    __device__ static Src src(const MoeJob &j, bool down, bool shared)
    {
        return down ? (shared ? j.hs16 : j.h16) : (shared ? j.xs16 : j.x16);
    }
    __device__ static void load_act(Src act, int Kin, int sb, const int (&rows)[NR], uint8_t *st, int lane)
    {
        const int q = (lane & 3) ^ xt_swz(lane >> 2);
        const uint8_t *p = reinterpret_cast<const uint8_t *>(act + (size_t)rows[0] * Kin) + q * 16;
#pragma unroll
        for (int j = 0; j < 4; j++) lds_load16(p + (size_t)(4 * sb + j) * 64, st + 1024 * j);
    }
};

// ---------------------------------------------------------------------------
// gate/up: h = silu(W_gate x) * (W_up x) for 128 h rows of a unit of up to
// 32 pairs (two column blocks), as f32.
//
// The item's activations for the whole reduction (two blocks x n_embd / 256
// super-blocks, 149.5 KB at n_embd 4096) go to LDS at the item's start, so
// the step loop issues weight loads only: a CU returns vector-memory data in
// issue order, and activation loads issued step by step between the weight
// loads of later steps wait for those HBM reads (measured: a ring of one
// activation step ahead runs ~2 us per step, whatever the compute).  Each
// wavefront streams its gate and up tiles to two register sets, one step
// ahead, across item boundaries (the last step of an item loads the next
// item's first weights: the compiler's own loads, its waits exact).
template <class F>
__global__ __launch_bounds__(XT_WAVES * 64) void k_gu_rr(MoeJob job)
{
    constexpr int XR_NC = F::NC, XR_CHUNK = EXPERT_CHUNK * F::NC, XR_SCHUNK = SHARED_CHUNK * F::NC;
    __shared__ __align__(16) uint8_t s_act[XR_MAX_K / F::STEP][XR_NC * F::ASTEP];
    __shared__ int32_t s_pids[2][XR_CHUNK];          // routed items: their pair ids

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int H = job.H, N = job.n_tokens, K = job.top_k;
    const int n_ec = ldc(job.wl.n_ec, 0);
    const int nch = job.has_shared ? (N + XR_SCHUNK - 1) / XR_SCHUNK : 0;
    const int rg_n = job.FF / XR_ROWS;
    const int nsb = H / F::STEP;
    const int steps = nsb;                 // even (n_embd a multiple of 512)
    const int G = gridDim.x;

    int k = blockIdx.x;
    XrItem I = xr_decode<F::NC>(job, k, rg_n, n_ec, nch);
    if (!I.valid) return;
    if (tid < XR_CHUNK && !I.shared) s_pids[0][tid] = job.perm[I.t_first + min(tid, I.nt - 1)];
    int buf = 0;
    int npid = 0;                          // the next item's pair id of this lane (tid < 32)

    // this wavefront's gate and up tiles of item X (rows rg 128 + 16 wave)
    auto tiles = [&](const XrItem &X, const uint8_t *&tg, const uint8_t *&tu) {
        const WTensor &a = X.shared ? job.sg : job.eg;
        const WTensor &b = X.shared ? job.su : job.eu;
        const int t16 = (X.rg * XR_ROWS + 16 * wave) / 16;
        tg = F::tile(a.data + (size_t)X.e * a.nb2, t16, H);
        tu = F::tile(b.data + (size_t)X.e * b.nb2, t16, H);
    };
    // weight loads run one step ahead over the concatenation of the items:
    // (lg, lu) the cursor's tiles, l_sb its super-block; past the last item
    // the cursor stays on its last step (loaded again, never used)
    const uint8_t *lg, *lu;
    tiles(I, lg, lu);
    int l_sb = 0;
    bool l_last = false;                   // the cursor is on the schedule's last step
    XrItem NI{};
    auto load = [&](typename F::Tile (&o)[2]) __attribute__((always_inline)) {
        F::load(o[0], lg + F::step(l_sb), r16, g);
        F::load(o[1], lu + F::step(l_sb), r16, g);
        if (l_sb + 1 < steps) {
            l_sb++;
        } else if (!l_last) {
            // on to the next item's first step (NI is decoded by then)
            if (NI.valid) {
                tiles(NI, lg, lu);
                l_sb = 0;
            } else {
                l_last = true;
            }
        }
    };
    typename F::Tile o[2][2];
    NI = xr_decode<F::NC>(job, k + G, rg_n, n_ec, nch);
    load(o[0]);
    __syncthreads();                       // the first item's pair list

    for (;;) {
    // the item's activations: wavefront w loads super-blocks w, w + 8, ...
    // of both blocks
    {
        const auto &act = F::src(job, false, I.shared);
        const int32_t *pids = s_pids[buf];
#pragma unroll
        for (int c = 0; c < XR_NC; c++) {
            if (c >= I.nblk) continue;
            int rows[F::NR];
#pragma unroll
            for (int i = 0; i < F::NR; i++) rows[i] = xr_arow<false>(I, pids, N, K, c, F::row(lane, i));
            for (int sb = wave; sb < nsb; sb += XT_WAVES) F::load_act(act, H, sb, rows, &s_act[sb][c * F::ASTEP], lane);
        }
    }
    EXPERT_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // the next item's pair list (used after this item's steps)
    if (tid < XR_CHUNK && NI.valid && !NI.shared) npid = job.perm[NI.t_first + min(tid, NI.nt - 1)];

    float acc[XR_NC][2][4];
#pragma unroll
    for (int c = 0; c < XR_NC; c++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[c][r][i] = 0.0f;
    // (each tile folded once for both blocks, compute_folded2, measured
    // slower: 252 VGPRs against 220, 1.41 against 1.33 ms at 2048 tokens)
    auto step = [&](const typename F::Tile (&t)[2], int s) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < XR_NC; c++)
            if (c < I.nblk) F::compute2(t, &s_act[s][c * F::ASTEP], r16, g, acc[c]);
    };
    for (int s = 0; s < steps; s += 2) {
        load(o[1]);
        step(o[0], s);
        load(o[0]);
        step(o[1], s + 1);
    }

    // h = silu(gate) * up, f32 (the two digits of a shared token summed)
    const int col = I.rg * XR_ROWS + 16 * wave + r16;
    const int32_t *pids = s_pids[buf];
#pragma unroll
    for (int c = 0; c < XR_NC; c++) {
        if (c >= I.nblk) continue;
        if (!I.shared) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = EXPERT_CHUNK * c + 4 * g + i;
                if (q < I.nt) job.h[(size_t)pids[q] * job.FF + col] = silu(acc[c][0][i]) * acc[c][1][i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const int q = SHARED_CHUNK * c + 2 * g + (i >> 1);
                if (q < I.nt)
                    job.hs[(size_t)(I.t_first + q) * job.SF + col] =
                        silu(acc[c][0][i] + acc[c][0][i + 1]) * (acc[c][1][i] + acc[c][1][i + 1]);
            }
        }
    }
    if (tid < XR_CHUNK) s_pids[buf ^ 1][tid] = npid;
    // every wavefront is done with the activations and the pair list
    __syncthreads();
    if (!NI.valid) break;
    I = NI;
    k += G;
    buf ^= 1;
    NI = xr_decode<F::NC>(job, k + G, rg_n, n_ec, nch);
    }
}

// ---------------------------------------------------------------------------
// down: ye [pair][H] / ys [token][H] = W_down h for 512 n_embd rows of a unit
// (two passes of 256: each wavefront two 16-row tiles per pass).
constexpr int XR_DN_TILES = 2;                          // tiles per wavefront and pass
constexpr int XR_DN_PASS = XT_WAVES * 16 * XR_DN_TILES; // 256
constexpr int XR_DN_IT = 2;
constexpr int XR_DN_ROWS = XR_DN_PASS * XR_DN_IT;       // 512
constexpr int XR_DN_MAX_K = 1024;                       // moe_ff the down LDS holds

template <class F>
__global__ __launch_bounds__(XT_WAVES * 64) void k_dn_rr(MoeJob job)
{
    constexpr int XR_NC = F::NC, XR_CHUNK = EXPERT_CHUNK * F::NC, XR_SCHUNK = SHARED_CHUNK * F::NC;
    constexpr int MAX_SB = XR_DN_MAX_K / F::STEP;
    __shared__ __align__(16) uint8_t s_act[2][MAX_SB][XR_NC * F::ASTEP];
    // pair lists of items i, i + 1 (its activations load during item i) and
    // i + 2 (loaded from perm during item i, written at its end)
    __shared__ int32_t s_pids[3][XR_CHUNK];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int H = job.H, FF = job.FF, N = job.n_tokens, K = job.top_k;
    const int n_ec = ldc(job.wl.n_ec, 0);
    const int nch = job.has_shared ? (N + XR_SCHUNK - 1) / XR_SCHUNK : 0;
    const int rg_n = H / XR_DN_ROWS;
    const int nsb = FF / F::STEP;
    const int steps = XR_DN_IT * nsb;      // even
    const int G = gridDim.x;

    int k = blockIdx.x;
    XrItem I = xr_decode<F::NC>(job, k, rg_n, n_ec, nch);
    if (!I.valid) return;
    XrItem NI = xr_decode<F::NC>(job, k + G, rg_n, n_ec, nch);
    if (tid < XR_CHUNK && !I.shared) s_pids[0][tid] = job.perm[I.t_first + min(tid, I.nt - 1)];
    if (tid < XR_CHUNK && NI.valid && !NI.shared) s_pids[1][tid] = job.perm[NI.t_first + min(tid, NI.nt - 1)];
    __syncthreads();

    // activations of item X (its pair list in pids) into buffer b: wavefront
    // w loads the (block, step) pairs w, w + 8, ... of the NC x nsb
    auto load_act = [&](const XrItem &X, const int32_t *pids, int b) {
        const auto &act = F::src(job, true, X.shared);
        for (int i = wave; i < XR_NC * nsb; i += XT_WAVES) {
            const int c = i / nsb, sb = i - c * nsb;
            if (c >= X.nblk) break;
            int rows[F::NR];
#pragma unroll
            for (int q = 0; q < F::NR; q++) rows[q] = xr_arow<true>(X, pids, N, K, c, F::row(lane, q));
            F::load_act(act, FF, sb, rows, &s_act[b][sb][c * F::ASTEP], lane);
        }
    };

    // this wavefront's tiles of pass p of item X: rows rg 512 + 256 p + 32 wave + 16 r
    // (tiles t16 and t16 + 1; pass p's 16 tiles further)
    auto tile0 = [&](const XrItem &X) -> int { return (X.rg * XR_DN_ROWS + 32 * wave) / 16; };
    auto matrix = [&](const XrItem &X) -> const uint8_t * {
        const WTensor &W = X.shared ? job.sd : job.ed;
        return W.data + (size_t)X.e * W.nb2;
    };
    int lt = tile0(I);
    const uint8_t *lm = matrix(I);
    int l_st = 0;                          // the load cursor's step in its item
    bool l_last = false;
    auto load = [&](typename F::Tile (&o)[2]) __attribute__((always_inline)) {
        const int it = l_st >= nsb ? 1 : 0, sb = l_st - it * nsb;
        const int t = lt + it * (XR_DN_PASS / 16);
#pragma unroll
        for (int r = 0; r < 2; r++) F::load(o[r], F::tile(lm, t + r, FF) + F::step(sb), r16, g);
        if (l_st + 1 < steps) {
            l_st++;
        } else if (!l_last) {
            if (NI.valid) {
                lt = tile0(NI);
                lm = matrix(NI);
                l_st = 0;
            } else {
                l_last = true;
            }
        }
    };
    static_assert(XR_DN_IT == 2, "two passes");

    typename F::Tile o[2][2];
    load(o[0]);
    load_act(I, s_pids[0], 0);
    EXPERT_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    int buf = 0, pb = 0;                   // activation buffer (of 2), pair list (of 3)
    int npid = 0;

    for (;;) {
    // item i + 2's pair list (written at the end of this item), then item
    // i + 1's activations into the other buffer (issued here, ahead of this
    // item's weight loads)
    const XrItem NNI = xr_decode<F::NC>(job, k + 2 * G, rg_n, n_ec, nch);
    if (tid < XR_CHUNK && NNI.valid && !NNI.shared) npid = job.perm[NNI.t_first + min(tid, NNI.nt - 1)];
    const int pb1 = pb == 2 ? 0 : pb + 1, pb2 = pb1 == 2 ? 0 : pb1 + 1;
    if (NI.valid) load_act(NI, s_pids[pb1], buf ^ 1);

    float acc[XR_NC][2][4];
#pragma unroll
    for (int c = 0; c < XR_NC; c++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[c][r][i] = 0.0f;
    float *out = I.shared ? job.ys : job.ye;
    const int32_t *pids = s_pids[pb];
    int c_sb = 0, c_it = 0;
    auto step = [&](const typename F::Tile (&t)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < XR_NC; c++)
            if (c < I.nblk) F::compute2(t, &s_act[buf][c_sb][c * F::ASTEP], r16, g, acc[c]);
        if (++c_sb == nsb) {
            // the pass's results (the two digits of a shared token summed)
            const int row0 = I.rg * XR_DN_ROWS + c_it * XR_DN_PASS + 32 * wave + r16;
#pragma unroll
            for (int c = 0; c < XR_NC; c++) {
                if (c >= I.nblk) continue;
                if (!I.shared) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int q = EXPERT_CHUNK * c + 4 * g + i;
                        if (q < I.nt) {
                            float *op = out + (size_t)pids[q] * H + row0;
                            op[0] = acc[c][0][i];
                            op[16] = acc[c][1][i];
                        }
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        const int q = SHARED_CHUNK * c + 2 * g + (i >> 1);
                        if (q < I.nt) {
                            float *op = out + (size_t)(I.t_first + q) * H + row0;
                            op[0] = acc[c][0][i] + acc[c][0][i + 1];
                            op[16] = acc[c][1][i] + acc[c][1][i + 1];
                        }
                    }
                }
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[c][r][i] = 0.0f;
            }
            c_sb = 0;
            c_it++;
        }
    };
    for (int s = 0; s < steps; s += 2) {
        load(o[1]);
        step(o[0]);
        load(o[0]);
        step(o[1]);
    }
    if (tid < XR_CHUNK) s_pids[pb2][tid] = npid;
    // the next item's activations (and its first weights) have landed, and
    // every wavefront is done with this item's buffers
    EXPERT_WAIT_VM(0);
    __syncthreads();
    if (!NI.valid) break;
    I = NI;
    NI = NNI;
    k += G;
    buf ^= 1;
    pb = pb1;
    }
}

// ---------------------------------------------------------------------------
bool expert_tile_ok(int H, int FF, int SF, bool shared)
{
    if (H % 512 || FF % 256 || H % XR_DN_ROWS || FF % XR_ROWS) return false;
    if (H > XR_MAX_K || FF > XR_DN_MAX_K) return false;
    if (shared && SF != FF) return false;
    return true;
}

int expert_tile_chunk(int32_t type) { return EXPERT_CHUNK * (type == DMOE_TYPE_F16 ? FmtF16::NC : FmtQ4K::NC); }

// One workgroup per CU (the gate/up LDS holds one), a multiple of 8 (one row
// group per XCD); each runs its items until the schedule's units end.
hipError_t launch_expert_tile(int phase, const MoeJob &job, hipStream_t s)
{
    const int32_t t = job.eg.type;
    if (t != DMOE_TYPE_Q4_K && t != DMOE_TYPE_Q8_0 && t != DMOE_TYPE_F16) return hipErrorInvalidValue;
    if (!expert_tile_ok(job.H, job.FF, job.SF, job.has_shared) || job.wl.chunk != expert_tile_chunk(t) ||
        !job.wl.n_ec)
        return hipErrorInvalidValue;
    if (t == DMOE_TYPE_F16 ? (!job.x16 || !job.h16 || (job.has_shared && (!job.xs16 || !job.hs16)))
                           : (job.ax.K != job.H || job.ah.K != job.FF))
        return hipErrorInvalidValue;
    if (phase == 0 ? (!job.h || (job.has_shared && !job.hs)) : (!job.ye || (job.has_shared && !job.ys)))
        return hipErrorInvalidValue;
    int n_cu = 0;
    const hipError_t e = device_cu_count(&n_cu);
    if (e != hipSuccess) return e;
    const int grid = ((n_cu + 7) / 8) * 8;
    const dim3 gd(grid), bd(XT_WAVES * 64);
    if (phase == 0) {
        if (t == DMOE_TYPE_Q8_0)
            hipLaunchKernelGGL(k_gu_rr<FmtQ80>, gd, bd, 0, s, job);
        else if (t == DMOE_TYPE_F16)
            hipLaunchKernelGGL(k_gu_rr<FmtF16>, gd, bd, 0, s, job);
        else
            hipLaunchKernelGGL(k_gu_rr<FmtQ4K>, gd, bd, 0, s, job);
    } else {
        if (t == DMOE_TYPE_Q8_0)
            hipLaunchKernelGGL(k_dn_rr<FmtQ80>, gd, bd, 0, s, job);
        else if (t == DMOE_TYPE_F16)
            hipLaunchKernelGGL(k_dn_rr<FmtF16>, gd, bd, 0, s, job);
        else
            hipLaunchKernelGGL(k_dn_rr<FmtQ4K>, gd, bd, 0, s, job);
    }
    return hipGetLastError();
}

} // namespace dmoe
