// k_expert_gemm.hip — Q4_K expert products as a grouped int8-MFMA GEMM when
// many pairs reach each expert (prompt prefill and the sampler's large
// windows, N = 32 (blk + 1) of a thousand tokens and more):
// src/diffuse-moe-graph.cpp:264-269 (ggml's mul_mat_id over Q4_K weights
// with Q8_K activations) and the shared expert of :280-286 (F32 activations
// as two int8 digits).
//
// Units: work-list entries of up to 128 pairs of one expert (eight column
// blocks of 16) and chunks of 64 tokens of the shared expert (their a1 / a0
// digit rows interleaved, eight blocks of 16 rows).  Items: (unit, row
// group); gate/up items hold 128 h rows (wavefront w: the gate and the up
// tile of rows 16 w .. + 15), down items 256 n_embd rows (wavefront w: rows
// 32 w .. + 31, two tiles).  Workgroup b of G (one per CU, G a multiple of
// 8) runs items b, b + G, b + 2 G, ...: with row groups a multiple of 8 per
// unit, one row group of every unit runs on one XCD (workgroup b is placed
// on XCD b % 8) and consecutive units together, so the chunks of one expert
// read its weights once from HBM and then from that XCD's L2.
//
// Pipeline: one step per 256-value super-block of the reduction.  The
// step's 16 weight tiles (36 KB, each a 2304-byte run of the tiled layout)
// and its 128 activation rows (eight 4672-byte blocks) go to one LDS stage
// by LDS-direct loads, two stages, the next step's loads issued before the
// current step is computed and continuing across items.  A CU returns
// vector-memory data in issue order, so the weights and the activations of
// a step travel together.  Each wavefront folds its two tiles' sub-block
// scales into the int8 weight operands once per step (compute_folded's
// sh / sl split) and applies them to all eight blocks: per byte brought into
// the CU an item does 2.5 times the int8 products of a 32-pair unit of the
// tile kernels (k_expert_tile.hip), whose launches are bound by that intake.
//
// Arithmetic: the integer sums of every super-block are compute_sb's exactly
// (8 sum (sh q) a + sum (sl q) a = sum_j sc_j S_j), then one f32 epilogue per
// super-block in super-block order rounded by q4k_epi, so the outputs equal
// the tile and column-block kernels' bit for bit.  h goes to HBM as f32
// ([pair][moe_ff], [token][shared_ff]) and one conversion launch writes the
// down products' int8 layout; the down products go to ye [pair][n_embd] /
// ys [token][n_embd] for the combine launch, as with the tile kernels.
#include "dmoe_q4k.h"

namespace dmoe {

constexpr int XG_WAVES = 8;
constexpr int XG_NC = 8;                                     // column blocks of a unit
constexpr int XG_CHUNK = EXPERT_CHUNK * XG_NC;               // routed pairs of a unit (128)
constexpr int XG_SCHUNK = SHARED_CHUNK * XG_NC;              // shared tokens of a unit (64)
constexpr int XG_GU_ROWS = XG_WAVES * 16;                    // h rows of a gate/up item
constexpr int XG_DN_ROWS = XG_WAVES * 32;                    // n_embd rows of a down item
constexpr int XG_WBYTES = XG_WAVES * 2 * TILE_BYTES;         // weights of a stage (36,864)
constexpr int XG_STAGE = XG_WBYTES + XG_NC * ASTEP_BYTES;    // 74,240
static_assert(XG_STAGE % 16 == 0 && TILE_BYTES % 16 == 0 && ASTEP_BYTES % 16 == 0, "16-byte pieces");
static_assert(TPIECES > 128 && TPIECES <= 144, "a tile is two 64-lane loads and one of 16 lanes");

// Item k is row group k % rg_n of unit k / rg_n; a unit is work-list entry
// u < n_ec, else shared chunk u - n_ec.  Every field is wave-uniform.
struct XgItem {
    int rg, e, t_first, nt, nblk;
    bool shared, valid;
};

__device__ __forceinline__ XgItem xg_decode(const MoeJob &job, int k, int rg_n, int n_ec, int nch)
{
    XgItem I{};
    const int unit = k / rg_n;
    I.rg = k - unit * rg_n;
    I.valid = unit < n_ec + nch;
    if (!I.valid) return I;
    I.shared = unit >= n_ec;
    if (!I.shared) {
        I.e = ldc(job.wl.ec_expert, unit);
        const int c0 = ldc(job.wl.ec_chunk, unit) * XG_CHUNK;
        I.t_first = ldc(job.offsets, I.e) + c0;
        I.nt = min(XG_CHUNK, ldc(job.counts, I.e) - c0);
        I.nblk = (I.nt + EXPERT_CHUNK - 1) / EXPERT_CHUNK;
    } else {
        I.e = 0;
        I.t_first = (unit - n_ec) * XG_SCHUNK;
        I.nt = min(XG_SCHUNK, job.n_tokens - I.t_first);
        I.nblk = (I.nt + SHARED_CHUNK - 1) / SHARED_CHUNK;
    }
    return I;
}

// Activation row of block row r (0..15) of block c: routed rows from the
// item's pair ids (x by token, pid / K, for gate/up; h by pair for down);
// shared items interleave the a1 / a0 digit rows (a0 rows start at N).
// Rows past the item's last repeat it.
template <bool DOWN>
__device__ __forceinline__ int xg_arow(const XgItem &I, const int32_t *s_pids, int N, int K, int c, int r)
{
    if (I.shared) return I.t_first + min(SHARED_CHUNK * c + (r >> 1), I.nt - 1) + (r & 1) * N;
    const int p = s_pids[min(EXPERT_CHUNK * c + r, I.nt - 1)];
    return DOWN ? p : p / K;
}

// LDS-direct load of 16 bytes per active lane from a wave-uniform base plus a
// per-lane offset (lane l's bytes to LDS address lds + 16 l).  No non-temporal hint: the
// chunks of one expert read its weights through L2.
__device__ __forceinline__ void xg_lds16(const void *base, uint32_t voff, uint32_t lds)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint64_t sb = (uint64_t)lo | ((uint64_t)hi << 32);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sb), "s"(m0) : "memory", "m0");
}

// The same for 4 bytes per active lane (to lds + 4 l).
__device__ __forceinline__ void xg_lds4(const void *base, uint32_t voff, uint32_t lds)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint64_t sb = (uint64_t)lo | ((uint64_t)hi << 32);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" : : "v"(voff), "s"(sb), "s"(m0) : "memory", "m0");
}

// Two folded tiles against one block's activations of the step (the
// operands read once for both).
__device__ __forceinline__ void xg_products(const Q4KFolded (&f)[2], const uint8_t *ast, int r16, int g,
                                            float (&acc)[2][4])
{
    const uint4 *ap = reinterpret_cast<const uint4 *>(ast + r16 * 256);
    v4i a[4];
#pragma unroll
    for (int c = 0; c < 4; c++) a[c] = __builtin_bit_cast(v4i, ap[(4 * g + c) ^ (r16 & 11)]);
    const h4 ab = __builtin_bit_cast(h4, *reinterpret_cast<const uint2 *>(ast + ABS_OFF + r16 * 32 + 8 * g));
    const float4 dxv = *reinterpret_cast<const float4 *>(ast + AD_OFF + 16 * g);
    const float dx[4] = {dxv.x, dxv.y, dxv.z, dxv.w};
#pragma unroll
    for (int r = 0; r < 2; r++) {
        v4i sh = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[c], f[r].bh[c], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[c], f[r].bl[c], sl, 0, 0, 0);
        }
        f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
        s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, f[r].bm, s2, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int isum = 8 * sh[i] + sl[i];
            acc[r][i] = q4k_epi(acc[r][i], dx[i], f[r].d, (float)isum, f[r].dmin, s2[i]);
        }
    }
}

template <bool DOWN>
__global__ __launch_bounds__(XG_WAVES * 64) void k_gemm_q4k(MoeJob job)
{
    __shared__ __align__(16) uint8_t S[2][XG_STAGE];
    __shared__ int32_t s_pids[2][XG_CHUNK];          // routed items: their pair ids

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int H = job.H, FF = job.FF, N = job.n_tokens, K = job.top_k;
    const int n_ec = job.wl.n_ec ? ldc(job.wl.n_ec, 0) : 0;   // none: shared units only
    const int nch = job.has_shared ? (N + XG_SCHUNK - 1) / XG_SCHUNK : 0;
    const int rg_n = DOWN ? H / XG_DN_ROWS : FF / XG_GU_ROWS;
    const int Kin = DOWN ? FF : H;
    // down launches of a projection split the reduction into KS slices of
    // `steps` super-blocks (item k: slice k % KS of item k / KS)
    const int KS = DOWN && job.ks > 1 ? job.ks : 1;
    const int steps = Kin / 256 / KS;                // >= 2
    const int G = gridDim.x;

    int k = blockIdx.x;
    XgItem I = xg_decode(job, k / KS, rg_n, n_ec, nch);
    if (!I.valid) return;
    int slice = k % KS;
    XgItem NI = xg_decode(job, (k + G) / KS, rg_n, n_ec, nch);
    int nslice = (k + G) % KS;
    if (tid < XG_CHUNK && !I.shared) s_pids[0][tid] = job.perm[I.t_first + min(tid, I.nt - 1)];
    __syncthreads();

    // The load cursor (one step ahead of the products, across items): this
    // wavefront's two weight tiles and, for wavefront w < the cursor item's
    // blocks, block w's activation arrays (wave-uniform bases) and this
    // lane's byte offsets into them (32-bit: the host keeps every activation
    // array below 2 GiB).
    const uint8_t *wb0 = nullptr, *wb1 = nullptr;
    const uint8_t *aqb = nullptr, *absb = nullptr, *adb = nullptr;
    uint32_t aqo[4] = {0, 0, 0, 0}, abso = 0, ado = 0;
    bool act_on = false;
    // (the cursor's slice cs starts at super-block cs * steps of every row)
    auto set_cursor = [&](const XgItem &C, int cs, const int32_t *pids) {
        const int nsb = Kin / 256, sb0 = cs * steps;
        if (!DOWN) {
            const WTensor &a = C.shared ? job.sg : job.eg;
            const WTensor &b = C.shared ? job.su : job.eu;
            const int t16 = C.rg * (XG_GU_ROWS / 16) + wave;
            wb0 = a.data + (size_t)C.e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
            wb1 = b.data + (size_t)C.e * b.nb2 + (size_t)t16 * nsb * TILE_BYTES;
        } else {
            const WTensor &W = C.shared ? job.sd : job.ed;
            const int t16 = C.rg * (XG_DN_ROWS / 16) + 2 * wave;
            wb0 = W.data + (size_t)C.e * W.nb2 + ((size_t)t16 * nsb + sb0) * TILE_BYTES;
            wb1 = wb0 + (size_t)nsb * TILE_BYTES;
        }
        act_on = wave < C.nblk;
        if (act_on) {
            const ActI8 &A = DOWN ? (C.shared ? job.ahs : job.ah) : (C.shared ? job.axs : job.ax);
            aqb = reinterpret_cast<const uint8_t *>(A.q) + (size_t)sb0 * 256;
            absb = reinterpret_cast<const uint8_t *>(A.bs) + (size_t)sb0 * 32;
            adb = reinterpret_cast<const uint8_t *>(A.d) + (size_t)sb0 * 4;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = 4 * j + (lane >> 4);
                aqo[j] = (uint32_t)xg_arow<DOWN>(C, pids, N, K, wave, r) * (uint32_t)Kin + (((lane & 15) ^ (r & 11)) * 16);
            }
            abso = ((uint32_t)xg_arow<DOWN>(C, pids, N, K, wave, (lane >> 1) & 15) * (uint32_t)(Kin / 16) + (lane & 1) * 8) * 2;
            ado = (uint32_t)xg_arow<DOWN>(C, pids, N, K, wave, lane & 15) * (uint32_t)(Kin / 256) * 4;
        }
    };
    // the cursor's super-block sb into stage st (LDS addresses as 32-bit
    // offsets of the LDS aperture)
    const uint32_t s_lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)&S[0][0];
    auto issue = [&](int st, int sb) {
        const uint32_t wd = s_lds + st * XG_STAGE + wave * (2 * TILE_BYTES);
        const uint8_t *s0 = wb0 + (size_t)sb * TILE_BYTES, *s1 = wb1 + (size_t)sb * TILE_BYTES;
        const uint32_t vo = (uint32_t)lane * 16;
        xg_lds16(s0, vo, wd);
        xg_lds16(s0, vo + 1024, wd + 1024);
        xg_lds16(s1, vo, wd + TILE_BYTES);
        xg_lds16(s1, vo + 1024, wd + TILE_BYTES + 1024);
        if (lane < TPIECES - 128) {
            xg_lds16(s0, vo + 2048, wd + 2048);
            xg_lds16(s1, vo + 2048, wd + TILE_BYTES + 2048);
        }
        if (act_on) {
            const uint32_t ad = s_lds + st * XG_STAGE + XG_WBYTES + wave * ASTEP_BYTES;
            const uint8_t *qb = aqb + (size_t)sb * 256;
#pragma unroll
            for (int j = 0; j < 4; j++) xg_lds16(qb, aqo[j], ad + 1024 * j);
            if (lane < 32) xg_lds16(absb + (size_t)sb * 32, abso, ad + ABS_OFF);
            if (lane < 16) xg_lds4(adb + (size_t)sb * 4, ado, ad + AD_OFF);
        }
    };

    set_cursor(I, slice, s_pids[0]);
    issue(0, 0);
    int stg = 0;                                      // the stage the products read
    int buf = 0;                                      // the pair list of item I
    int npid = 0;                                     // the next item's pair id (tid < 128)

    for (;;) {
        float acc[XG_NC][2][4];
#pragma unroll
        for (int c = 0; c < XG_NC; c++)
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[c][r][i] = 0.0f;

        for (int s = 0; s < steps; s++) {
            // the next item's pair list (loaded during step 0) to LDS, then
            // this step's stage landed in every wavefront and the other stage
            // read by all of them
            if (s == 1 && tid < XG_CHUNK) s_pids[buf ^ 1][tid] = npid;
            EXPERT_WAIT_VM(0);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (s + 1 < steps) {
                issue(stg ^ 1, s + 1);
            } else if (NI.valid) {
                set_cursor(NI, nslice, s_pids[buf ^ 1]);
                issue(stg ^ 1, 0);
            }
            if (s == 0 && tid < XG_CHUNK && NI.valid && !NI.shared)
                npid = job.perm[NI.t_first + min(tid, NI.nt - 1)];

            const uint8_t *st = S[stg];
            Q4KFolded f[2];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                Q4KTile t;
                read_tile(t, st + wave * (2 * TILE_BYTES) + r * TILE_BYTES, r16, g);
                fold_tile(t, g, f[r]);
            }
#pragma unroll
            for (int c = 0; c < XG_NC; c++)
                if (c < I.nblk) xg_products(f, st + XG_WBYTES + c * ASTEP_BYTES, r16, g, acc[c]);
            stg ^= 1;
        }

        const int32_t *pids = s_pids[buf];
        if (!DOWN) {
            // h = silu(gate) * up, f32 (the two digits of a shared token summed)
            const int col = I.rg * XG_GU_ROWS + 16 * wave + r16;
#pragma unroll
            for (int c = 0; c < XG_NC; c++) {
                if (c >= I.nblk) continue;
                if (!I.shared) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int q = EXPERT_CHUNK * c + 4 * g + i;
                        if (q < I.nt) job.h[(size_t)pids[q] * FF + col] = silu(acc[c][0][i]) * acc[c][1][i];
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
        } else {
            const int row0 = I.rg * XG_DN_ROWS + 32 * wave + r16;
            float *out = I.shared ? job.ys + (size_t)slice * N * H : job.ye;
#pragma unroll
            for (int c = 0; c < XG_NC; c++) {
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
            }
        }
        if (!NI.valid) break;
        I = NI;
        slice = nslice;
        k += G;
        buf ^= 1;
        NI = xg_decode(job, (k + G) / KS, rg_n, n_ec, nch);
        nslice = (k + G) % KS;
    }
    // every wavefront leaves with no loads in flight
    EXPERT_WAIT_VM(0);
}

// ---------------------------------------------------------------------------
bool expert_gemm_q4k_ok(int H, int FF, int SF, bool shared)
{
    if (H % XG_DN_ROWS || FF % XG_GU_ROWS || H < 512 || FF < 512 || H % 256 || FF % 256) return false;
    if (shared && SF != FF) return false;
    return true;
}

// One workgroup per CU (the two stages fill the LDS), a multiple of 8 (one
// row group per XCD); each runs its items until the schedule's units end.
hipError_t launch_expert_gemm_q4k(int phase, const MoeJob &job, hipStream_t s)
{
    // routed experts (eg / eu / ed), the shared one (sg / su / sd) or both;
    // a projection is a down launch of shared units only (no routed weights;
    // the work list's count may be null there), optionally in ks reduction
    // slices
    const bool routed = job.eg.data || job.ed.data;
    const WTensor &wr = phase == 0 ? job.eg : job.ed, &ws = phase == 0 ? job.sg : job.sd;
    if ((routed && wr.type != DMOE_TYPE_Q4_K) || (job.has_shared && ws.type != DMOE_TYPE_Q4_K) ||
        (!routed && !job.has_shared))
        return hipErrorInvalidValue;
    if (!expert_gemm_q4k_ok(job.H, job.FF, job.SF, job.has_shared) || job.wl.chunk != XG_CHUNK ||
        (routed && !job.wl.n_ec))
        return hipErrorInvalidValue;
    if (phase == 0 ? ((routed && job.ax.K != job.H) || (job.has_shared && job.axs.K != job.H))
                   : ((routed && job.ah.K != job.FF) || (job.has_shared && job.ahs.K != job.SF)))
        return hipErrorInvalidValue;
    // slices (read by the down launch only): shared units only, each slice
    // two or more super-blocks
    if (phase == 1 && job.ks > 1 && (routed || (job.FF / 256) % job.ks || job.FF / 256 / job.ks < 2))
        return hipErrorInvalidValue;
    // the activation arrays' byte offsets are 32-bit: x (N rows, two digit
    // rows per token for the shared expert) and h (N k and 2 N rows)
    const long N = job.n_tokens;
    if (phase == 0 ? 2L * N * job.H >= (1L << 31)
                   : N * job.top_k * job.FF >= (1L << 31) || 2L * N * job.SF >= (1L << 31))
        return hipErrorInvalidValue;
    if (phase == 0 ? ((routed && !job.h) || (job.has_shared && !job.hs))
                   : ((routed && !job.ye) || (job.has_shared && !job.ys)))
        return hipErrorInvalidValue;
    int n_cu = 0;
    const hipError_t e = device_cu_count(&n_cu);
    if (e != hipSuccess) return e;
    const int grid = ((n_cu + 7) / 8) * 8;
    if (phase == 0)
        hipLaunchKernelGGL(k_gemm_q4k<false>, dim3(grid), dim3(XG_WAVES * 64), 0, s, job);
    else
        hipLaunchKernelGGL(k_gemm_q4k<true>, dim3(grid), dim3(XG_WAVES * 64), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
