// k_gemm.hip — grouped F16 expert products on MFMA (gfx950), the prefill path.
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 for F16
// expert weights (ggml's mul_mat_id converts the activations to F16, its
// vec_dot_type, and accumulates f16 x f16 products in f32) and the shared
// expert of :280-286 (F32 semantics: its F16 weights are exact, the f32
// activations run as two f16 passes, hi = f16(x) and lo = f16(x - hi)):
//   phase 0: h = silu(W_gate x) * (W_up x), written as the f16 activations of
//            phase 1 (routed) or as their hi / lo pair (shared)
//   phase 1: y = W_down h
//
// Work item: one expert, a block of up to 128 of its (token, slot) pairs (or
// 128 tokens of the shared expert) and a group of output rows (256 moe_ff rows
// of gate and of up, or 512 n_embd rows of down).  Items of one expert and
// row group but different pair blocks are a row-group count apart, so they run
// together and share the weight rows through the caches.  Each 32-wide k
// step stages the 128 activation rows (8 KB) and the 512 weight rows (32 KB)
// in LDS with the LDS-direct global loads (global_load_lds_dwordx4: no
// registers held, so a 4-stage ring keeps three steps of loads in flight to
// cover HBM latency); each of the 8 wavefronts computes a 128 x 64 output
// tile (all 128 activation rows, its own 64 weight rows) as 8 x 4
// v_mfma_f32_16x16x32_f16 (operand layout as in k_expert.hip: srcA lane l =
// activation row l%16, k = 8*(l/16)+e; srcB = weight row, same k; D lane l =
// weight row l%16, activation rows 4*(l/16)+i).  (Items of 256 pairs x 256
// weight rows, half of every stage the activation tile: the touched experts'
// pairs, ~100 on average at the prefill's routing, padded 2.9x, and the
// weights streamed at ~3.5 TB/s.)
#include "dmoe_internal.h"

#include <type_traits>

namespace dmoe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int GWAVES = 8;
constexpr int GT = GWAVES * 64;      // threads per workgroup
constexpr int GNW = 512;             // weight rows per item (gate/up: 256 moe_ff rows of each)
constexpr int GS = 4;                // LDS pipeline stages (4 x 40 KB: all of the CU's LDS)
constexpr int GTA = GM * GK * 2;     // bytes of a stage's activation tile (64-byte rows)
constexpr int GTW = GNW * GK * 2;    // bytes of a stage's weight tile
constexpr int GSTAGE = GTA + GTW;
constexpr int GPA = GTA / 16 / GT;   // 16-byte pieces per thread and stage: activations
constexpr int GPW = GTW / 16 / GT;   // weights
constexpr int GLOADS = GPA + GPW;    // LDS-direct loads per thread and stage

__device__ __forceinline__ float gsilu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ uint16_t f2h_rn(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// The 16-byte k-chunk q (0..3) of tile row r sits in slot q ^ swz(r) of the
// row.  A ds_read_b128 serves 16 lanes per cycle over the 64 banks: the four
// lane quads (4 consecutive lanes) of one half-wave whose quad indices have
// equal bit parity (measured on gfx950 with the LDS bank-conflict counter).
// The operand reads (lane l: row l % 16, chunk l / 16) are conflict-free
// with the slot flipped by row bits 1..2.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }

// s_waitcnt with vmcnt(n) (n < 64) and lgkmcnt(0); expcnt untouched
#define GEMM_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x70)

// LDS-direct load of 16 bytes per lane: lane l's bytes go to LDS address
// lds + 16 l (lds: a wave-uniform LDS byte address).  Written as inline assembly so that the
// compiler does not order every later LDS read after it (it cannot tell the
// ring's buffers apart and would wait for all loads in flight); completion is
// awaited explicitly with GEMM_WAIT_VM before the barrier of each step.
__device__ __forceinline__ void lds_load16(const void *src, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 : : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// The same with a wave-uniform 64-bit base (held in SGPRs) and a 32-bit
// per-lane byte offset: one VGPR per stream instead of a 64-bit address.
// (No non-temporal hint: the chunks of an expert read its rows through L2.)
__device__ __forceinline__ void lds_load16_base(const void *base, uint32_t voff, uint32_t lds)
{
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint64_t sb = (uint64_t)lo | ((uint64_t)hi << 32);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 : : "v"(voff), "s"(sb), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// LDS byte address of a shared-memory object
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

template <int PHASE>
__global__ __launch_bounds__(GT) void k_gemm_f16(GemmJob job)
{
    constexpr bool DOWN = PHASE == 1;
    constexpr int GN = DOWN ? GN_DN : GN_GU;         // output rows per item
    static_assert(GPA == 1 && GPW == 4 && GNW == 2 * GN_GU && GNW == GN_DN && GN_GU == 256 && GK == 32,
                  "tile shapes: a stage's weight tile is four 128-row blocks of the tiled layout");
    // stage s: activation tile at S[s][0 .. GTA), weight tile at S[s][GTA ..);
    // row r of a tile is 64 bytes at r * 64, its k-chunks swizzled by swz(r)
    __shared__ __align__(16) uint8_t S[GS][GSTAGE];
    const uint32_t s_base = __builtin_amdgcn_readfirstlane(lds_addr(&S[0][0]));

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + GM - 1) / GM : 0;
    const int rg = (DOWN ? H : FF) / GN, rg_sh = (DOWN ? H : SF) / GN;
    // Items by XCD: workgroup b runs on XCD b % 8 (round-robin dispatch).  The
    // units (expert chunks, expert-major, then the shared expert's token
    // chunks) are split into 8 contiguous segments of equal work (a shared
    // unit does two passes), one per XCD, so that the row groups of a unit
    // (one activation block) and the chunks of an expert (one weight slice)
    // meet in the same L2.  Within a segment the shared units' items come
    // first (twice as long: started first, the routed items fill in behind
    // them; dispatched last, they would finish a round after the rest), then
    // the routed ones; item m of either part is unit m / row-groups, row group
    // m % row-groups.
    static_assert(GEMM_BLOCKS % 8 == 0, "grid by XCD");
    const int xcd = blockIdx.x & 7, G8 = gridDim.x >> 3, lb = blockIdx.x >> 3;
    const long w_routed = (long)n_ec * rg, w_total = w_routed + 2L * nch * rg_sh;
    auto seg = [&](int x) -> int {
        const long t = w_total * x / 8;
        return t <= w_routed ? (int)((t + rg - 1) / rg)
                             : n_ec + (int)((t - w_routed + 2 * rg_sh - 1) / (2 * rg_sh));
    };
    const int u0 = seg(xcd), u1 = seg(xcd + 1);
    const int nr = max(0, min(u1, n_ec) - u0);                             // routed units
    const int s0 = max(u0, n_ec) - n_ec, ns = max(0, u1 - max(u0, n_ec)); // shared chunks
    const int seg_items = nr * rg + ns * rg_sh;
    // wave grid 1 (activation rows) x 8 (weight rows): 128 x 64 per wave
    const int tok0 = 0;
    const int wq = wave;
    // byte offsets of this lane's operand chunk g in a tile (swz depends on
    // row bits 1..2 only: the same for every 16-row tile): activation rows
    // 16 ti + r16 at aoff + 1024 ti; the wave's four 16-row weight tiles at
    // boff + bstep(tw): down: rows 64 wq + 16 tw; gate/up: 32 moe_ff rows of
    // gate (tiles 0, 1) and the same rows of up (tiles 2, 3)
    const int aoff = (tok0 + r16) * 64 + ((g ^ swz(r16)) << 4);
    const int boff = ((DOWN ? 64 : 32) * wq + r16) * 64 + ((g ^ swz(r16)) << 4);
    auto bstep = [](int tw) -> int { return DOWN ? 1024 * tw : (tw < 2 ? 1024 * tw : GN * 64 + 1024 * (tw - 2)); };

    for (int m = lb; m < seg_items; m += G8) {
        const bool shared = m < ns * rg_sh;
        const int mm = shared ? m : m - ns * rg_sh;
        const int rgn = shared ? rg_sh : rg;
        const int unit = (shared ? s0 : u0) + mm / rgn, rb = mm % rgn;
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * GM;
            t_first = job.offsets[e] + c0;
            nt = min(GM, job.counts[e] - c0);
        } else {
            t_first = unit * GM;
            nt = min(GM, N - t_first);
        }
        const int Kin = DOWN ? (shared ? SF : FF) : H;
        const int nsteps = Kin / GK;
        const int total_steps = (shared ? 2 : 1) * nsteps;
        // activations: rows of a [rows][Kin] f16 array (split: lo rows after the hi rows)
        const uint16_t *A = DOWN ? (shared ? job.hs16 : job.h16) : (shared ? job.xs16 : job.x16);
        const size_t lo_off = (size_t)N * Kin;           // split arrays only

        // weight rows of the item (tiled layout, 128-row blocks of 8 KB per k
        // step): gate rows 0..255 and up rows 256..511 of the same moe_ff rows
        // (blocks 2 rb, 2 rb + 1 of each), or 512 down rows (blocks 4 rb ..
        // 4 rb + 3).  (The fields are selected here, not in a lambda: a lambda
        // that captured the argument struct would copy it to private memory.)
        const WTensor &w0 = DOWN ? (shared ? job.sd : job.ed) : (shared ? job.sg : job.eg);
        const WTensor &w1 = DOWN ? (shared ? job.sd : job.ed) : (shared ? job.su : job.eu);
        const size_t kblk = (size_t)nsteps * 8192;       // one 128-row block
        const uint8_t *wb0 = w0.data + (size_t)e * w0.nb2 + (size_t)(DOWN ? 4 * rb : 2 * rb) * kblk;
        const uint8_t *wb1 = DOWN ? wb0 + 2 * kblk : w1.data + (size_t)e * w1.nb2 + (size_t)(2 * rb) * kblk;
        // piece c = i * GT + tid of a tile (16 bytes at c * 16): row c >> 2,
        // slot c & 3, holding k-chunk (c & 3) ^ swz(row).  A wavefront's pieces
        // of one load are 1 KB of consecutive LDS, as the LDS-direct load
        // writes, and of the tiled weights in HBM: weight piece i * GT + tid
        // is piece tid of 128-row block i of the item (block i & 1 of wb0 for
        // i < 2, of wb1 after), its k step ks at ks * 8192.
        const uint8_t *ap[GPA], *bp[GPW];
#pragma unroll
        for (int i = 0; i < GPA; i++) {
            const int c = i * GT + tid, row = c >> 2;
            const int q = (c & 3) ^ swz(row);
            int arow;
            if (shared) {
                arow = t_first + min(row, nt - 1);
            } else {
                const int p = job.perm[t_first + min(row, nt - 1)];
                arow = DOWN ? p : p / K;
            }
            ap[i] = reinterpret_cast<const uint8_t *>(A + (size_t)arow * Kin) + q * 16;
        }
#pragma unroll
        for (int i = 0; i < GPW; i++) {
            const uint64_t b = (uint64_t)(uintptr_t)((i < 2 ? wb0 : wb1) + (size_t)(i & 1) * kblk);
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
            bp[i] = reinterpret_cast<const uint8_t *>((uintptr_t)((uint64_t)lo | ((uint64_t)hi << 32)));
        }
        const uint32_t bv = (uint32_t)tid * 16;
        // stage st of the k loop into LDS buffer st % GS: GLOADS loads per
        // thread (none past the last stage, so nothing is in flight when the
        // item ends)
        auto issue = [&](int st) {
            if (st >= total_steps) return;
            const int pass = st >= nsteps ? 1 : 0;
            const int ks = st - pass * nsteps;
            const size_t ab = (size_t)ks * GK * 2 + (pass ? lo_off * 2 : 0);
            const size_t wbk = (size_t)ks * 8192;
            const uint32_t sb = s_base + (uint32_t)((st % GS) * GSTAGE + wave * 1024);
#pragma unroll
            for (int i = 0; i < GPA; i++) lds_load16(ap[i] + ab, sb + i * GT * 16);
#pragma unroll
            for (int i = 0; i < GPW; i++) lds_load16_base(bp[i], bv + (uint32_t)wbk, sb + GTA + i * GT * 16);
        };
        // Operand reads of a stage (buffer buf, at the LDS byte offset of the
        // buffer in S): the lane offsets go through an empty asm so that the
        // compiler keeps one register each and adds the buffer offset per
        // step, instead of holding a precomputed address per buffer.
        auto read_w = [&](uint32_t boffs, int t) -> h8 {
            return *reinterpret_cast<const h8 *>(&S[0][0] + boffs + bstep(t));
        };
        auto read_a = [&](uint32_t aoffs, int ti) -> h8 {
            return *reinterpret_cast<const h8 *>(&S[0][0] + aoffs + 1024 * ti);
        };

        f4 acc[8][4];
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int tw = 0; tw < 4; tw++) acc[ti][tw] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
        // operand register sets: set c holds a stage's 8 activation and 4
        // weight operands; step st computes from set st & 1 and reads stage
        // st + 1 into the other set between its MFMAs
        h8 ra[2][8], rw[2][4];
        // Step st: wait until stage st + 1 has landed (the GS - 2 stages after
        // it may be in flight; in the last steps fewer follow: wait for all)
        // and until this wavefront's reads of stage st (issued in step st - 1)
        // are done, barrier (all wavefronts' loads of stage st + 1 are in LDS,
        // and the buffer of stage st, whose operands are all in registers, is
        // free), refill that buffer with stage st + GS, then run the 32 MFMAs
        // of stage st from registers,
        // reading stage st + 1's operands (if next) in between: one or two
        // reads ahead of each group of four MFMAs.  The scheduling groups fix
        // that interleave; the reads complete during the step and are awaited
        // before the next step's first MFMA.
        // NTI (8, 4 or 0): the wavefront's 16-row activation blocks that hold
        // pairs of the item; the MFMAs and operand reads of the others are
        // skipped (an item of fewer than 128 pairs repeats its last row)
        auto step = [&](auto nti_c, int st, int c, bool tail, bool next) {
            constexpr int NTI = decltype(nti_c)::value;
            if (!tail)
                GEMM_WAIT_VM(GLOADS * (GS - 2));
            else
                GEMM_WAIT_VM(0);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (!tail) issue(st + GS);
            uint32_t al = aoff, bl = boff;
            asm volatile("" : "+v"(al), "+v"(bl));
            const uint32_t nb = (uint32_t)(((st + 1) % GS) * GSTAGE);
            const uint32_t aoffs = al + nb, boffs = bl + nb + GTA;
#pragma unroll
            for (int ti = 0; ti < NTI; ti++) {
                if (next) {
                    if (ti < 4) rw[c ^ 1][ti] = read_w(boffs, ti);
                    ra[c ^ 1][ti] = read_a(aoffs, ti);
                }
#pragma unroll
                for (int tw = 0; tw < 4; tw++)
                    acc[ti][tw] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ra[c][ti], rw[c][tw], acc[ti][tw], 0, 0, 0);
                if (next) {
                    if (ti < 4)
                        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    else
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        };

        // the previous item's LDS reads are done in every wavefront
        GEMM_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int st = 0; st < GS; st++) issue(st);
        // stage 0 in LDS, its operands in set 0
        if (GS - 1 < total_steps)
            GEMM_WAIT_VM(GLOADS * (GS - 1));
        else
            GEMM_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int t = 0; t < 4; t++) rw[0][t] = read_w(boff + GTA, t);
#pragma unroll
        for (int ti = 0; ti < 8; ti++) ra[0][ti] = read_a(aoff, ti);
        // total_steps is even (Kin % 64 == 0): two steps per iteration, one
        // operand set each.  Steps st with st + GS - 1 < total_steps refill
        // the ring (when a stage is left) and wait for a fixed count; the last
        // ones wait for all loads.
        auto run = [&](auto nti_c) {
            int st = 0;
            for (; st + 1 + GS - 1 < total_steps; st += 2) {
                step(nti_c, st, 0, false, true);
                step(nti_c, st + 1, 1, false, true);
            }
            for (; st < total_steps; st += 2) {
                // every stage is issued by now
                step(nti_c, st, 0, st + GS - 1 >= total_steps, true);
                step(nti_c, st + 1, 1, true, st + 2 < total_steps);
            }
        };
        // (down only: skipping them in the gate/up launch measured slower)
        const int wrows = nt - tok0;                     // the wavefront's activation rows with pairs
        if (!DOWN || wrows > 64)
            run(std::integral_constant<int, 8>());
        else if (wrows > 0)
            run(std::integral_constant<int, 4>());
        else
            run(std::integral_constant<int, 0>());

        // results: output row of tile tw for lane r16; activation rows 16 ti + 4 g + i
        // (the row base goes through an empty asm so that the compiler does not
        // hold the 32 row indices in registers across the item loop)
        int ebase = tok0 + 4 * g, erow = r16;
        asm volatile("" : "+v"(ebase), "+v"(erow));
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tt = ebase + 16 * ti + i;
                if (tt >= nt) continue;
                if (!DOWN) {
#pragma unroll
                    for (int tj = 0; tj < 2; tj++) {
                        const int row = rb * GN + 32 * wq + 16 * tj + erow;
                        const float hv = gsilu(acc[ti][tj][i]) * acc[ti][2 + tj][i];
                        if (!shared) {
                            const int p = job.perm[t_first + tt];
                            job.h16[(size_t)p * FF + row] = f2h_rn(hv);
                        } else {
                            const int t = t_first + tt;
                            const uint16_t hi = f2h_rn(hv);
                            job.hs16[(size_t)t * SF + row] = hi;
                            job.hs16[(size_t)N * SF + (size_t)t * SF + row] =
                                f2h_rn(hv - (float)__builtin_bit_cast(_Float16, hi));
                        }
                    }
                } else {
                    float *o = shared ? job.ys + (size_t)(t_first + tt) * H
                                      : job.ye + (size_t)job.perm[t_first + tt] * H;
#pragma unroll
                    for (int tw = 0; tw < 4; tw++) o[rb * GN + 64 * wq + 16 * tw + erow] = acc[ti][tw][i];
                }
            }
    }
}

// F16 matrices [rows][K] (ggml row layout, mats of them) -> the tiled layout
// the GEMM streams: per matrix, 128-row blocks, k-step-major inside a block
// (the 128 rows x 32 values of k step ks of block b are the 8 KB at
// (b * K/32 + ks) * 8192), row r of the 8 KB at r * 64 with its 16-byte chunk
// q at slot q ^ swz(r) -- the LDS layout of a stage, so the GEMM copies a
// block's k step to LDS as it lies.  One thread per 16-byte chunk.
__global__ __launch_bounds__(256) void k_tile_f16(const uint8_t *__restrict__ src, size_t nb1, size_t nb2,
                                                  int rows, int K, int mats, uint8_t *__restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int cpr = K / 8;                            // 16-byte chunks of a row
    const size_t per_mat = (size_t)rows * cpr;
    if (i >= per_mat * mats) return;
    const int m = (int)(i / per_mat);
    const size_t j = i - (size_t)m * per_mat;
    const int r = (int)(j / cpr), c = (int)(j % cpr);
    const int ks = c >> 2, q = c & 3, rl = r & 127;
    const uint4 v = *reinterpret_cast<const uint4 *>(src + (size_t)m * nb2 + (size_t)r * nb1 + (size_t)c * 16);
    uint8_t *out = dst + (size_t)m * rows * K * 2 + ((size_t)(r >> 7) * (K / GK) + ks) * 8192 +
                   rl * 64 + ((q ^ swz(rl)) << 4);
    *reinterpret_cast<uint4 *>(out) = v;
}

hipError_t launch_tile_f16(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s)
{
    if (rows % 128 || K % GK || nb1 % 16 || (mats > 1 && nb2 % 16)) return hipErrorInvalidValue;
    const size_t total = (size_t)rows * (K / 8) * mats;
    hipLaunchKernelGGL(k_tile_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, nb1, nb2,
                       rows, K, mats, dst);
    return hipGetLastError();
}

// x (f32 rows) -> f16 rows, or the hi / lo f16 pair (lo rows after the hi rows)
__global__ __launch_bounds__(256) void k_cvt_f16(const float *__restrict__ src, size_t n, int split,
                                                 uint16_t *__restrict__ dst)
{
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 v = *reinterpret_cast<const float4 *>(src + i);
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        hi[k] = f2h_rn(x[k]);
        lo[k] = f2h_rn(x[k] - (float)__builtin_bit_cast(_Float16, hi[k]));
    }
    uint2 ph, pl;
    ph.x = (uint32_t)hi[0] | ((uint32_t)hi[1] << 16);
    ph.y = (uint32_t)hi[2] | ((uint32_t)hi[3] << 16);
    *reinterpret_cast<uint2 *>(dst + i) = ph;
    if (split) {
        pl.x = (uint32_t)lo[0] | ((uint32_t)lo[1] << 16);
        pl.y = (uint32_t)lo[2] | ((uint32_t)lo[3] << 16);
        *reinterpret_cast<uint2 *>(dst + n + i) = pl;
    }
}

hipError_t launch_cvt_f16(const float *src, int rows, int K, int split, uint16_t *dst, hipStream_t s)
{
    const size_t n = (size_t)rows * K;
    if (K % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cvt_f16, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, src, n, split, dst);
    return hipGetLastError();
}

bool gemm_shapes_ok(int H, int FF, int SF, bool shared)
{
    // whole row groups; an even number of k steps per pass
    return H % GN_DN == 0 && H % (2 * GK) == 0 && FF % GN_GU == 0 && FF % (2 * GK) == 0 &&
           (!shared || (SF % GN_GU == 0 && SF % (2 * GK) == 0));
}

hipError_t launch_gemm_f16(int phase, const GemmJob &job, hipStream_t s)
{
    if (!gemm_shapes_ok(job.H, job.FF, job.SF, job.has_shared)) return hipErrorInvalidValue;
    if (phase == 0)
        hipLaunchKernelGGL(k_gemm_f16<0>, dim3(GEMM_BLOCKS), dim3(GT), 0, s, job);
    else
        hipLaunchKernelGGL(k_gemm_f16<1>, dim3(GEMM_BLOCKS), dim3(GT), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
