// k_expert.hip — grouped Q4_K expert products on int8 MFMA (gfx950).
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 (ggml's
// mul_mat_id over Q4_K weights with Q8_K activations) and the shared expert of
// :280-286 (F32 activations, here two int8 digits), as one persistent launch
// per phase:
//   phase 0: h = silu(W_gate x) * (W_up x)       (gate and up of the same rows)
//   phase 1: y = W_down h
// (the conversion of h to the int8 layout runs in between, k_prep.hip).
//
// Arithmetic.  A Q4_K row is, per 256-value super-block, w = d*sc_j*q - dmin*m_j
// (j = 32-value sub-block, q in 0..15, sc_j, m_j 6-bit).  With int8
// activations a and their scale d_x this is ggml's vec_dot_q4_K_q8_K:
//   sum_k w a = d * sum_j sc_j S_j - dmin * sum_j m_j B_j,
//   S_j = sum_{k in j} q_k a_k (int32),  B_j = sum_{k in j} a_k.
// S_j comes from one v_mfma_i32_16x16x32_i8 per sub-block (the nibbles are the
// int8 operand), sum_j sc_j S_j from integer multiply-adds (exact), the min
// term from v_mfma_f32_16x16x16_f16 on the sums of 16 (exact integers in f16).
// The super-block result is scaled by d_x and accumulated in f32.
//
// Operand layout (checked on the hardware): srcA lane l = activation row l%16,
// k = 8*(l/16) + byte; srcB lane l = weight row l%16, same k; D lane l = weight
// row l%16, activation rows 4*(l/16)+i.  The tiled weight layout (k_quant.hip)
// puts the 32 quant bytes lane group g needs (bytes 32c + 8g .. +8 of each
// 32-byte chunk c: low nibbles = sub-block 2c, high = 2c+1) side by side, and
// repacks the 6-bit scales so that each is one bit-field extract.
//
// Memory.  A workgroup's eight wavefronts share one work item (16 activation
// rows).  Per step (one super-block) each wavefront copies its own weight
// tiles (contiguous 2304-byte runs) into a private ring of LDS stages, and six
// of them copy the step's activations into the workgroup's activation ring,
// with LDS-direct loads (global_load_lds_dwordx4): two steps stay in flight
// without holding registers.
#include "dmoe_prep.h"

namespace dmoe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Tuning constants (overridable at compile time).
#ifndef DMOE_X_WSTAGES
#define DMOE_X_WSTAGES 3         // LDS stages of each wavefront's weight ring
#endif
#ifndef DMOE_X_DN_IT
#define DMOE_X_DN_IT 2           // row passes of a down item (shared activation tile)
#endif
#ifndef DMOE_X_BLOCKS
#define DMOE_X_BLOCKS 1024       // persistent grid
#endif
#ifndef DMOE_X_WAVES
#define DMOE_X_WAVES 8           // wavefronts per workgroup (one workgroup per CU)
#endif
constexpr int WAVES = DMOE_X_WAVES;
constexpr int RT = 2;                        // 16-row weight tiles per wave per step
constexpr int WSTAGES = DMOE_X_WSTAGES;
constexpr int DN_IT = DMOE_X_DN_IT;
static_assert(DN_IT >= 1 && DN_IT <= 4, "row passes of a down item");
constexpr int GU_IT = 2;                         // row passes of a gate/up item
constexpr int GROWS_GU = WAVES * 16 * GU_IT;     // gate/up rows of an item: one h super-block
constexpr int GROWS_DN = WAVES * 16 * RT * DN_IT;   // down rows of an item
constexpr int TILE_BYTES = 16 * Q4K_BYTES;   // one tile x one super-block
constexpr int WSTEP_BYTES = RT * TILE_BYTES;             // one wave's weights of one step
constexpr int TPIECES = TILE_BYTES / 16;                 // 16-byte pieces of a tile (144)
constexpr int WLOADS = RT * 3;                           // LDS-direct loads per step: 64 + 64 + 16 pieces a tile
static_assert(TILE_BYTES % 16 == 0 && TPIECES > 128 && TPIECES <= 192, "tile pieces");

__device__ __forceinline__ float h16f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }

struct Q4KTile {        // a lane's share of one 16-row tile in one super-block
    uint4 h;            // d, dmin, repacked scales
    uint4 q0, q1;       // the 32 quant bytes of lane group g
};

// A weight tile of one super-block (a 2304-byte run of the tiled layout,
// copied to a ring stage as it lies): piece k of row r16's repacked block at
// slot 16 k + r16 (k = 0: d, dmin, scales; k = 1 + 2g, 2 + 2g: the quant bytes
// of lane group g), so that every read below is free of LDS bank conflicts.
__device__ __forceinline__ void read_tile(Q4KTile &t, const uint8_t *tile, int r16, int g)
{
    const uint4 *p = reinterpret_cast<const uint4 *>(tile);
    t.h = p[r16];
    t.q0 = p[(1 + 2 * g) * 16 + r16];
    t.q1 = p[(2 + 2 * g) * 16 + r16];
}

// LDS-direct load of 16 bytes per active lane: lane l's bytes go to LDS address
// lds + 16 l (lds wave-uniform).  Inline assembly, so that the compiler does not
// order every later LDS read after it (it cannot tell the ring's stages apart
// and would wait for all loads in flight); completion is awaited with an
// explicit s_waitcnt on the vector-memory counter.
__device__ __forceinline__ void lds_load16(const void *src, const void *lds)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(m0) : "memory", "m0");
}

// The same with the source as a wave-uniform base (an SGPR pair) plus a
// 32-bit per-lane byte offset (global_load's saddr form): the base advances by
// scalar adds, the offsets stay fixed, so issuing a step costs no VALU.
__device__ __forceinline__ void lds_load16_sa(const void *base, uint32_t voff, const void *lds)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
    // the base is wave-uniform by construction; readfirstlane makes that
    // visible to the compiler, so the operand is always an SGPR pair (the
    // builtin returns a signed int: each half is widened as uint32_t, never
    // sign-extended)
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint64_t sb = (uint64_t)lo | ((uint64_t)hi << 32);
    // nt: the weights are streamed once per forward (non-temporal hint; the
    // streaming read rate measured 6.8 TB/s with it against 6.05 without)
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" : : "v"(voff), "s"(sb), "s"(m0) : "memory", "m0");
}

// s_waitcnt with vmcnt(n), lgkmcnt(0), expcnt untouched (n < 16)
#define EXPERT_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x70 | (n))

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w)
{
    return __builtin_amdgcn_ubfe(v, off, w);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Activations of one step (one super-block of the item's 16 rows) in a stage
// of the workgroup's activation ring:
//   q  [16][256] int8 at 0: 16-byte unit u of row r at unit u ^ (r & 11), which
//      makes the operand reads (lane l: row l % 16, units 4 (l / 16) .. + 3)
//      free of LDS bank conflicts
//   bs [16][16] f16 at ABS_OFF (sums of 16)
//   d  [16] f32 at AD_OFF
constexpr int ABS_OFF = 4096, AD_OFF = 4608, ASTEP_BYTES = 4672;
constexpr int ADMA_WAVES = 6;       // wavefronts that load a step's activations

// LDS-direct load of 4 bytes per active lane (to lds + 4 l).
__device__ __forceinline__ void lds_load4(const void *src, const void *lds)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(src), "s"(m0) : "memory", "m0");
}

// One super-block of RT weight tiles against the step's activations.
__device__ __forceinline__ void compute_sb(const Q4KTile (&cur)[RT], const uint8_t *ast, int r16, int g,
                                           float (&acc)[RT][4])
{
    // activation operands of the 8 sub-blocks: row r16, bytes 64g .. 64g+63
    // (16-byte units 4g .. 4g+3, swizzled)
    const uint4 *ap = reinterpret_cast<const uint4 *>(ast + r16 * 256);
    const uint4 a01 = ap[(4 * g + 0) ^ (r16 & 11)], a23 = ap[(4 * g + 1) ^ (r16 & 11)];
    const uint4 a45 = ap[(4 * g + 2) ^ (r16 & 11)], a67 = ap[(4 * g + 3) ^ (r16 & 11)];
    const long a[8] = {
        (long)((uint64_t)a01.y << 32 | a01.x), (long)((uint64_t)a01.w << 32 | a01.z),
        (long)((uint64_t)a23.y << 32 | a23.x), (long)((uint64_t)a23.w << 32 | a23.z),
        (long)((uint64_t)a45.y << 32 | a45.x), (long)((uint64_t)a45.w << 32 | a45.z),
        (long)((uint64_t)a67.y << 32 | a67.x), (long)((uint64_t)a67.w << 32 | a67.z)};
    const h4 ab = __builtin_bit_cast(h4, *reinterpret_cast<const uint2 *>(ast + ABS_OFF + r16 * 32 + 8 * g));
    const float4 dxv = *reinterpret_cast<const float4 *>(ast + AD_OFF + 16 * g);
    const float dx[4] = {dxv.x, dxv.y, dxv.z, dxv.w};
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const Q4KTile &t = cur[r];
        // six-bit scales (repacked: sc0..sc4 | sc5..sc7 m0 m1 | m2..m6, m7 in bits 30..31)
        const uint32_t sc[8] = {bfe(t.h.y, 0, 6),  bfe(t.h.y, 6, 6),  bfe(t.h.y, 12, 6),
                                bfe(t.h.y, 18, 6), bfe(t.h.y, 24, 6), bfe(t.h.z, 0, 6),
                                bfe(t.h.z, 6, 6),  bfe(t.h.z, 12, 6)};
        const uint32_t msrc = g == 0 ? t.h.z : t.h.w;
        const uint32_t moff = g == 0 ? 18u : 12u * (uint32_t)g - 12u;
        const uint32_t m7 = (t.h.y >> 30) | ((t.h.z >> 30) << 2) | ((t.h.w >> 30) << 4);
        const uint32_t ma = bfe(msrc, moff, 6);
        const uint32_t mb = g == 3 ? m7 : bfe(msrc, moff + 6, 6);
        const _Float16 fa = (_Float16)(float)ma, fb = (_Float16)(float)mb;
        const h4 bm = {fa, fa, fb, fb};
        // nibbles -> int8 operands: dwords 2c, 2c+1 hold chunk c of lane group g
        const uint32_t w[8] = {t.q0.x, t.q0.y, t.q0.z, t.q0.w, t.q1.x, t.q1.y, t.q1.z, t.q1.w};
        // all eight sub-block products of the tile first, then their scales
        // (the MFMA results are read only after the last one is issued)
        v4i sj[8];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t l0 = w[2 * c] & 0x0F0F0F0Fu, l1 = w[2 * c + 1] & 0x0F0F0F0Fu;
            const uint32_t h0 = (w[2 * c] >> 4) & 0x0F0F0F0Fu, h1 = (w[2 * c + 1] >> 4) & 0x0F0F0F0Fu;
            const long blo = (long)((uint64_t)l1 << 32 | l0), bhi = (long)((uint64_t)h1 << 32 | h0);
            const v4i z = {0, 0, 0, 0};
            sj[2 * c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[2 * c], blo, z, 0, 0, 0);
            sj[2 * c + 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[2 * c + 1], bhi, z, 0, 0, 0);
        }
        // |S_j| <= 32 * 15 * 127 and sc_j < 64: 24-bit products are exact
        // (v_mad_i32_i24, full rate; a 32-bit multiply is quarter rate). The
        // empty asm pins each step as one multiply-add: left free, the
        // compiler splits the chain into v_mul_i32_i24 + v_add3 pairs.
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                isum[i] = __mul24((int)sc[j], sj[j][i]) + isum[i];
                asm volatile("" : "+v"(isum[i]));
            }
        f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
        s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, bm, s2, 0, 0, 0);
        const float d = h16f(t.h.x & 0xffffu), dmin = h16f(t.h.x >> 16);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r][i] += dx[i] * (d * (float)isum[i] - dmin * s2[i]);
    }
}

// The same products for NC column blocks that share the step's weight tiles,
// with the sub-block scales folded into the weight operand: sc_j = 8 sh_j +
// sl_j (sh_j, sl_j < 8), so sh_j q and sl_j q (q < 16) are int8 values below
// 106 and
//   sum_j sc_j S_j = 8 sum_k (sh q)_k a_k + sum_k (sl q)_k a_k,
// two int32 sums over the whole super-block, each from four
// v_mfma_i32_16x16x64_i8 (sub-blocks 2c and 2c+1 side by side in one 16-byte
// operand: the activation bytes 64g + 16c .. +15 as they lie in LDS, and the
// weight dwords of chunk c).  The integers equal the per-sub-block sums of
// compute_sb exactly, so the results are bit-identical; the tile's operands
// are formed once for all NC blocks instead of 32 scale multiply-adds per
// tile and block.
struct Q4KFolded {
    v4i bh[4], bl[4];   // (sh q), (sl q) operands of chunks 0..3
    h4 bm;              // min-term operand
    float d, dmin;
};

__device__ __forceinline__ void fold_tile(const Q4KTile &t, int g, Q4KFolded &f)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    // scale j: 6 bits at 6j of dword y (j < 5), at 6 (j - 5) of dword z
    uint32_t sh[8], sl[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t src = j < 5 ? t.h.y : t.h.z;
        const uint32_t off = j < 5 ? 6u * j : 6u * (j - 5);
        sl[j] = bfe(src, off, 3);
        sh[j] = bfe(src, off + 3, 3);
    }
    const uint32_t w[8] = {t.q0.x, t.q0.y, t.q0.z, t.q0.w, t.q1.x, t.q1.y, t.q1.z, t.q1.w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t l0 = w[2 * c] & 0x0F0F0F0Fu, l1 = w[2 * c + 1] & 0x0F0F0F0Fu;
        const uint32_t h0 = (w[2 * c] >> 4) & 0x0F0F0F0Fu, h1 = (w[2 * c + 1] >> 4) & 0x0F0F0F0Fu;
        // byte-wise products by a scale below 8: each byte stays below 128, so
        // a 16-bit lane product carries nothing across its two bytes
        auto mul = [](uint32_t v, uint32_t s) -> int {
            const u16x2 a = __builtin_bit_cast(u16x2, v);
            const u16x2 b = {(unsigned short)s, (unsigned short)s};
            return __builtin_bit_cast(int, (u16x2)(a * b));
        };
        f.bh[c] = (v4i){mul(l0, sh[2 * c]), mul(l1, sh[2 * c]), mul(h0, sh[2 * c + 1]), mul(h1, sh[2 * c + 1])};
        f.bl[c] = (v4i){mul(l0, sl[2 * c]), mul(l1, sl[2 * c]), mul(h0, sl[2 * c + 1]), mul(h1, sl[2 * c + 1])};
    }
    const uint32_t msrc = g == 0 ? t.h.z : t.h.w;
    const uint32_t moff = g == 0 ? 18u : 12u * (uint32_t)g - 12u;
    const uint32_t m7 = (t.h.y >> 30) | ((t.h.z >> 30) << 2) | ((t.h.w >> 30) << 4);
    const uint32_t ma = bfe(msrc, moff, 6);
    const uint32_t mb = g == 3 ? m7 : bfe(msrc, moff + 6, 6);
    const _Float16 fa = (_Float16)(float)ma, fb = (_Float16)(float)mb;
    f.bm = (h4){fa, fa, fb, fb};
    f.d = h16f(t.h.x & 0xffffu);
    f.dmin = h16f(t.h.x >> 16);
}

// One folded tile against one column block's activations of the step.
__device__ __forceinline__ void compute_folded(const Q4KFolded &f, const uint8_t *ast, int r16, int g, float (&acc)[4])
{
    const uint4 *ap = reinterpret_cast<const uint4 *>(ast + r16 * 256);
    v4i a[4];
#pragma unroll
    for (int c = 0; c < 4; c++) a[c] = __builtin_bit_cast(v4i, ap[(4 * g + c) ^ (r16 & 11)]);
    const h4 ab = __builtin_bit_cast(h4, *reinterpret_cast<const uint2 *>(ast + ABS_OFF + r16 * 32 + 8 * g));
    const float4 dxv = *reinterpret_cast<const float4 *>(ast + AD_OFF + 16 * g);
    const float dx[4] = {dxv.x, dxv.y, dxv.z, dxv.w};
    v4i sh = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[c], f.bh[c], sh, 0, 0, 0);
        sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[c], f.bl[c], sl, 0, 0, 0);
    }
    f4 s2 = {0.0f, 0.0f, 0.0f, 0.0f};
    s2 = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, f.bm, s2, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int isum = 8 * sh[i] + sl[i];
        acc[i] += dx[i] * (f.d * (float)isum - f.dmin * s2[i]);
    }
}

// Work items of phase 0: routed (work-list entry ec, group of GROWS_GU rows),
// then shared (chunk of 8 NC tokens, group of GROWS_GU rows); phase 1 the
// same with groups of GROWS_DN rows.  A routed item's activation rows are the
// pairs of its entry (one expert, up to 16 NC consecutive pairs of it, in NC
// column blocks of 16); a shared item's are the a1 / a0 digit rows of its
// tokens interleaved (t a1, t a0, ...; 8 tokens per column block), so that
// each lane's four outputs are (t, a1), (t, a0), (t+1, a1), (t+1, a0) and the
// two digits' products are summed in-lane.  NC > 1 (many tokens per expert)
// multiplies every weight tile read from HBM by NC activation blocks: the
// weights stream once per 16 NC pairs instead of once per 16.
//
// Step s of an item is super-block s % nsb of row pass s / nsb.  Its weights
// (each wavefront's own tiles) and its activations (the workgroup's 16 NC
// rows, loaded by wavefronts 0..5) go to ring stage s % WST with LDS-direct
// loads issued WST - 1 steps ahead; one barrier per step makes the
// activations visible to all wavefronts and frees the stage for refilling.
template <int PHASE, int NC>
__global__ __launch_bounds__(WAVES * 64, 2) void k_expert_q4k(MoeJob job)
{
    constexpr bool DOWN = PHASE == 1;
    // row passes per item (a down item of 4 column blocks takes one, which
    // keeps its accumulators and two items' pointers in registers)
    constexpr int IT = DOWN ? (NC >= 4 ? 1 : DN_IT) : GU_IT;
    constexpr int GROWS = DOWN ? WAVES * 16 * RT * IT : GROWS_GU;
    // ring depths: one column block runs both rings WSTAGES deep, loads of
    // a step issued together WSTAGES - 1 steps ahead; NC > 1 blocks keep the
    // weight ring three deep (two steps of HBM loads in flight) and the
    // activation ring two deep (its loads come from L2, one step ahead), which
    // is what the LDS holds next to NC activation blocks per stage
    constexpr int WST = NC == 1 ? WSTAGES : 3;           // weight ring
    constexpr int AST = NC == 1 ? WSTAGES : 2;           // activation ring
    constexpr int CH = EXPERT_CHUNK * NC;            // pairs of a routed item
    constexpr int SCH = SHARED_CHUNK * NC;           // tokens of a shared item
    __shared__ __align__(16) uint8_t s_act[AST][NC * ASTEP_BYTES];
    __shared__ __align__(16) uint8_t s_w[WAVES][WST][WSTEP_BYTES];
    static_assert(NC * 16 * 256 * 4 <= WAVES * WST * WSTEP_BYTES, "h of a gate/up item fits the weight ring");
    static_assert(WAVES * 256 * 4 <= AST * NC * ASTEP_BYTES, "conversion scratch fits the activation ring");
    static_assert(NC == 1 || (WST == 3 && AST == 2), "the NC > 1 issue order below assumes these depths");

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + SCH - 1) / SCH : 0;
    const int rg = (DOWN ? H : FF) / GROWS, rg_sh = (DOWN ? H : SF) / GROWS;
    const int routed_items = n_ec * rg;
    const int total = routed_items + nch * rg_sh;
    const int Kin = DOWN ? FF : H;                   // reduction length (SF == FF when shared)
    const int nsb = Kin / 256;
    const int steps = IT * nsb;
    // weight loads of a step: tile r's pieces 64 j + lane (j = 0, 1, and 2 for
    // lanes below TPIECES - 128) from the tile's step run, to slot 64 j + lane
    // of the tile's place in the stage
    const uint32_t loff = lane * 16;
    // activation load of this wavefront (wavefronts 0..5): which block row
    // (ar) and piece; 0..3: q units of rows 4w .. 4w+3, 4: bs halves, 5: d
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);       // q: logical unit of this lane's slot
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);

    // The pointers of one work item.
    struct ItemPtrs {
        const uint8_t *tb[IT][RT];   // this wave's weight tiles of pass it
        const int8_t *aq[NC];        // the lane's activation load sources, per block
        const uint16_t *abs_[NC];
        const float *ad[NC];
        int t_first, nt, rbase, nblk;
        bool shared;
    };
    auto setup = [&](int item, ItemPtrs &P) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn;                 // work-list entry or shared chunk
        const int rbase = (j - unit * rgn) * GROWS;
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * CH;
            t_first = job.offsets[e] + c0;
            nt = min(CH, job.counts[e] - c0);
        } else {
            t_first = unit * SCH;
            nt = min(SCH, N - t_first);
        }
        if (!DOWN) {
            const WTensor &a = shared ? job.sg : job.eg;
            const WTensor &b = shared ? job.su : job.eu;
#pragma unroll
            for (int it = 0; it < IT; it++) {
                const int t16 = (rbase + it * (WAVES * 16) + wave * 16) / 16;
                P.tb[it][0] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
                P.tb[it][1] = b.data + (size_t)e * b.nb2 + (size_t)t16 * nsb * TILE_BYTES;
            }
        } else {
            const WTensor &a = shared ? job.sd : job.ed;
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const int t16 = (rbase + it * (WAVES * 32) + wave * 32) / 16 + r;
                    P.tb[it][r] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
                }
        }
        // the activation row of block row ar of each block: tokens in phase
        // 0, pairs in phase 1; shared rows interleave the a1 and a0 digit
        // rows (a0 rows start at N).  Rows past the item's last repeat it (a
        // block past it loads the last row again and is not computed).
        const ActI8 &act = DOWN ? (shared ? job.ahs : job.ah) : (shared ? job.axs : job.ax);
        const int per = shared ? SHARED_CHUNK : EXPERT_CHUNK;   // items of a block
#pragma unroll
        for (int c = 0; c < NC; c++) {
            int arow;
            if (shared) {
                arow = t_first + min(per * c + (ar >> 1), nt - 1) + (ar & 1) * N;
            } else {
                const int p = job.perm[t_first + min(per * c + ar, nt - 1)];
                arow = DOWN ? p : p / K;
            }
            P.aq[c] = act.q + (size_t)arow * Kin + aunit * 16;
            P.abs_[c] = act.bs + (size_t)arow * (Kin / 16) + (lane & 1) * 8;
            P.ad[c] = act.d + (size_t)arow * nsb;
        }
        P.t_first = t_first;
        P.nt = nt;
        P.rbase = rbase;
        P.nblk = (nt + per - 1) / per;
        P.shared = shared;
    };

    // row pass of step s (at most four passes: no division)
    auto pass_of = [&](int s) -> int {
        int it = 0;
#pragma unroll
        for (int q = 1; q < IT; q++) it += s >= q * nsb ? 1 : 0;
        return it;
    };
    // weights of step s of item P to weight stage gstep % WST
    auto issue_w = [&](const ItemPtrs &P, int s, int gstep) {
        if (s >= steps) return;
        const int it = pass_of(s), sb = s - it * nsb;
        const int stg = gstep % WST;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint8_t *t = P.tb[0][r];
#pragma unroll
            for (int q = 1; q < IT; q++)
                if (it == q) t = P.tb[q][r];
            t += (size_t)sb * TILE_BYTES;
            const uint8_t *d = &s_w[wave][stg][r * TILE_BYTES];
            lds_load16_sa(t, loff, d);
            lds_load16_sa(t, loff + 1024, d + 1024);
            if (lane < TPIECES - 128) lds_load16_sa(t, loff + 2048, d + 2048);
        }
    };
    // activations of step s of item P to activation stage gstep % AST
    auto issue_a = [&](const ItemPtrs &P, int s, int gstep) {
        if (s >= steps) return;
        const int it = pass_of(s), sb = s - it * nsb;
        const int stg = gstep % AST;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            uint8_t *st = &s_act[stg][c * ASTEP_BYTES];
            if (wave < 4)
                lds_load16(P.aq[c] + sb * 256, st + 1024 * wave);
            else if (wave == 4 && aload)
                lds_load16(P.abs_[c] + sb * 16, st + ABS_OFF);
            else if (wave == 5 && aload)
                lds_load4(P.ad[c] + sb, st + AD_OFF);
        }
    };
    // both parts of step s (the one-block order: weights, then activations)
    auto issue = [&](const ItemPtrs &P, int s, int gstep) {
        issue_w(P, s, gstep);
        issue_a(P, s, gstep);
    };

    // Down items end with global stores only, so the rings run on from one
    // item of this workgroup to its next: the last steps of an item issue
    // the next item's first WST - 1 steps (ring positions continue), and
    // the next item starts without draining.  Gate/up items convert h through
    // the rings after their last step, so each starts from drained rings.
    constexpr bool XPF = DOWN;
    ItemPtrs cur, nx;
    bool primed = false;             // cur's first WST - 1 steps are issued
    int g0 = 0;                      // ring position of cur's step 0
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        if (primed)
            cur = nx;
        else
            setup(item, cur);
        const int nitem = item + gridDim.x;
        const bool has_next = XPF && steps >= 2 && nitem < total;
        if (has_next) setup(nitem, nx);
        const bool shared = cur.shared;
        const int t_first = cur.t_first, nt = cur.nt, rbase = cur.rbase, nblk = cur.nblk;

        if (!primed) {
            // the previous item's reads of the rings are done in every wavefront
            g0 = 0;
            EXPERT_WAIT_VM(0);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if constexpr (NC == 1) {
#pragma unroll
                for (int s = 0; s < WST - 1; s++) issue(cur, s, s);
            } else {
                // W(0), A(0), W(1): step 0 waits with only W(1) in flight
                issue_w(cur, 0, 0);
                issue_a(cur, 0, 0);
                issue_w(cur, 1, 1);
            }
        }

        float acc[IT][NC][RT][4];
#pragma unroll
        for (int it = 0; it < IT; it++)
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int r = 0; r < RT; r++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[it][c][r][i] = 0.0f;
        for (int s = 0; s < steps; s++) {
            // step s's loads have landed once the WST - 2 later steps' are
            // all that may be in flight (a wavefront issues WLOADS loads per step,
            // plus NC when it loads activations; the previous item's output
            // stores, when they follow, only make this stricter); when fewer
            // later steps were issued (the item's last steps, no next item
            // primed): wait for all.  The barrier makes that true of every
            // wavefront and frees the stage read in the step before.
            if constexpr (NC == 1) {
                if (s + WST - 2 < steps || has_next) {
                    if (wave < ADMA_WAVES)
                        EXPERT_WAIT_VM((WLOADS + 1) * (WST - 2));
                    else
                        EXPERT_WAIT_VM(WLOADS * (WST - 2));
                } else {
                    EXPERT_WAIT_VM(0);
                }
            } else {
                // issue order per step: A(s + 1), then W(s + 2); so when
                // step s runs only W(s + 1) may still be in flight (every
                // earlier load, A(s) included, was issued before it)
                if (s + 1 < steps || has_next)
                    EXPERT_WAIT_VM(WLOADS);
                else
                    EXPERT_WAIT_VM(0);
            }
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if constexpr (NC == 1) {
                const int sn = s + WST - 1;
                if (sn < steps)
                    issue(cur, sn, g0 + sn);
                else if (has_next)
                    issue(nx, sn - steps, g0 + sn);
            } else {
                const int sa = s + 1, sw = s + 2;
                if (sa < steps)
                    issue_a(cur, sa, g0 + sa);
                else if (has_next)
                    issue_a(nx, sa - steps, g0 + sa);
                if (sw < steps)
                    issue_w(cur, sw, g0 + sw);
                else if (has_next)
                    issue_w(nx, sw - steps, g0 + sw);
            }
            const int it = pass_of(s);
            const int stg = (g0 + s) % WST, astg = (g0 + s) % AST;
            if constexpr (NC == 1) {
                Q4KTile cur_t[RT];
#pragma unroll
                for (int r = 0; r < RT; r++) read_tile(cur_t[r], &s_w[wave][stg][r * TILE_BYTES], r16, g);
#pragma unroll
                for (int q = 0; q < IT; q++)
                    if (it == q) compute_sb(cur_t, s_act[astg], r16, g, acc[q][0]);
            } else {
                // each tile's operands formed once, then every column block
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    Q4KTile t;
                    read_tile(t, &s_w[wave][stg][r * TILE_BYTES], r16, g);
                    Q4KFolded f;
                    fold_tile(t, g, f);
#pragma unroll
                    for (int c = 0; c < NC; c++)
                        if (c < nblk)
#pragma unroll
                            for (int q = 0; q < IT; q++)
                                if (it == q) compute_folded(f, &s_act[astg][c * ASTEP_BYTES], r16, g, acc[q][c][r]);
                }
            }
        }
        primed = has_next;
        g0 += steps;

        if (!DOWN) {
            // h = silu(gate) * up for the item's activation rows and its 256
            // moe_ff rows (one super-block), then converted in place to the
            // down products' operand layout (routed: Q8_K, shared: two int8
            // digits; dmoe_prep.h) -- no f32 h in HBM.  The rings are idle
            // (no loads in flight after the last step): h goes through the
            // weight-ring LDS, the conversion scratch through the activation
            // ring's.
            float *s_h = reinterpret_cast<float *>(&s_w[0][0][0]);      // [16 NC][256]
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
#pragma unroll
            for (int it = 0; it < IT; it++) {
                const int col = it * (WAVES * 16) + wave * 16 + r16;
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    if (c >= nblk) continue;
                    if (!shared) {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            s_h[(16 * c + 4 * g + i) * 256 + col] = silu(acc[it][c][0][i]) * acc[it][c][1][i];
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i += 2)
                            s_h[(8 * c + 2 * g + (i >> 1)) * 256 + col] =
                                silu(acc[it][c][0][i] + acc[it][c][0][i + 1]) *
                                (acc[it][c][1][i] + acc[it][c][1][i + 1]);
                    }
                }
            }
            __syncthreads();
            float *sv = reinterpret_cast<float *>(&s_act[0][0]) + wave * 256;
            const int sb = rbase / 256, nsb_h = (shared ? SF : FF) / 256;
            for (int t = wave; t < nt; t += WAVES) {
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = s_h[t * 256 + lane + 64 * c];
                if (!shared)
                    prep_values(v, job.ah, ACT_Q8K, job.perm[t_first + t], N * K, sb, nsb_h, sv);
                else
                    prep_values(v, job.ahs, ACT_SPLIT, t_first + t, N, sb, nsb_h, sv);
            }
            continue;
        }

        // results of the down products
        float *out = shared ? job.ys : job.ye;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int row0 = rbase + it * (WAVES * 32) + wave * 32;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if (c >= nblk) continue;
                if (!shared) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int q = 16 * c + 4 * g + i;
                        if (q >= nt) continue;
                        float *o = out + (size_t)job.perm[t_first + q] * H + row0 + r16;
#pragma unroll
                        for (int r = 0; r < RT; r++) o[16 * r] = acc[it][c][r][i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        const int q = 8 * c + 2 * g + (i >> 1);
                        if (q >= nt) continue;
                        float *o = out + (size_t)(t_first + q) * H + row0 + r16;
#pragma unroll
                        for (int r = 0; r < RT; r++) o[16 * r] = acc[it][c][r][i] + acc[it][c][r][i + 1];
                    }
                }
            }
        }
    }
}

int expert_rows_per_item(int phase) { return phase == 0 ? GROWS_GU : GROWS_DN; }

bool expert_k_ok(int K) { return K % 256 == 0; }

template <int PHASE>
static hipError_t launch_phase(int nc, const MoeJob &job, dim3 grid, hipStream_t s)
{
    switch (nc) {
    case 1: hipLaunchKernelGGL((k_expert_q4k<PHASE, 1>), grid, dim3(WAVES * 64), 0, s, job); break;
    case 2: hipLaunchKernelGGL((k_expert_q4k<PHASE, 2>), grid, dim3(WAVES * 64), 0, s, job); break;
    case 4: hipLaunchKernelGGL((k_expert_q4k<PHASE, 4>), grid, dim3(WAVES * 64), 0, s, job); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_expert_q4k(int phase, const MoeJob &job, hipStream_t s, int nc)
{
    if (job.FF % GROWS_GU || job.FF % 256 || job.H % GROWS_DN || job.H % 256 ||
        job.ax.K != job.H || job.ah.K != job.FF ||
        (job.has_shared && (job.SF != job.FF || job.ahs.K != job.SF)))
        return hipErrorInvalidValue;
    // routed work-list entries hold 16 nc pairs
    if ((nc != 1 && nc != 2 && nc != 4) || (job.wl.n_ec && job.wl.chunk != EXPERT_CHUNK * nc))
        return hipErrorInvalidValue;
    if (phase == 0) return launch_phase<0>(nc, job, dim3(DMOE_X_BLOCKS), s);
    // one workgroup per compute unit (one fits at a time), so that each
    // runs its items back to back with the rings running on between them
    static int n_cu[64] = {0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (n_cu[dev] <= 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        n_cu[dev] = n > 0 ? n : DMOE_X_BLOCKS;
    }
    return launch_phase<1>(nc, job, dim3(n_cu[dev]), s);
}

} // namespace dmoe

