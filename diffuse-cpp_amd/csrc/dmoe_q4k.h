// dmoe_q4k.h — Q4_K tile operands, LDS-direct loads and the int8 MFMA
// products shared by the Q4_K kernels (k_expert.hip: expert items;
// k_proj.hip: projections of few tokens).
//
// A weight tile is 16 rows x one 256-value super-block of the tiled layout
// (k_quant.hip): 144 16-byte pieces, piece 16 k + r of row r (k = 0: d, dmin
// and the repacked scales; k = 1 + 2 g, 2 + 2 g: the quant bytes lane group g
// needs).  An activation step (one super-block of 16 int8 rows) lies in LDS
// as the ASTEP layout below.  compute_sb / compute_folded form ggml's
// vec_dot_q4_K_q8_K products of a tile against the step's rows.
#pragma once

#include "dmoe_prep.h"

namespace dmoe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int TILE_BYTES = 16 * Q4K_BYTES;   // one tile x one super-block
constexpr int TPIECES = TILE_BYTES / 16;     // 16-byte pieces of a tile (144)
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

// One super-block of NT weight tiles against the step's activations.
template <int NT>
__device__ __forceinline__ void compute_sb(const Q4KTile (&cur)[NT], const uint8_t *ast, int r16, int g,
                                           float (&acc)[NT][4])
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
    for (int r = 0; r < NT; r++) {
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
        for (int i = 0; i < 4; i++) acc[r][i] = q4k_epi(acc[r][i], dx[i], d, (float)isum[i], dmin, s2[i]);
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
        acc[i] = q4k_epi(acc[i], dx[i], f.d, (float)isum, f.dmin, s2[i]);
    }
}

} // namespace dmoe
