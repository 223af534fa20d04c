// dmoe_q80.h — the Q8_0 tile products shared by the Q8_0 expert kernels
// (k_expert_q80.hip: LDS rings; k_expert_tile.hip: many tokens per expert).
//
// A weight tile is 16 rows x one 256-value step of the Q8_0 tiled layout
// (k_tile_q80): piece 0 of row r the eight fp16 block scales, pieces
// 1 + 4g .. 4 + 4g lane group g's quants (byte 8j + b of the group's 64 =
// quant 8g + b of block j).  An activation step (one 16-row block) in LDS:
// q [16][256] int8 with the Q4_K kernels' swizzle (16-byte unit u of row r
// at u ^ (r & 11)), then the per-32 scales [8 blocks][16 rows] f32 at
// Q80_AD_OFF.
#pragma once

#include "dmoe_device.h"

namespace dmoe {

constexpr int Q80_STEP_ROW = 8 * Q8_0_BYTES;          // 272 bytes of a row per 256 values
constexpr int Q80_TILE = 16 * Q80_STEP_ROW;           // 4352
constexpr int Q80_ASTEP = 4096 + 512;                 // one block's activation step in LDS
constexpr int Q80_AD_OFF = 4096;

typedef int q80_v4i __attribute__((ext_vector_type(4)));

// ggml's vec_dot_q8_0_q8_0 for one tile step against one activation block:
// per 32-value block jb, sum += (float)(sum_k q_w q_x) * (d_w * d_x) (the
// scale product exact in f32), the eight blocks in order by explicit fused
// multiply-adds (so every kernel rounds alike whatever its contraction
// setting), then acc += sum.  a: the activation operands of block jb (row
// r16, lane group g's bytes); w: the weight operands; wd: the tile's piece 0
// of row r16; ast: the activation step (for the scales).
__device__ __forceinline__ void q80_products(const long (&a)[8], const long (&w)[8], const uint4 &wd,
                                             const uint8_t *ast, int g, float (&acc)[4])
{
    const uint32_t wds[4] = {wd.x, wd.y, wd.z, wd.w};
    q80_v4i sj[8];
#pragma unroll
    for (int jb = 0; jb < 8; jb++) {
        const q80_v4i z = {0, 0, 0, 0};
        sj[jb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[jb], w[jb], z, 0, 0, 0);
    }
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int jb = 0; jb < 8; jb++) {
        const uint32_t hw = jb & 1 ? wds[jb >> 1] >> 16 : wds[jb >> 1] & 0xffffu;
        const float dw = (float)__builtin_bit_cast(_Float16, (uint16_t)hw);
        // scales of block jb for activation rows 4g .. 4g+3
        const float4 dx = *reinterpret_cast<const float4 *>(ast + Q80_AD_OFF + jb * 64 + 16 * g);
        const float dxa[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int i = 0; i < 4; i++) sum[i] = __builtin_fmaf((float)sj[jb][i], dw * dxa[i], sum[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] += sum[i];
}

// The activation operands of row r16, lane group g from a step in LDS.
__device__ __forceinline__ void q80_act_ops(const uint8_t *ast, int r16, int g, long (&a)[8])
{
    const uint4 *ap = reinterpret_cast<const uint4 *>(ast + r16 * 256);
    const uint4 a01 = ap[(4 * g + 0) ^ (r16 & 11)], a23 = ap[(4 * g + 1) ^ (r16 & 11)];
    const uint4 a45 = ap[(4 * g + 2) ^ (r16 & 11)], a67 = ap[(4 * g + 3) ^ (r16 & 11)];
    a[0] = (long)((uint64_t)a01.y << 32 | a01.x);
    a[1] = (long)((uint64_t)a01.w << 32 | a01.z);
    a[2] = (long)((uint64_t)a23.y << 32 | a23.x);
    a[3] = (long)((uint64_t)a23.w << 32 | a23.z);
    a[4] = (long)((uint64_t)a45.y << 32 | a45.x);
    a[5] = (long)((uint64_t)a45.w << 32 | a45.z);
    a[6] = (long)((uint64_t)a67.y << 32 | a67.x);
    a[7] = (long)((uint64_t)a67.w << 32 | a67.z);
}

// The weight operands of a tile step from lane group g's four quant pieces.
__device__ __forceinline__ void q80_w_ops(const uint4 &w01, const uint4 &w23, const uint4 &w45, const uint4 &w67,
                                          long (&w)[8])
{
    w[0] = (long)((uint64_t)w01.y << 32 | w01.x);
    w[1] = (long)((uint64_t)w01.w << 32 | w01.z);
    w[2] = (long)((uint64_t)w23.y << 32 | w23.x);
    w[3] = (long)((uint64_t)w23.w << 32 | w23.z);
    w[4] = (long)((uint64_t)w45.y << 32 | w45.x);
    w[5] = (long)((uint64_t)w45.w << 32 | w45.z);
    w[6] = (long)((uint64_t)w67.y << 32 | w67.x);
    w[7] = (long)((uint64_t)w67.w << 32 | w67.z);
}

} // namespace dmoe
