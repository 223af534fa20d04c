// dmoe_internal.h — device-side types and launch declarations shared by the
// HIP sources of libdmoe (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/dmoe.h"

// Q8_K is an activation-only type (ggml id 15): the vec_dot_type of Q4_K.
#define DMOE_ACT_Q8_K 15

namespace dmoe {

// ---------------------------------------------------------------------------
// Block byte sizes (GGUF layouts).
constexpr int QK_K = 256;          // super-block of Q4_K / Q8_K
constexpr int QK8_0 = 32;          // block of Q8_0
constexpr int Q4K_BYTES = 144;     // f16 d, f16 dmin, u8 scales[12], u8 qs[128]
constexpr int Q8_0_BYTES = 34;     // f16 d, i8 qs[32]
constexpr int Q6K_BYTES = 210;     // u8 ql[128], u8 qh[64], i8 scales[16], f16 d

// Activation operand of one expert product, in the layout the kernels read.
//   F32 : f32  [rows][n]
//   F16 : f16  [rows][n]
//   Q8_0: i8 qs[rows][n], f32 d[rows][n/32]   (d = fp16-rounded block scale)
//   Q8_K: i8 qs[rows][n], f32 d[rows][n/256], i16 bsums[rows][n/16]
struct ActBuf {
    int32_t type;
    int32_t n;          // elements per row
    void *vals;         // f32 / f16 / i8 values
    float *d;           // block scales (Q8_0, Q8_K)
    int16_t *bsums;     // Q8_K only
};

// One expert tensor (or the shared one) on the device.
struct WTensor {
    int32_t type;
    const uint8_t *data;
    size_t nb1;         // bytes between rows
    size_t nb2;         // bytes between experts
};

// Routing scratch of one forward.
struct RouteBufs {
    float *logits;      // [N][E]
    float *probs;       // [N][E]
    float *bmax;        // [B][E]
    float *thr;         // [B]
    uint8_t *allowed;   // [B][E]
    int32_t *idx;       // [N][K]
    float *weights;     // [N][K]
    int32_t *counts;    // [E]
    int32_t *offsets;   // [E+1]
    int32_t *perm;      // [N*K]
    int32_t *hist;      // [groups][E] pairs of each routing group per expert
    int32_t *lrank;     // [N*K] rank of a pair among its group's pairs of its expert
    float *sel;         // [N][E] selection scores probs + bias
};

// Group scores kept in LDS by the routing kernel (group tokens x experts).
constexpr int ROUTE_LDS = 8192;

// Work list of the expert kernels: one entry per (expert, chunk of `chunk`
// consecutive pairs of that expert), in expert order.
struct WorkList {
    int32_t chunk;
    int32_t *n_ec;       // [1]
    int32_t *ec_expert;  // [E + N*K/chunk + 1]
    int32_t *ec_chunk;
};

// Activations of the Q4_K expert products (k_expert.hip), int8 per value.
// Per row of K values and per 256-value super-block the bytes are stored in the
// order the MFMA lanes read them: position 64g + 8j + b holds value
// 32j + 8g + b of the super-block (j = 32-value sub-block, g = lane group,
// b = byte), so that a lane group's eight 8-byte pieces are contiguous.
//   ACT_Q8K  : ggml's Q8_K quantisation (d = Q8_K scale, q in [-127, 127]).
//   ACT_SPLIT: f32 values (the shared expert) as two int8 digits: with a
//              power-of-two scale s per super-block, X = round(v / s),
//              |X| <= 32512, X = 256*a1 + a0; rows 0..rows-1 hold a1 (d = 256 s)
//              and rows rows..2*rows-1 hold a0 (d = s).
// bs holds the f16 sums of each 16 consecutive values (exact: |sum| <= 2048).
//   ACT_Q80  : ggml's Q8_0 quantisation per 32 values (d = amax/127,
//              q = roundf(v * (1/d)), d kept as its fp16 rounding); d holds
//              one scale per 32 values and bs is unused (the Q8_0 expert
//              kernel, k_expert_q80.hip).
//   ACT_SPLIT32: ACT_SPLIT with the power-of-two scale chosen per 32 values,
//              d per 32 values, bs unused (the Q8_0 kernel's shared expert).
enum ActMode { ACT_Q8K = 0, ACT_SPLIT = 1, ACT_Q80 = 2, ACT_SPLIT32 = 3 };
struct ActI8 {
    int32_t K;
    int8_t *q;          // [rows][K]
    uint16_t *bs;       // [rows][K/16] (Q8K, SPLIT)
    float *d;           // [rows][K/256] (Q8K, SPLIT) or [rows][K/32] (Q80, SPLIT32)
};

// The expert products of one forward (routed experts + the shared one),
// k_expert.hip: phase 0 (gate/up) and phase 1 (down) launches.
struct MoeJob {
    WTensor eg, eu, ed;      // routed gate, up, down (tiled Q4_K)
    WTensor sg, su, sd;      // shared expert
    int32_t has_shared;
    int32_t H, FF, SF;       // n_embd, moe_ff, shared_ff
    int32_t n_tokens, top_k;
    const int32_t *perm, *offsets, *counts;
    int32_t E, ec_cap;       // routed experts (offsets / counts length), work-list length (0: none)
    WorkList wl;
    ActI8 ax, axs;         // x converted: Q8_K (rows: tokens), split (shared)
    float *h, *hs;           // gate/up results [N*K][FF], [N][SF]
    ActI8 ah, ahs;         // h and hs converted for the down products
    float *ye, *ys;          // down results [N*K][H], [N][H]
    // Grouped Q4_K GEMM down launches with only shared units (a projection of
    // many tokens, k_expert_gemm.hip): the reduction in ks slices, slice s's
    // results at ys + s N H (0 or 1: one slice, ys itself)
    int32_t ks;
    // F16 experts (k_expert_tile.hip): x and h as f16 rows, the shared
    // expert's as hi / lo pairs (lo rows after the hi rows)
    const uint16_t *x16, *xs16;
    uint16_t *h16, *hs16;
};

// Alternative kernels kept selectable for measurement, read from the
// environment by dmoe_create into its context (never in a forward):
//   DMOE_Q4K_COLUMN_BLOCKS = 1, 2, 4  column blocks of the Q4_K items (0: by tokens per expert)
//   DMOE_DOWN_FUSED = 1               few-token Q4_K down products as the single fused launch
//   DMOE_GATEUP_LDS = 1               the LDS-ring gate/up kernel instead of the register ring
//   DMOE_EXPERT_TILE = 0 / 1          the tile kernels (k_expert_tile.hip) off / on for every N
//   DMOE_EXPERT_GEMM = 0 / 1          the Q4_K grouped GEMM (k_expert_gemm.hip) off / on for every N
//   DMOE_PROJ_GEMM = 0 / 1            Q4_K projections (attention, LM head) past the few-token
//                                     kernel on that GEMM off / on for every N
struct KernelSwitches {
    int q4k_column_blocks = 0;
    int expert_tile = -1;                // -1: by tokens per expert
    int expert_gemm = -1;                // -1: by tokens per expert
    int proj_gemm = -1;                  // -1: by tokens
    int attn_waves = 0;                  // 0: by grid size, else 4 or 8 per workgroup
    bool down_fused = false;
    bool gateup_lds = false;
};

struct RouteParams {
    int32_t n_tokens, n_experts, top_k, capacity, block_size;
    int32_t use_block;      // block routing on (diffuse-moe-graph.cpp:215-216)
    int32_t norm_topk_prob;
    float routed_scaling;
    int32_t bias_small;     // no bias, or every bias finite with |bias| < 1e19
    const float *bias;      // [E] or null
};

// ---------------------------------------------------------------------------
// Kernel launchers (each returns the hipGetLastError of its launch).
// F16 expert products on MFMA, the prefill path (k_gemm.hip).
constexpr int GM = 128;             // (token, slot) pairs per work item
constexpr int GK = 32;              // k per pipeline step
constexpr int GN_GU = 256;          // moe_ff rows of a gate/up item (gate and up)
constexpr int GN_DN = 512;          // n_embd rows of a down item
constexpr int GEMM_BLOCKS = 1024;   // persistent grid
struct GemmJob {
    WTensor eg, eu, ed;      // routed gate, up, down (F16, ggml row layout)
    WTensor sg, su, sd;      // shared expert (F16)
    int32_t has_shared;
    int32_t H, FF, SF;       // n_embd, moe_ff, shared_ff
    int32_t n_tokens, top_k;
    const int32_t *perm, *offsets, *counts;
    WorkList wl;             // chunk == GM
    const uint16_t *x16;     // [N][H]  f16(x)
    const uint16_t *xs16;    // [2N][H] hi / lo pair of x (shared expert)
    uint16_t *h16;           // [N*K][FF] f16(h)
    uint16_t *hs16;          // [2N][SF] hi / lo pair of the shared h
    float *ye, *ys;          // down results [N*K][H], [N][H]
};
hipError_t launch_gemm_f16(int phase, const GemmJob &job, hipStream_t s);
bool gemm_shapes_ok(int H, int FF, int SF, bool shared);
// x (f32) -> f16, or its hi / lo f16 pair (lo rows after the hi rows)
hipError_t launch_cvt_f16(const float *src, int rows, int K, int split, uint16_t *dst, hipStream_t s);
// F16 matrices -> the tiled layout of k_gemm.hip: per matrix, 128-row blocks,
// k-step-major (rows x 32 values of k step ks of block b at
// (b*K/32 + ks)*8192), row r of a step at (r%128)*64 with 16-byte chunk q at
// slot q ^ ((r >> 1) & 3).
hipError_t launch_tile_f16(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s);

// Residual add and RMSNorm of the residual stream (k_norm.hip): per row of H
// floats (H % 4 == 0, 16-byte aligned rows), h += y (y may be null), then
// x = rms_norm(h, eps) * gain (gain may be null).
// rows of h_in (+ the sum of y's ks slices, kstride floats apart, written to
// h_out when given) -> rms_norm * gain to x (f32, when given) and / or act
// (two int8 digit rows per row, ACT_SPLIT, when act.q is given); H <= 8192
struct NormArgs {
    const float *h_in;
    float *h_out;
    const float *y;
    int32_t ks;
    size_t kstride;
    const float *gain;
    float *x;
    ActI8 act;
    int32_t rows, H;
    float eps;
};
hipError_t launch_norm_fused(const NormArgs &a, hipStream_t s);
hipError_t launch_residual_rmsnorm(float *h, const float *y, const float *gain, float *x, int rows, int H,
                                   float eps, hipStream_t s);

// One activation conversion into the MFMA operand layout.
struct PrepJob {
    const float *src;
    int32_t rows, K, mode;   // K % 256 == 0
    ActI8 out;
};

// Routing + dispatch (k_router.hip).  When the forward is one routing group
// (route_single), up to two activation conversions may ride along in the
// same launch: their workgroups run beside the routing workgroup, on compute
// units it leaves idle.
hipError_t launch_route(const RouteParams &rp, const RouteBufs &rb, const WorkList &wl, hipStream_t s,
                        const PrepJob *jobs = nullptr, int njobs = 0);
bool route_fits_lds(const RouteParams &rp);
bool route_single(const RouteParams &rp);
// Front kernel (k_prep.hip): router logits L = Wg x in one fixed fp32 order,
// probs = sigmoid(L), sel = probs + bias, plus up to two activation
// conversions of x, in one launch.
hipError_t launch_front(const float *W, const float *bias, const float *x, int N, int H, int E,
                        const RouteBufs &rb, const PrepJob *jobs, int njobs, hipStream_t s);
// probs and sel from given logits (routing-only entry point)
hipError_t launch_scores(const float *logits, const float *bias, int N, int E,
                         const RouteBufs &rb, hipStream_t s);
// Up to two activation conversions in one launch.
hipError_t launch_prep(const PrepJob *jobs, int njobs, hipStream_t s);
// p[0 .. n) = v
hipError_t launch_fill_i32(int32_t *p, int32_t v, int n, hipStream_t s);
// The attention half of the layer (k_attn.hip).
struct AttnDims {
    int32_t n, nh, nkv, hd, rd;          // tokens, heads, kv heads, head_dim, rotary_dim
    int32_t qk_norm, block;              // use_qk_norm, block_length (0: bidirectional)
    float eps, theta_scale, scale;       // rms eps, powf(base, -2/rd), 1/sqrt(hd)
    int32_t waves;                       // attention wavefronts per workgroup: 4, 8, 0 by grid size
};
// fused QKV rows [N][(nh + 2 nkv) hd] (the sum of ks slices kstride floats
// apart) -> QK RMSNorm, partial NEOX RoPE -> head-major Q [nh][N][hd], K, V
// [nkv][N][hd]
hipError_t launch_qk_rope(const float *qkv, int ks, size_t kstride, const float *qn, const float *kn,
                          const AttnDims &a, float *Qh, float *Kh, float *Vh, hipStream_t s);
// block-causal GQA attention -> out [N][nh hd]
hipError_t launch_attn(const float *Qh, const float *Kh, const float *Vh, const AttnDims &a, float *out,
                       hipStream_t s);
// Per row of V logits: the argmax (first index of the largest) and its
// softmax probability 1 / sum exp(l - max) (k_head.hip), through per-chunk
// partials (argmax_partials_bytes of workspace).
struct ArgmaxPart {
    float m;                             // the chunk's largest logit
    int idx;                             // its first index (V: none above -inf)
    double sum;                          // sum of exp(l - m) over the chunk
};
size_t argmax_partials_bytes(int N, int V);
hipError_t launch_argmax_prob(const float *logits, int N, int V, ArgmaxPart *part, int32_t *tokens,
                              float *probs, hipStream_t s);
// Q4_K projections of few tokens with F32 weight semantics (k_proj.hip):
// matrices w[0..M-1] (tiled Q4_K, R rows, reduction K) against x as two int8
// digit rows per token (ACT_SPLIT); the reduction runs in KS slices.
constexpr int PROJ_MAX_TOKENS = 32;
struct ProjJob {
    const uint8_t *w[2];
    int32_t M, R, K, N, KS;
    ActI8 x;
    float *out;              // partial: [M][KS][N][R] slice sums; else y [N][ldo] (M = KS = 1)
    int32_t partial, ldo;
};
bool proj_ok(int R, int K, int N);
struct ProjPlan {
    int T;                   // 16-row tiles per wavefront
    int KS;                  // reduction slices
};
ProjPlan proj_plan(int R, int K, int M, int N);          // the launch shape for a projection
size_t proj_partial_floats(int R, int K, int M, int N);  // partial buffer of that KS
hipError_t launch_proj_q4k(const ProjJob &j, hipStream_t s);
// the same for Q6_K matrices (tiled by launch_tile_q6k)
hipError_t launch_proj_q6k(const ProjJob &j, hipStream_t s);
// y [N][ldy] = the KS slices of part [KS][N][R] added in slice order
hipError_t launch_proj_reduce(const float *part, int KS, int N, int R, float *y, int ldy, hipStream_t s);
// h = silu(gate) up from part [2][KS][N][R], to ah (two int8 digit rows per token)
hipError_t launch_proj_swiglu(const float *part, int KS, int N, int R, const ActI8 &ah, hipStream_t s);

// Grouped Q4_K expert products on MFMA (k_expert.hip).  phase 0: h = silu(gate x)
// * (up x); phase 1: y = down h.
constexpr int EXPERT_CHUNK = 16;    // pairs of one expert per work item
constexpr int SHARED_CHUNK = 8;     // tokens per shared-expert work item
// nc: activation column blocks of 16 pairs per routed item (1, 2 or 4; the
// work list's chunk is 16 nc): each weight tile read serves 16 nc pairs.
hipError_t launch_expert_q4k(int phase, const MoeJob &job, hipStream_t s, int nc = 1, bool gateup_lds = false);
// Expert products with each item's activations held in LDS (k_expert_tile.hip):
// Q4_K and Q8_0 experts with many tokens per expert, F16 experts with few.
// Units of up to expert_tile_chunk(type) pairs (the work list's chunk) or
// half as many shared tokens; phase 0 writes f32 h / hs ([N K][FF],
// [N][SF]) for a conversion launch into ah / ahs (Q4_K, Q8_0) or h16 / hs16
// (F16), phase 1 writes ye / ys for the combine.
bool expert_tile_ok(int H, int FF, int SF, bool shared);
int expert_tile_chunk(int32_t type);
hipError_t launch_expert_tile(int phase, const MoeJob &job, hipStream_t s);
// Q4_K expert products as a grouped int8-MFMA GEMM for many pairs per expert
// (k_expert_gemm.hip): units of up to 128 pairs (the work list's chunk) or
// 64 shared tokens, a step's weights and activations streamed through LDS
// together; h / hs and ye / ys as with the tile kernels.
constexpr int EXPERT_GEMM_CHUNK = 128;
bool expert_gemm_q4k_ok(int H, int FF, int SF, bool shared);
hipError_t launch_expert_gemm_q4k(int phase, const MoeJob &job, hipStream_t s);
// Down products of the Q4_K experts and the weighted combine in one launch
// for few tokens (k_down_rows.hip): one workgroup per 16 output rows, every
// touched expert's 16-row tile, results folded in slot order in LDS.
constexpr int DR_MAX_PAIRS = 1024;      // (token, slot) pairs of one launch
constexpr int DR_MAX_TOKENS = 128;
struct DownRowsJob {
    WTensor ed, sd;                 // tiled Q4_K down weights (routed, shared)
    int32_t has_shared;
    int32_t N, K, E, H, FF;         // tokens, top_k, experts, n_embd, moe_ff (== shared_ff)
    const int32_t *perm, *offsets, *counts;
    WorkList wl;                    // chunk == EXPERT_CHUNK
    int32_t ec_cap;                 // allocated work-list length
    ActI8 ah, ahs;                  // h in the int8 layout (routed pairs; shared digit rows)
    const float *weights;           // [N][K] gate weights
    float *y;                       // [N][H] segment output
    float *ye, *ys;                 // k_down_span: per-pair [N K][H] and shared [N][H] products
};
bool down_rows_ok(int N, int K, int E, int H, int FF);
hipError_t launch_down_rows(const DownRowsJob &job, hipStream_t s);
// The same products by spans of (unit, 16-row tile) work, one workgroup per
// CU, to ye / ys; launch_combine folds them (k_down_span.hip).
bool down_span_ok(int N, int K, int E, int H, int FF, int has_shared);
hipError_t launch_down_span(const DownRowsJob &job, hipStream_t s);
// Compute units of the current device (k_expert.hip).
hipError_t device_cu_count(int *out);
// The same products for Q8_0 experts (k_expert_q80.hip): activations in the
// ActI8 layout with ACT_Q80 / ACT_SPLIT32 scales, weights in the Q8_0 tiled
// layout of launch_tile_q80.
hipError_t launch_expert_q80(int phase, const MoeJob &job, hipStream_t s);
int expert_q80_rows_per_item(int phase);
// GGUF Q8_0 rows -> tiled layout: per matrix, 16-row tiles, 256-value-step-
// major (16 rows x 256 values of step sb of tile t: the 4352-byte run at
// (t*nsb + sb)*4352); a row's 272 bytes of a step are seventeen 16-byte
// pieces, piece k of row r at (16k + r)*16: piece 0 the eight fp16 scales,
// pieces 1+4g .. 4+4g the quants 8g .. 8g+7 of blocks 0..7 (8 bytes each).
hipError_t launch_tile_q80(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s);
int expert_rows_per_item(int phase);     // output rows one work item covers
bool expert_k_ok(int K);                 // reduction length the expert kernels accept
// Q4_K row layout -> tiled layout of k_expert.hip (k_quant.hip): per matrix,
// 16-row tiles, super-block-major (the 16 rows of super-block sb of tile t
// are the 2304-byte run at (t*nsb + sb)*2304); inside a run, byte b of the
// repacked block of row r (r < 16) is at ((b/16)*16 + r)*16 + b%16.  In the
// repacked 144-byte block d and dmin stay in bytes 0..3, the twelve scale
// bytes are repacked (dword 1: sc0..sc4, dword 2: sc5..sc7 m0 m1, dword 3:
// m2..m6, six bits each; m7 in bits 30..31 of the three dwords, low bits
// first) and the 128 quant bytes are reordered so that byte 16 + 32g + 8c + b
// holds quant byte 32c + 8g + b.
hipError_t launch_tile_q4k(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s);
// Q6_K rows -> the tiled layout of the Q6_K projections (k_quant.hip
// describes the 3360-byte tile-step runs); same byte count.
hipError_t launch_tile_q6k(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s);

hipError_t launch_act_quant(const float *src, int rows, int n, const ActBuf &dst,
                            hipStream_t s);

// h[pair][ff] = silu(Wg[e] x) * (Wu[e] x) for every routed (token, slot) pair.
hipError_t launch_gateup_routed(const WTensor &wg, const WTensor &wu, const ActBuf &xq,
                                const RouteParams &rp, const RouteBufs &rb, int ff,
                                float *h, hipStream_t s);
// ye[pair][H] = Wd[e] hq[pair]
hipError_t launch_down_routed(const WTensor &wd, const ActBuf &hq, const RouteParams &rp,
                              const RouteBufs &rb, int H, float *ye, hipStream_t s);
// Shared expert with f32 activations on dequantised weights.
hipError_t launch_gateup_shared(const WTensor &wg, const WTensor &wu, const float *x,
                                int N, int H, int sff, float *hs, hipStream_t s);
hipError_t launch_down_shared(const WTensor &wd, const float *hs, int N, int sff, int H,
                              float *ys, hipStream_t s);
// y[t] = sum_slot fl(ye*w) (left fold) + ys
hipError_t launch_combine(const float *ye, const float *weights, const float *ys,
                          int N, int K, int H, float *y, hipStream_t s);

hipError_t launch_quantize_weights(int32_t type, const float *src, void *dst,
                                   int64_t nrows, int64_t n_per_row, hipStream_t s);

} // namespace dmoe
