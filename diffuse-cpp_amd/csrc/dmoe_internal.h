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
};

struct RouteParams {
    int32_t n_tokens, n_experts, top_k, capacity, block_size;
    int32_t use_block;      // block routing on (diffuse-moe-graph.cpp:215-216)
    int32_t norm_topk_prob;
    float routed_scaling;
};

// ---------------------------------------------------------------------------
// Kernel launchers (each returns the hipGetLastError of its launch).
hipError_t launch_router_logits(const float *W, const float *x, int N, int H, int E,
                                float *logits, hipStream_t s);
hipError_t launch_route(const RouteParams &rp, const float *logits, const float *bias,
                        const RouteBufs &rb, hipStream_t s);
hipError_t launch_dispatch(const RouteParams &rp, const RouteBufs &rb, hipStream_t s);

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
