/*
 * dmoe_oracle.h — CPU oracle for the LLaDA2 block-routed MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  The parity tests compare against it: tests/, the smoke
 * entry and the CPU-baseline leg of bench.py may load it; the product library
 * (libdmoe.so) never links, loads or calls it.
 *
 * It restates, in plain C, what src/diffuse-moe-graph.cpp:188-289 computes
 * when ggml executes that graph on the CPU (every function cites the line it
 * follows).  ggml itself is absent from the reference checkout (empty git
 * submodule), so the ggml-internal semantics below are restated from ggml's
 * published algorithms and are marked "ggml-internal" where they cannot be
 * checked against the reference's own files.
 *
 * Parity status of each function (how it is pinned by tests/):
 *   dmo_f16_to_f32 / dmo_f32_to_f16  pinned: numpy float16 on all 65536 halves
 *                                    and on random/edge f32 inputs
 *   dmo_expf                         pinned: numpy float64 exp rounded to f32
 *                                    (correctly rounded) on 10^7 inputs + edges
 *   dmo_dequant_row (F16/Q8_0/Q4_K)  pinned: hand-built blocks with known values,
 *                                    all 8 get_scale_min_k4 indices
 *   dmo_dequant_row (Q6_K)           pinned: hand-built blocks (every quant
 *                                    value 0..63 at every position class,
 *                                    negative scales, the published bit
 *                                    layout written out independently)
 *   dmo_quantize_row_act (Q8_K/Q8_0) pinned: hand-computed blocks, half-even /
 *                                    half-away rounding cases, numpy restatement
 *   dmo_vec_dot                      pinned: float64 dot of the dequantised rows
 *                                    (integer parts exact, closed-form bound)
 *   dmo_router_logits                pinned: float64 matmul bound + a brute-force
 *                                    numpy emulation of the canonical order
 *   dmo_route                        pinned: brute force on tiny inputs, fold KAT
 *                                    (0x3f61fdaf, 0x3ea25e9b), slack / ties /
 *                                    cap>=E / N%blk!=0 special cases
 *   dmo_dispatch                     pinned: permutation / histogram / scan
 *                                    invariants
 *   dmo_layer_forward                pinned: float64 numpy layer on dequantised
 *                                    weights within an analytic error budget
 *   dmo_dense_forward                pinned: float64 numpy SwiGLU on dequantised
 *                                    weights within the same error budget
 *   dmo_rms_norm                     pinned: float64 numpy on random rows, an
 *                                    all-equal row (closed form)
 *   dmo_argmax_prob                  pinned: known answers (ties to the first
 *                                    index, NaN first element, one-hot and
 *                                    uniform rows) and float64 softmax
 *   dmo_head_forward                 pinned: float64 numpy logits on the
 *                                    dequantised output weight
 *   dmo_rope_neox                    pinned: float64 rotation with the same
 *                                    angle chain (and the closed-form angle
 *                                    within the chain's rounding); norm kept
 *   dmo_attn_forward                 pinned: float64 numpy attention (mask,
 *                                    GQA head map, RoPE, QK norm, residual)
 */
#ifndef DMOE_ORACLE_H
#define DMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/dmoe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- block formats (ggml / GGUF) --------------------------------------- */
#define DMO_QK_K 256
#define DMO_QK8_0 32

typedef struct { uint16_t d; int8_t qs[32]; } dmo_block_q8_0;            /* 34 B  */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } dmo_block_q4_K; /* 144 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } dmo_block_q8_K;  /* 292 B */
/* Q6_K: low 4 bits of the 256 quants, their high 2 bits, 16 signed 8-bit
 * sub-block scales (one per 16 weights), the f16 super-block scale */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } dmo_block_q6_K; /* 210 B */

float    dmo_f16_to_f32(uint16_t h);
uint16_t dmo_f32_to_f16(float f);
void     dmo_f16_to_f32_n(const uint16_t *h, float *f, int64_t n);
void     dmo_f32_to_f16_n(const float *f, uint16_t *h, int64_t n);

/* AVX-512 VNNI versions of the Q4_K x Q8_K and Q8_0 x Q8_0 dots
 * (dmoe_cpu_simd.c; bit-identical to the scalar dots, for the timed CPU
 * baseline).  dmo_set_simd(1) routes dmo_vec_dot through them when the CPU
 * has AVX-512 F / BW and VNNI; returns whether it does. */
int      dmo_simd_available(void);
int      dmo_set_simd(int on);
float    dmo_dot_q4K_simd(int64_t n, const dmo_block_q4_K *w, const dmo_block_q8_K *x);
float    dmo_dot_q8_0_simd(int64_t n, const dmo_block_q8_0 *w, const dmo_block_q8_0 *x);
float    dmo_dot_f32_simd(int64_t n, const float *w, const float *x);
float    dmo_dot_f16_simd(int64_t n, const uint16_t *w, const uint16_t *x);
void     dmo_rows_q4K_simd(int64_t n, const dmo_block_q4_K *w, const uint8_t *act, size_t act_stride,
                           const int32_t *rows_in, int n_in, float *out, size_t out_stride);

float    dmo_expf(float x);
void     dmo_expf_n(const float *x, float *y, int64_t n);
float    dmo_sigmoid(float x);

size_t   dmo_row_size(int32_t type, int64_t n);
int32_t  dmo_vec_dot_type(int32_t type);   /* activation type ggml converts to */

/* get_scale_min_k4 of ggml's Q4_K */
void     dmo_q4K_scale_min(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
int      dmo_q6K_quant(const dmo_block_q6_K *b, int i);

int      dmo_dequant_row(int32_t type, const void *src, float *dst, int64_t n);
/* weight quantisers used to build synthetic GGUF tensors */
int      dmo_quantize_rows(int32_t type, const float *src, void *dst,
                           int64_t nrows, int64_t n_per_row, int n_threads);
/* activation quantisers (ggml vec_dot_type semantics): type is Q8_K (id 15),
 * Q8_0, F16 or F32 */
#define DMO_TYPE_Q8_K 15
int      dmo_quantize_row_act(int32_t act_type, const float *src, void *dst, int64_t n);

/* dot of one weight row (type wtype) with one activation row already in
 * dmo_vec_dot_type(wtype). */
float    dmo_vec_dot(int32_t wtype, int64_t n, const void *wrow, const void *xrow);

/* ---- router -------------------------------------------------------------- */
void dmo_router_logits(const float *W, int64_t w_row_stride, const float *x,
                       int n_tokens, int n_embd, int n_experts, float *logits);

int  dmo_use_block_routing(const dmoe_hparams *hp, int n_tokens);

/* the block max fold of n scores s[0], s[stride], ... */
float dmo_block_fold(const float *s, int n, int stride);

/* Routing from logits.  probs [N][E]; bmax [B][E], thr [B], allowed [B][E]
 * (only written with block routing; may be NULL); idx, weights [N][k]. */
int  dmo_route(const dmoe_hparams *hp, const float *bias, const float *logits,
               int n_tokens, float *probs, float *bmax, float *thr,
               uint8_t *allowed, int32_t *idx, float *weights);

void dmo_dispatch(const int32_t *idx, int n_tokens, int top_k, int n_experts,
                  int32_t *counts, int32_t *offsets, int32_t *perm);

/* ---- whole segment -------------------------------------------------------
 * y = moe_out for x [N][n_embd].  dbg may be NULL.  n_threads <= 0: all. */
int  dmo_layer_forward(const dmoe_hparams *hp, const dmoe_layer_desc *desc,
                       const float *x, int n_tokens, float *y,
                       dmoe_debug *dbg, int n_threads);

/* Dense SwiGLU MLP of the first_k_dense layers (src/diffuse-moe-graph.cpp:
 * 181-187): y = W_down (silu(W_gate x) * (W_up x)), weights cast to F32,
 * F32 activations.  gate, up [n_embd, n_ff]; down [n_ff, n_embd]. */
int  dmo_dense_forward(int n_embd, int n_ff, const dmoe_tensor *gate, const dmoe_tensor *up,
                       const dmoe_tensor *down, const float *x, int n_tokens, float *y,
                       int n_threads);

/* ---- step tail ------------------------------------------------------------
 * ggml_rms_norm (binary64 sum of the f32 squares) times w (may be NULL). */
void dmo_rms_norm(const float *x, const float *w, int n, float eps, float *out);
/* sample_token at temperature 0 (src/diffuse-sampler.cpp:29-49). */
void dmo_argmax_prob(const float *logits, int n_vocab, int32_t *token, float *prob);
/* src/diffuse-moe-graph.cpp:295-300 then the sampler's argmax and confidence:
 * x = rms_norm(h, eps) * norm_w, logits = output x (output [n_embd, n_vocab]
 * cast to F32), per token the argmax and its softmax probability.
 * logits_out [N][V] may be NULL. */
int  dmo_head_forward(int n_embd, int n_vocab, const float *norm_w, const dmoe_tensor *output,
                      const float *h, int n_tokens, float eps, int32_t *tokens, float *probs,
                      float *logits_out, int n_threads);

/* ---- attention half of the layer -----------------------------------------
 * ggml_rope_ext, NEOX mode, n_dims rotated of head_dim, at position pos. */
void dmo_rope_neox(float *x, int head_dim, int n_dims, int pos, float base);
/* src/diffuse-moe-graph.cpp:116-178: h_out = h + wo attn(h), moe_in =
 * rms_norm(h_out) * post_attn_norm (may be NULL). */
int  dmo_attn_forward(const dmoe_attn_hparams *ap, const dmoe_attn_desc *desc, const float *h,
                      int n_tokens, float *h_out, float *moe_in, int n_threads);

#ifdef __cplusplus
}
#endif

#endif
