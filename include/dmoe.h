/*
 * dmoe.h — C ABI of the MI355X-native LLaDA2 block-routed MoE layer.
 *
 * One call computes the MoE segment that Akicou/diffuse-cpp builds out of
 * ggml ops in src/diffuse-moe-graph.cpp:188-289: sigmoid router with a
 * selection-only expert bias, per-block expert capacity, per-token top-k inside
 * the allowed set, renormalised and scaled gate weights, grouped SwiGLU
 * experts over GGUF block-quantised weights, weighted combine and the
 * always-on shared expert.  The output is `moe_out` (diffuse-moe-graph.cpp:288),
 * i.e. the segment output BEFORE the residual add of :291-292.
 *
 * Conventions
 *  - Plain pointers and sizes only.  No exception crosses this boundary; every
 *    entry point returns a dmoe_status and never calls exit()
 *    (the reference aborts with DIFFUSE_DIE, src/diffuse-common.h:23-26).
 *  - Tensor shapes use ggml `ne` order (ne[0] contiguous), byte strides `nb`,
 *    exactly as the ggml_tensor fields the reference holds in
 *    diffuse_moe_layer (src/diffuse-common.h:72-82).
 *  - Activations are row-major float32 [n_tokens][n_embd], i.e. ggml
 *    [n_embd, N] (diffuse-moe-graph.cpp:200).
 *  - One dmoe_ctx per host thread / stream: no internal locking
 *    (the reference serialises callers with a mutex,
 *    tools/diffuse-server.cpp:462).
 */
#ifndef DMOE_H
#define DMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, as enumerated in tools/quantize_streaming.py:109-110.
 * Q6_K is the type the reference's quantisers give output.weight (both Q4_K
 * schemes), the layer-0 ffn tensors (Q4_K_M) and every tensor of the q6_k
 * scheme (tools/quantize_streaming.py:113-124, tools/quantize.cpp:40-45). */
#define DMOE_TYPE_F32   0
#define DMOE_TYPE_F16   1
#define DMOE_TYPE_Q8_0  8
#define DMOE_TYPE_Q4_K 12
#define DMOE_TYPE_Q6_K 14

typedef enum dmoe_status {
    DMOE_OK                   = 0,
    DMOE_ERR_INVALID_ARG      = 1, /* null pointer, non-positive size        */
    DMOE_ERR_UNSUPPORTED_TYPE = 2, /* tensor type outside the list above     */
    DMOE_ERR_SHAPE            = 3, /* ne/nb inconsistent with the hparams    */
    DMOE_ERR_HIP              = 4, /* a HIP runtime call failed              */
    DMOE_ERR_OOM              = 5, /* device allocation failed               */
    DMOE_ERR_NONFINITE        = 6, /* NaN / Inf in the host input activations */
    DMOE_ERR_FORMAT           = 7, /* malformed GGUF file or key of the wrong type */
    DMOE_ERR_NOT_FOUND        = 8  /* GGUF file, key or tensor not present    */
} dmoe_status;

/* A view of one ggml tensor (ggml_tensor's type/data/ne/nb).  `data` points at
 * the unmodified GGUF block bytes. */
typedef struct dmoe_tensor {
    int32_t     type;
    const void *data;
    int64_t     ne[4];
    size_t      nb[4];
} dmoe_tensor;

/* MoE hyper-parameters: the diffuse_model fields of
 * src/diffuse-common.h:103-118, read from GGUF at src/diffuse-model.cpp:143-158. */
typedef struct dmoe_hparams {
    int32_t n_embd;          /* hparams.n_embd                                 */
    int32_t n_experts;       /* expert_count                                   */
    int32_t top_k;           /* expert_used_count                              */
    int32_t capacity;        /* expert_capacity   (default 48)                 */
    int32_t block_size;      /* moe_block_size    (default 32)                 */
    int32_t moe_ff;          /* expert_feed_forward_length                     */
    int32_t n_shared;        /* expert_shared_count (0: no shared expert)      */
    int32_t shared_ff;       /* ne[1] of moe_shared_gate                       */
    int32_t norm_topk_prob;  /* norm_topk_prob    (default 1)                  */
    float   routed_scaling;  /* routed_scaling_factor (2.5 for LLaDA2-flash)   */
} dmoe_hparams;

/* The MoE tensors of one layer (diffuse_moe_layer, src/diffuse-common.h:72-82):
 *   gate_w    moe_gate.weight          F32/F16 [n_embd, n_experts]
 *   gate_bias moe_gate_bias.weight     F32     [n_experts]      (data may be NULL)
 *   exp_gate  moe_experts_gate.weight  T       [n_embd, moe_ff, n_experts]
 *   exp_up    moe_experts_up.weight    T       [n_embd, moe_ff, n_experts]
 *   exp_down  moe_experts_down.weight  T       [moe_ff, n_embd, n_experts]
 *   sh_gate   moe_shared_gate.weight   Ts      [n_embd, shared_ff]
 *   sh_up     moe_shared_up.weight     Ts      [n_embd, shared_ff]
 *   sh_down   moe_shared_down.weight   Ts      [shared_ff, n_embd]
 * T, Ts in {F32, F16, Q8_0, Q4_K}; the three routed tensors share one T and the
 * three shared tensors share one Ts.  Shared tensors are ignored when
 * n_shared == 0. */
typedef struct dmoe_layer_desc {
    dmoe_tensor gate_w, gate_bias;
    dmoe_tensor exp_gate, exp_up, exp_down;
    dmoe_tensor sh_gate, sh_up, sh_down;
} dmoe_layer_desc;

/* Optional host-side copies of the routing intermediates (any field may be
 * NULL).  Sizes with N = n_tokens, E = n_experts, k = top_k, B = N/block_size:
 *   logits  [N][E] f32  router logits        (diffuse-moe-graph.cpp:203)
 *   probs   [N][E] f32  sigmoid(logits)      (:204)
 *   bmax    [B][E] f32  block max fold       (:223-229)   block routing only
 *   thr     [B]    f32  capacity threshold   (:232-236)   block routing only
 *   allowed [B][E] u8   1 = expert allowed   (:241-242)   block routing only
 *   idx     [N][k] i32  selected experts, descending selection score,
 *                       ties to the lower expert id     (:252)
 *   weights [N][k] f32  gate weights         (:253-262)
 *   counts  [E]    i32  (token, slot) pairs per expert
 *   offsets [E]    i32  exclusive prefix sum of counts
 *   perm    [N*k]  i32  pair ids t*k+slot grouped by expert: stable counting
 *                       sort of the t-major pair list (ggml_mul_mat_id order)
 *   use_block_routing   set to 1 when block routing ran (:215-216), else 0 */
typedef struct dmoe_debug {
    float   *logits;
    float   *probs;
    float   *bmax;
    float   *thr;
    uint8_t *allowed;
    int32_t *idx;
    float   *weights;
    int32_t *counts;
    int32_t *offsets;
    int32_t *perm;
    int32_t *use_block_routing;
} dmoe_debug;

typedef struct dmoe_ctx   dmoe_ctx;
typedef struct dmoe_layer dmoe_layer;

/* Create a context bound to HIP device `hip_device`.
 * Replaces the backend set-up of diffuse_context_new_gpu
 * (include/diffuse.h:65, src/diffuse-backend.h:76-101) for this segment. */
int  dmoe_create(int hip_device, dmoe_ctx **out);
void dmoe_destroy(dmoe_ctx *ctx);

/* Text of the last error on this context (never NULL). */
const char *dmoe_last_error(const dmoe_ctx *ctx);

/* Copy one layer's MoE tensors from host memory into HBM, once.  The caller
 * may free its host copy afterwards.  Replaces the (stubbed) weight offload of
 * src/diffuse-backend.h:104-121 for the MoE tensors of one layer. */
int  dmoe_layer_upload(dmoe_ctx *ctx, const dmoe_hparams *hp,
                       const dmoe_layer_desc *desc, dmoe_layer **out);

/* Same, but every `data` pointer in `desc` is already a device pointer on the
 * context's GPU.  Strides are taken from nb[].  Expert tensors whose type and
 * sizes fit the MFMA kernels (Q4_K: n_embd, moe_ff, shared_ff multiples of
 * 256 and of the kernels' row groups; F16: n_embd a multiple of 256, moe_ff
 * and shared_ff of 128) are rewritten once into a library-owned tiled copy in
 * HBM; every other tensor is referenced without copying (the caller keeps it
 * alive until dmoe_layer_free). */
int  dmoe_layer_wrap_device(dmoe_ctx *ctx, const dmoe_hparams *hp,
                            const dmoe_layer_desc *desc, dmoe_layer **out);

/* The dense SwiGLU MLP of the first_k_dense layers, y = W_down (silu(W_gate x)
 * * (W_up x)) (src/diffuse-moe-graph.cpp:181-187, the ffn_gate / ffn_up /
 * ffn_down tensors of diffuse_moe_layer, src/diffuse-common.h:67-70; loaded at
 * src/diffuse-model.cpp:183-185), with the weights' F32 semantics of
 * ensure_f32_moe (:8-12):
 *   gate, up  T [n_embd, n_ff]     down  T [n_ff, n_embd]     T in the list above
 * The result is a dmoe_layer run by dmoe_layer_forward / _forward_device /
 * _forward_device_noalloc (no routing: a dmoe_debug gets use_block_routing 0
 * and nothing else).  _upload copies host tensors into HBM; _wrap_device takes
 * device tensors (Q4_K, Q8_0 and F16 ones are rewritten into a library-owned
 * tiled copy, others referenced). */
int  dmoe_dense_upload(dmoe_ctx *ctx, int32_t n_embd, int32_t n_ff,
                       const dmoe_tensor *gate, const dmoe_tensor *up,
                       const dmoe_tensor *down, dmoe_layer **out);
int  dmoe_dense_wrap_device(dmoe_ctx *ctx, int32_t n_embd, int32_t n_ff,
                            const dmoe_tensor *gate, const dmoe_tensor *up,
                            const dmoe_tensor *down, dmoe_layer **out);

/* The step tail: the final norm and LM head (src/diffuse-moe-graph.cpp:
 * 295-300) and the temperature-0 sampling of every position
 * (sample_token, src/diffuse-sampler.cpp:29-49), without the logits leaving
 * the GPU:
 *   x = rms_norm(h, eps) * output_norm        output_norm F32 [n_embd] (F16 too for _upload)
 *   logits = output x                         output T [n_embd, n_vocab], F32 weight semantics
 *   tokens[t] = first index of the largest logit, probs[t] = 1 / sum exp(l - max)
 * (output_norm / output of diffuse_model, src/diffuse-common.h:95-96).  The
 * result is a dmoe_layer for dmoe_head_forward / _forward_device only. */
int  dmoe_head_upload(dmoe_ctx *ctx, int32_t n_embd, int32_t n_vocab,
                      const dmoe_tensor *output_norm, const dmoe_tensor *output,
                      dmoe_layer **out);
int  dmoe_head_wrap_device(dmoe_ctx *ctx, int32_t n_embd, int32_t n_vocab,
                           const dmoe_tensor *output_norm, const dmoe_tensor *output,
                           dmoe_layer **out);
/* h [n_tokens][n_embd] f32 (the residual stream after the last layer);
 * tokens, probs [n_tokens]; logits [n_tokens][n_vocab] may be NULL (the
 * reference copies all of them out, src/diffuse-moe-graph.cpp:331-332).
 * Host buffers, synchronous. */
int  dmoe_head_forward(dmoe_ctx *ctx, const dmoe_layer *head, const float *h,
                       int32_t n_tokens, float eps, int32_t *tokens, float *probs,
                       float *logits);
/* Device buffers, queued on `stream` without synchronising. */
int  dmoe_head_forward_device(dmoe_ctx *ctx, const dmoe_layer *head, const float *h_dev,
                              int32_t n_tokens, float eps, int32_t *tokens_dev,
                              float *probs_dev, float *logits_dev, void *stream);

/* ---- attention half of the layer (src/diffuse-moe-graph.cpp:116-178) ----
 * h_out = h + wo attn(rms_norm(h) * attn_norm) and moe_in =
 * rms_norm(h_out) * post_attn_norm (the MoE segment's input; no gain when
 * post_attn_norm.data is NULL):
 *   qkv = W_qkv x (fused [Q heads; K heads; V heads], :124-134), QK RMSNorm
 *   over head_dim times q_norm / k_norm (:141-146), partial NEOX RoPE of the
 *   first rotary_dim dims at position t (:154-155), flash attention with the
 *   block-causal mask of :19-55 (query i sees key j iff j / block_length <=
 *   i / block_length; every key when block_length <= 0), GQA query head h on
 *   kv head h / (n_head / n_head_kv), scale 1 / sqrt(head_dim) (:165-167),
 *   output projection and residual (:172-175), post-attention RMSNorm
 *   (:177-178).  Projection weights have F32 semantics (ensure_f32_moe).
 * Limits: n_embd and n_head * head_dim multiples of 256, head_dim 64 or 128,
 * rotary_dim even and <= head_dim, n_head a multiple of n_head_kv; other
 * shapes are refused with DMOE_ERR_SHAPE. */
typedef struct dmoe_attn_hparams {
    int32_t n_embd, n_head, n_head_kv, head_dim, rotary_dim;
    int32_t use_qk_norm;     /* model.use_qk_norm                           */
    int32_t block_length;    /* hparams.block_length (0: bidirectional)     */
    float   rope_base;       /* hparams.rope_theta (rope.freq_base)         */
    float   rms_eps;         /* hparams.rms_norm_eps                        */
} dmoe_attn_hparams;

/* diffuse_moe_layer's attention tensors (src/diffuse-common.h:60-65):
 *   attn_norm, post_attn_norm F32 [n_embd] (post_attn_norm data may be NULL)
 *   qkv  T [n_embd, (n_head + 2 n_head_kv) head_dim]
 *   q_norm, k_norm F32 [head_dim] (ignored unless use_qk_norm)
 *   wo   T [n_head head_dim, n_embd] */
typedef struct dmoe_attn_desc {
    dmoe_tensor attn_norm, qkv, q_norm, k_norm, wo, post_attn_norm;
} dmoe_attn_desc;

int  dmoe_attn_upload(dmoe_ctx *ctx, const dmoe_attn_hparams *ap, const dmoe_attn_desc *desc,
                      dmoe_layer **out);
int  dmoe_attn_wrap_device(dmoe_ctx *ctx, const dmoe_attn_hparams *ap,
                           const dmoe_attn_desc *desc, dmoe_layer **out);
/* h, h_out [n_tokens][n_embd] (h_out may be h); moe_in may be NULL.  Host
 * buffers, synchronous. */
int  dmoe_attn_forward(dmoe_ctx *ctx, const dmoe_layer *attn, const float *h, int32_t n_tokens,
                       float *h_out, float *moe_in);
/* Device buffers (16-byte aligned), queued on `stream` without synchronising. */
int  dmoe_attn_forward_device(dmoe_ctx *ctx, const dmoe_layer *attn, const float *h_dev,
                              int32_t n_tokens, float *h_out_dev, float *moe_in_dev,
                              void *stream);

/* Release a layer's device buffers.  The layer records its own device, so it
 * may be freed before or after the context that created it. */
void dmoe_layer_free(dmoe_layer *layer);

/* Which expert kernels a layer's forward runs, chosen at upload from the
 * weight types and shapes (a diagnostic without a counterpart in the
 * reference, whose expert products all run in ggml_mul_mat_id,
 * src/diffuse-moe-graph.cpp:266-269 and :282-285):
 *   DMOE_PATH_Q4K_MFMA  Q4_K routed + shared experts on int8 MFMA tiles
 *   DMOE_PATH_Q80_MFMA  Q8_0 routed + shared experts on int8 MFMA tiles
 *   DMOE_PATH_F16_GEMM  F16 experts on the f16 MFMA grouped GEMM
 *   DMOE_PATH_Q6K_MFMA  Q6_K dense MLP, step-tail LM head or attention
 *                       projections on int8 MFMA tiles (few-token kernel, in
 *                       chunks of 32 tokens)
 *   DMOE_PATH_GEMV      every other type / shape mix (F32 experts; Q6_K
 *                       routed or shared experts; widths
 *                       that are not whole MFMA work items; a shared expert
 *                       whose type or width differs from the routed ones)
 * Returns -1 for a NULL layer. */
#define DMOE_PATH_GEMV      0
#define DMOE_PATH_Q4K_MFMA  1
#define DMOE_PATH_Q80_MFMA  2
#define DMOE_PATH_F16_GEMM  3
#define DMOE_PATH_Q6K_MFMA  4
int  dmoe_layer_kernel_path(const dmoe_layer *layer);

/* moe_out = MoE(x) for host buffers x, y of n_tokens*n_embd floats.
 * Synchronous.  Replaces src/diffuse-moe-graph.cpp:188-289 (`cur` in,
 * `moe_out` out).  Host input containing NaN/Inf is rejected with
 * DMOE_ERR_NONFINITE.  `dbg` may be NULL. */
int  dmoe_layer_forward(dmoe_ctx *ctx, const dmoe_layer *layer,
                        const float *x, int32_t n_tokens, float *y,
                        dmoe_debug *dbg);

/* Device-pointer variant: x_dev, y_dev live on the context's GPU, work is
 * queued on `stream` (a hipStream_t; NULL = the null stream) and the call
 * returns without synchronising. */
int  dmoe_layer_forward_device(dmoe_ctx *ctx, const dmoe_layer *layer,
                               const float *x_dev, int32_t n_tokens,
                               float *y_dev, void *stream);

/* The device-pointer forward without any device allocation: no hipMalloc,
 * hipFree or allocating library call, and no profiling events.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it).  Its workspace is a fixed array of DMOE_NOALLOC_SCRATCH_BYTES in
 * device memory, one per GPU, held until the process ends; a forward whose
 * workspace would exceed it (the LLaDA2-flash Q4_K layer takes up to 314
 * tokens, nine whole 32-token blocks) is rejected with DMOE_ERR_INVALID_ARG
 * before anything is queued.  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams, other contexts, other threads) race, so the
 * caller serialises them.  Results are identical to
 * dmoe_layer_forward_device. */
#define DMOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int  dmoe_layer_forward_device_noalloc(dmoe_ctx *ctx, const dmoe_layer *layer,
                                       const float *x_dev, int32_t n_tokens,
                                       float *y_dev, void *stream);

/* Routing only, from caller-supplied router logits [N][E] (host).  Runs the
 * GPU router stages that follow the logits product (diffuse-moe-graph.cpp:
 * 204-262) plus the dispatch grouping; outputs go to `dbg` (logits is
 * ignored).  Lets routing be checked bit for bit on injected logits. */
int  dmoe_route_logits(dmoe_ctx *ctx, const dmoe_hparams *hp,
                       const float *bias /* [E] or NULL */,
                       const float *logits, int32_t n_tokens,
                       dmoe_debug *dbg);

/* Bytes of one row of n elements of `type` (ggml_row_size). */
size_t dmoe_row_size(int32_t type, int64_t n);

/* Quantise nrows rows of n_per_row f32 values (device memory) into `type`
 * blocks (device memory), on `stream`.  Counterpart of quantize_to_type in
 * tools/quant_lib.c:16-27 (which wraps ggml_quantize_chunk); used to build
 * synthetic GGUF expert tensors directly in HBM.  The Q4_K quantiser is a
 * plain min/max one, not ggml's iterative make_qkx2_quants. */
int  dmoe_quantize_device(dmoe_ctx *ctx, int32_t type, const float *src_dev,
                          void *dst_dev, int64_t nrows, int64_t n_per_row,
                          void *stream);

/* The residual stream around the segment, on device pointers: per row of
 * n_embd floats, h += y (skipped when y is NULL; the segment output added to
 * the residual, src/diffuse-moe-graph.cpp:292), then x = rms_norm(h, eps),
 * times gain[n_embd] when gain is not NULL (the next segment's input,
 * :175-178: ggml_rms_norm then ggml_mul by the norm weight).  h and x must
 * not overlap; n_embd % 4 == 0 and 16-byte aligned pointers.  Queued on
 * `stream` without synchronising. */
int  dmoe_residual_rmsnorm(dmoe_ctx *ctx, float *h_dev, const float *y_dev,
                           const float *gain_dev, float *x_dev, int32_t n_rows,
                           int32_t n_embd, float eps, void *stream);

/* ---- GGUF ingestion ------------------------------------------------------
 * A read-only memory map of a GGUF file (v2/v3, the container
 * tools/quantize_streaming.py:13-88 parses) with the MoE hyper-parameters and
 * tensors the reference's loader binds (src/diffuse-model.cpp:143-198).  The
 * dmoe_tensor views point into the mapping (host memory), so a layer goes to
 * HBM with dmoe_layer_upload / dmoe_dense_upload straight from the file; they
 * stay valid until dmoe_gguf_close.  Replaces gguf_init_from_file and the key
 * helpers of src/diffuse-model.cpp:5-73 for these tensors; where the
 * reference dies (DIFFUSE_DIE) on a missing key or tensor these return
 * DMOE_ERR_NOT_FOUND, on a malformed file DMOE_ERR_FORMAT. */
typedef struct dmoe_gguf dmoe_gguf;

/* Open and parse `path`; err (may be NULL) receives a message on failure. */
int  dmoe_gguf_open(const char *path, dmoe_gguf **out, char *err, size_t errlen);
void dmoe_gguf_close(dmoe_gguf *g);

/* Key lookup with the reference's prefix search: "diffuse.<suffix>", then
 * "qwen2.", "llama." (get_u32_multi / get_f32_multi, src/diffuse-model.cpp:
 * 21-45).  Integer keys of any integer type convert when the value fits. */
int  dmoe_gguf_get_u32(const dmoe_gguf *g, const char *suffix, uint32_t *val);
int  dmoe_gguf_get_f32(const dmoe_gguf *g, const char *suffix, float *val);

/* Any tensor by name (ggml_get_tensor): type, data, ne and ggml strides. */
int  dmoe_gguf_find_tensor(const dmoe_gguf *g, const char *name, dmoe_tensor *out);
int  dmoe_gguf_tensor_count(const dmoe_gguf *g);
const char *dmoe_gguf_tensor_name(const dmoe_gguf *g, int i);

/* The MoE hyper-parameters with the reference's defaults
 * (src/diffuse-model.cpp:143-158: capacity 48, moe_block_size = block_length
 * or 32, norm_topk_prob 1, routed_scaling 1.0); n_embd and n_layer
 * (embedding_length, block_count) are required; shared_ff is ne[1] of the
 * first moe_shared_gate tensor.  n_layer / first_k_dense may be NULL. */
int  dmoe_gguf_moe_hparams(const dmoe_gguf *g, dmoe_hparams *hp, int32_t *n_layer,
                           int32_t *first_k_dense);

/* The MoE tensors of layer il (blk.<il>.moe_gate, moe_gate_bias (optional),
 * moe_experts_gate/up/down, moe_shared_gate/up/down when expert_shared_count
 * > 0), src/diffuse-model.cpp:187-196. */
int  dmoe_gguf_layer_desc(const dmoe_gguf *g, int32_t il, dmoe_layer_desc *desc);

/* The dense MLP of layer il (blk.<il>.ffn_gate/up/down, :183-185); n_ff may
 * be NULL. */
int  dmoe_gguf_dense_desc(const dmoe_gguf *g, int32_t il, dmoe_tensor *gate,
                          dmoe_tensor *up, dmoe_tensor *down, int32_t *n_ff);

/* The attention hyper-parameters (src/diffuse-model.cpp:83-93, :148-150):
 * embedding_length, attention.head_count and attention.head_count_kv are
 * required; head_dim defaults to n_embd / n_head, rotary_dim to head_dim,
 * use_qk_norm and block_length to 0, rope.freq_base to 1e6,
 * attention.layer_norm_rms_epsilon to 1e-6. */
int  dmoe_gguf_attn_hparams(const dmoe_gguf *g, dmoe_attn_hparams *ap);

/* The attention tensors of layer il (blk.<il>.attn_norm, post_attn_norm,
 * attn_qkv, attn_output; attn_q_norm / attn_k_norm when use_qk_norm),
 * src/diffuse-model.cpp:171-179. */
int  dmoe_gguf_attn_desc(const dmoe_gguf *g, int32_t il, int32_t use_qk_norm,
                         dmoe_attn_desc *desc);

/* Per-stage timing.  While enabled, every forward records a HIP event pair
 * around each pipeline stage on the stream it runs on; dmoe_profile_read
 * waits for the recorded work, adds each stage's elapsed milliseconds and
 * launch count since the last read into total_ms[s] / calls[s]
 * (s < DMOE_N_STAGES; either array may be NULL) and resets the tally.
 * Replaces the per-forward wall-clock timers of the reference
 * (src/diffuse-sampler.cpp:171-176) at stage granularity. */
#define DMOE_N_STAGES 10
int  dmoe_profile_enable(dmoe_ctx *ctx, int enable);
int  dmoe_profile_read(dmoe_ctx *ctx, float *total_ms, int32_t *calls);
const char *dmoe_stage_name(int stage);

#ifdef __cplusplus
}
#endif

#endif /* DMOE_H */
