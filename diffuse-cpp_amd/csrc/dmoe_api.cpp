// dmoe_api.cpp — host side of the C ABI declared in include/dmoe.h.
//
// Owns the device copies of one layer's MoE tensors and a per-context
// workspace, validates shapes and types at the boundary, and queues the
// kernel pipeline that replaces src/diffuse-moe-graph.cpp:188-289:
//
//   router_logits -> route -> dispatch -> act_quant(x) -> gate/up (+SwiGLU)
//   -> act_quant(h) -> down -> [shared gate/up, shared down] -> combine
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <functional>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "dmoe_internal.h"

using namespace dmoe;

struct dmoe_ctx {
    int device = 0;
    KernelSwitches sw;              // kernel choices, read from the environment at creation
    hipStream_t stream = nullptr;
    // device address of this GPU's `scratch` array (the allocation-free forward)
    uint8_t *scratch = nullptr;
    std::string err;
    // workspace, grown on demand
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // per-stage timing
    bool prof = false;
    struct Mark { int stage; hipEvent_t a, b; };
    std::vector<Mark> marks;        // recorded since the last read
    std::vector<hipEvent_t> pool;   // free events
};

struct dmoe_layer {
    dmoe_ctx *ctx = nullptr;       // creating context (not used by dmoe_layer_free)
    int device = 0;                // HIP device holding the layer's buffers
    dmoe_hparams hp{};
    float *gate_w = nullptr;       // [E][H] f32
    float *gate_bias = nullptr;    // [E] or null
    int32_t bias_small = 1;        // no bias, or every bias finite with |bias| < 1e19
    WTensor eg{}, eu{}, ed{};
    WTensor sg{}, su{}, sd{};
    bool has_shared = false;
    // a dense SwiGLU MLP (first_k_dense layers): the three tensors sit in the
    // shared-expert slots (sg, su, sd), hp.n_embd / hp.shared_ff give its shape
    bool dense = false;
    // the step tail: final norm weight in gate_w (f32 [n_embd]), the output
    // (LM head) weight in sd as a shared down matrix of n_vocab rows
    bool head = false;
    int32_t n_vocab = 0;
    // the attention half of the layer: its projections as shared down
    // matrices (aqkv: (nh + 2 nkv) hd rows of n_embd; awo: n_embd rows of
    // nh hd), its norms f32
    bool attn = false;
    dmoe_attn_hparams ahp{};
    WTensor aqkv{}, awo{};
    float *attn_norm = nullptr, *post_norm = nullptr, *qn = nullptr, *kn = nullptr;
    std::vector<void *> owned;
};

// Workspace of dmoe_layer_forward_device_noalloc: a fixed array in device
// memory.  Every GPU the library runs on holds its own copy, at its own
// address, until the process ends.  In host code `scratch` is only a handle
// for hipGetSymbolAddress; kernels and copies take the per-device address.
static __device__ __align__(256) uint8_t scratch[DMOE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 256;
std::mutex g_scratch_mu;
uint8_t *g_scratch_addr[kMaxDevices];   // device address of `scratch`, per HIP device

// Resolves this GPU's address of `scratch` once per device; the device must
// be current.  Returns the hipGetSymbolAddress status.
hipError_t scratch_address(int device, uint8_t **out)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_addr[device] = (uint8_t *)p;
    }
    *out = g_scratch_addr[device];
    return hipSuccess;
}

int set_err(dmoe_ctx *ctx, int code, const char *fmt, ...)
{
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return code;
}

#define HIP_TRY(ctx, expr)                                                                         \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return set_err((ctx), e_ == hipErrorOutOfMemory ? DMOE_ERR_OOM : DMOE_ERR_HIP,         \
                           "%s failed: %s", #expr, hipGetErrorString(e_));                         \
    } while (0)

bool type_supported(int32_t t)
{
    return t == DMOE_TYPE_F32 || t == DMOE_TYPE_F16 || t == DMOE_TYPE_Q8_0 || t == DMOE_TYPE_Q4_K ||
           t == DMOE_TYPE_Q6_K;
}

// elements per block of the weight type (ggml_blck_size)
int64_t block_elems(int32_t t)
{
    switch (t) {
    case DMOE_TYPE_Q4_K: return 256;
    case DMOE_TYPE_Q6_K: return 256;
    case DMOE_TYPE_Q8_0: return 32;
    case DMOE_TYPE_F16: return 8;      // the kernels read 16-byte units
    case DMOE_TYPE_F32: return 4;
    default: return 0;
    }
}

size_t row_bytes(int32_t t, int64_t n)
{
    switch (t) {
    case DMOE_TYPE_F32: return (size_t)n * 4;
    case DMOE_TYPE_F16: return (size_t)n * 2;
    case DMOE_TYPE_Q8_0: return (n % 32) ? 0 : (size_t)(n / 32) * Q8_0_BYTES;
    case DMOE_TYPE_Q4_K: return (n % 256) ? 0 : (size_t)(n / 256) * Q4K_BYTES;
    case DMOE_TYPE_Q6_K: return (n % 256) ? 0 : (size_t)(n / 256) * Q6K_BYTES;
    default: return 0;
    }
}

// activation type of the routed products (ggml vec_dot_type)
int32_t act_type_of(int32_t wt)
{
    return wt == DMOE_TYPE_Q4_K || wt == DMOE_TYPE_Q6_K ? DMOE_ACT_Q8_K : wt;
}

size_t act_row_vals_bytes(int32_t at, int64_t n)
{
    switch (at) {
    case DMOE_TYPE_F32: return (size_t)n * 4;
    case DMOE_TYPE_F16: return (size_t)n * 2;
    default: return (size_t)n;       // int8 values
    }
}

// Check one weight tensor view against the expected ne; rows contiguous.
int check_tensor(dmoe_ctx *ctx, const char *name, const dmoe_tensor &t, int64_t ne0, int64_t ne1,
                 int64_t ne2, bool device_mode)
{
    if (!t.data) return set_err(ctx, DMOE_ERR_INVALID_ARG, "%s: data is NULL", name);
    if (!type_supported(t.type))
        return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "%s: unsupported ggml type %d", name, t.type);
    if (t.ne[0] != ne0 || t.ne[1] != ne1 || (ne2 > 0 && t.ne[2] != ne2) ||
        (ne2 <= 0 && t.ne[2] > 1) || t.ne[3] > 1)
        return set_err(ctx, DMOE_ERR_SHAPE,
                       "%s: ne = [%lld,%lld,%lld,%lld], expected [%lld,%lld,%lld]", name,
                       (long long)t.ne[0], (long long)t.ne[1], (long long)t.ne[2],
                       (long long)t.ne[3], (long long)ne0, (long long)ne1, (long long)ne2);
    if (ne0 % block_elems(t.type))
        return set_err(ctx, DMOE_ERR_SHAPE, "%s: ne0 = %lld is not a multiple of %lld", name,
                       (long long)ne0, (long long)block_elems(t.type));
    const size_t rb = row_bytes(t.type, ne0);
    if (t.nb[1] < rb) return set_err(ctx, DMOE_ERR_SHAPE, "%s: nb[1] below the row size", name);
    if (ne2 > 0 && t.nb[2] < t.nb[1] * (size_t)ne1)
        return set_err(ctx, DMOE_ERR_SHAPE, "%s: nb[2] below nb[1]*ne[1]", name);
    if (device_mode) {
        // the kernels load 16-byte units (2-byte for Q8_0 and Q6_K blocks,
        // 34 and 210 bytes long)
        const size_t al = t.type == DMOE_TYPE_Q8_0 || t.type == DMOE_TYPE_Q6_K ? 2 : 16;
        if ((uintptr_t)t.data % al || t.nb[1] % al || (ne2 > 0 && t.nb[2] % al))
            return set_err(ctx, DMOE_ERR_SHAPE, "%s: device data/strides not %zu-byte aligned",
                           name, al);
    }
    return DMOE_OK;
}

int validate(dmoe_ctx *ctx, const dmoe_hparams *hp, const dmoe_layer_desc *d, bool device_mode)
{
    if (!hp || !d) return set_err(ctx, DMOE_ERR_INVALID_ARG, "hparams / desc is NULL");
    const int H = hp->n_embd, E = hp->n_experts, K = hp->top_k, FF = hp->moe_ff;
    if (H <= 0 || H % 256)
        return set_err(ctx, DMOE_ERR_SHAPE, "n_embd = %d must be a positive multiple of 256", H);
    if (E <= 0 || E > 1024) return set_err(ctx, DMOE_ERR_SHAPE, "n_experts = %d outside 1..1024", E);
    if (K <= 0 || K > 32 || K > E)
        return set_err(ctx, DMOE_ERR_SHAPE, "top_k = %d outside 1..min(32, n_experts)", K);
    if (FF <= 0) return set_err(ctx, DMOE_ERR_SHAPE, "moe_ff = %d", FF);
    if (hp->block_size < 0 || hp->capacity < 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "negative block_size / capacity");
    if (hp->block_size > 1 && hp->capacity > 0 && hp->capacity < E && hp->block_size > 4096)
        return set_err(ctx, DMOE_ERR_SHAPE, "block_size = %d above 4096", hp->block_size);

    const dmoe_tensor &gw = d->gate_w;
    if (!gw.data) return set_err(ctx, DMOE_ERR_INVALID_ARG, "gate_w: data is NULL");
    if (gw.type != DMOE_TYPE_F32 && !(gw.type == DMOE_TYPE_F16 && !device_mode))
        return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "gate_w: type %d (F32%s expected)", gw.type,
                       device_mode ? "" : " or F16");
    if (gw.ne[0] != H || gw.ne[1] != E)
        return set_err(ctx, DMOE_ERR_SHAPE, "gate_w: ne = [%lld,%lld], expected [%d,%d]",
                       (long long)gw.ne[0], (long long)gw.ne[1], H, E);
    if (gw.nb[1] < row_bytes(gw.type, H))
        return set_err(ctx, DMOE_ERR_SHAPE, "gate_w: nb[1] below the row size");
    if (device_mode && ((uintptr_t)gw.data % 16 || gw.nb[1] != (size_t)H * 4))
        return set_err(ctx, DMOE_ERR_SHAPE, "gate_w: device router must be contiguous, 16-byte aligned");
    if (d->gate_bias.data) {
        if (d->gate_bias.type != DMOE_TYPE_F32)
            return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "gate_bias: type %d (F32 expected)",
                           d->gate_bias.type);
        if (d->gate_bias.ne[0] != E)
            return set_err(ctx, DMOE_ERR_SHAPE, "gate_bias: ne0 = %lld, expected %d",
                           (long long)d->gate_bias.ne[0], E);
    }
    int rc;
    if ((rc = check_tensor(ctx, "exp_gate", d->exp_gate, H, FF, E, device_mode))) return rc;
    if ((rc = check_tensor(ctx, "exp_up", d->exp_up, H, FF, E, device_mode))) return rc;
    if ((rc = check_tensor(ctx, "exp_down", d->exp_down, FF, H, E, device_mode))) return rc;
    if (d->exp_up.type != d->exp_gate.type || d->exp_down.type != d->exp_gate.type)
        return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "routed expert tensors differ in type");
    if (hp->n_shared > 0 && d->sh_gate.data) {
        const int SF = hp->shared_ff;
        if (SF <= 0) return set_err(ctx, DMOE_ERR_SHAPE, "shared_ff = %d", SF);
        if ((rc = check_tensor(ctx, "sh_gate", d->sh_gate, H, SF, 0, device_mode))) return rc;
        if ((rc = check_tensor(ctx, "sh_up", d->sh_up, H, SF, 0, device_mode))) return rc;
        if ((rc = check_tensor(ctx, "sh_down", d->sh_down, SF, H, 0, device_mode))) return rc;
        if (d->sh_up.type != d->sh_gate.type || d->sh_down.type != d->sh_gate.type)
            return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "shared expert tensors differ in type");
    }
    return DMOE_OK;
}

float f16_to_f32_host(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;
        memcpy(&u, &v, 4);
        u |= sign;
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// Copy one (possibly strided) host tensor into a compact device buffer.
int upload_tensor(dmoe_ctx *ctx, dmoe_layer *L, const dmoe_tensor &t, int64_t nrows,
                  int64_t nmats, WTensor &out)
{
    const size_t rb = row_bytes(t.type, t.ne[0]);
    const size_t bytes = rb * (size_t)nrows * (size_t)nmats;
    void *dev = nullptr;
    HIP_TRY(ctx, hipMalloc(&dev, bytes));
    L->owned.push_back(dev);
    const uint8_t *src = (const uint8_t *)t.data;
    if (t.nb[1] == rb && (nmats == 1 || t.nb[2] == rb * (size_t)nrows)) {
        HIP_TRY(ctx, hipMemcpy(dev, src, bytes, hipMemcpyHostToDevice));
    } else {
        HIP_TRY(ctx, hipMemcpy2D(dev, rb, src, t.nb[1], rb, (size_t)nrows, hipMemcpyHostToDevice));
        for (int64_t m = 1; m < nmats; m++)
            HIP_TRY(ctx, hipMemcpy2D((uint8_t *)dev + (size_t)m * rb * nrows, rb,
                                     src + (size_t)m * t.nb[2], t.nb[1], rb, (size_t)nrows,
                                     hipMemcpyHostToDevice));
    }
    out.type = t.type;
    out.data = (const uint8_t *)dev;
    out.nb1 = rb;
    out.nb2 = rb * (size_t)nrows;
    return DMOE_OK;
}

WTensor wrap_tensor(const dmoe_tensor &t)
{
    WTensor w;
    w.type = t.type;
    w.data = (const uint8_t *)t.data;
    w.nb1 = t.nb[1];
    w.nb2 = t.nb[2];
    return w;
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace carve-up for one forward of N tokens.
struct Workspace {
    float *x, *y;
    RouteBufs rb;
    WorkList wl;
    ActBuf xq, hq;                       // GEMV-path activations
    ActI8 ax, axs, ah, ahs;              // MFMA-path activations (routed / shared)
    uint16_t *x16, *xs16, *h16, *hs16;   // GEMM-path f16 activations (split: hi / lo rows)
    float *h, *ye, *hs, *ys;
    float *bias;
};

// The MFMA expert path covers Q4_K routed experts (and a Q4_K shared expert)
// with reduction lengths that are whole super-blocks.
bool use_mfma_path(const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared)
{
    // whole super-blocks along K, whole work items along the output rows
    const int gu = expert_rows_per_item(0), dn = expert_rows_per_item(1);
    if (wtype != DMOE_TYPE_Q4_K || hp.n_embd % 256 || hp.moe_ff % 256) return false;
    if (hp.moe_ff % gu || hp.n_embd % dn) return false;
    // the shared expert's down product runs in the routed one's launch plan
    if (shared && (stype != DMOE_TYPE_Q4_K || hp.shared_ff != hp.moe_ff)) return false;
    // an item's activation rows are held whole in LDS
    if (!expert_k_ok(hp.n_embd) || !expert_k_ok(hp.moe_ff)) return false;
    return true;
}

// Activation column blocks of 16 pairs per routed Q4_K work item, by the
// tokens per expert the forward brings: pairs per expert averaged over all
// experts (N k / E) of 64 or more take 4 blocks, of 32 or more 2, else 1.  A
// weight tile read from HBM then serves up to 64 pairs instead of 16 (the
// prefill-sized windows); few tokens per expert keep the 16-pair items, whose
// finer work division fills the chip.  DMOE_Q4K_COLUMN_BLOCKS (1, 2, 4)
// overrides the choice.
int q4k_column_blocks(const KernelSwitches &sw, const dmoe_hparams &hp, int N)
{
    if (sw.q4k_column_blocks) return sw.q4k_column_blocks;
    const long avg = (long)N * hp.top_k / (hp.n_experts > 0 ? hp.n_experts : 1);
    return avg >= 64 ? 4 : avg >= 32 ? 2 : 1;
}

bool use_q80_path(const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared);
bool use_gemm_path(const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared);

// The tile kernels of k_expert_tile.hip (units of up to 32 pairs of an expert,
// 16 for F16, whose activations stay in LDS for the whole reduction; h
// through HBM as f32 and one conversion), by the forward's pairs per expert
// averaged over all experts (N k / E): Q8_0 at every N (at one 32-token
// block of the flash layer 146 against 160 us for the item kernels); Q4_K
// from 8 on (the flash layer from 256 tokens; fewer take the few-token
// kernels: 91 against 110 us at 32 tokens); F16 below 8 (more take the
// grouped GEMM of 256-pair items).  DMOE_EXPERT_TILE = 0 / 1 turns the
// choice off / on for every N (with the shapes the tile kernels take).
// The Q4_K grouped GEMM of k_expert_gemm.hip (units of up to 128 pairs, each
// step's weight tiles applied to all of a unit's pairs): by the forward's
// pairs per expert averaged over all experts, N k / E of at least
// GEMM_Q4K_MIN_AVG.  DMOE_EXPERT_GEMM = 0 / 1 turns it off / on for every N;
// DMOE_EXPERT_TILE or DMOE_Q4K_COLUMN_BLOCKS set selects their kernels.
constexpr long GEMM_Q4K_MIN_AVG = 64;

bool use_q4k_gemm(const KernelSwitches &sw, const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared,
                  int N)
{
    if (!use_mfma_path(hp, wtype, stype, shared) || !expert_gemm_q4k_ok(hp.n_embd, hp.moe_ff, hp.shared_ff, shared))
        return false;
    // 32-bit byte offsets into the activation arrays
    if ((long)N * hp.top_k * hp.moe_ff >= (1L << 31) || 2L * N * hp.n_embd >= (1L << 31)) return false;
    if (sw.expert_gemm >= 0) return sw.expert_gemm == 1;
    if (sw.expert_tile >= 0 || sw.q4k_column_blocks) return false;
    const long avg = (long)N * hp.top_k / (hp.n_experts > 0 ? hp.n_experts : 1);
    return avg >= GEMM_Q4K_MIN_AVG;
}

bool use_tile_path(const KernelSwitches &sw, const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared,
                   int N)
{
    if (use_q4k_gemm(sw, hp, wtype, stype, shared, N)) return false;
    const bool f16 = use_gemm_path(hp, wtype, stype, shared);
    if (!(use_mfma_path(hp, wtype, stype, shared) || use_q80_path(hp, wtype, stype, shared) || f16) ||
        !expert_tile_ok(hp.n_embd, hp.moe_ff, hp.shared_ff, shared))
        return false;
    if (sw.expert_tile >= 0) return sw.expert_tile == 1;
    if (sw.q4k_column_blocks && wtype == DMOE_TYPE_Q4_K) return false;
    if (wtype == DMOE_TYPE_Q8_0) return true;
    const long avg = (long)N * hp.top_k / (hp.n_experts > 0 ? hp.n_experts : 1);
    return f16 ? avg < 8 : avg >= 8;
}

// Few tokens of Q4_K experts: the down products and the combine run as one
// launch over 16-row tiles of every expert (k_down_rows.hip); it takes the
// 16-pair work list.
bool use_down_rows(const KernelSwitches &sw, const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared,
                   int N)
{
    return use_mfma_path(hp, wtype, stype, shared) && !use_tile_path(sw, hp, wtype, stype, shared, N) &&
           !use_q4k_gemm(sw, hp, wtype, stype, shared, N) &&
           down_rows_ok(N, hp.top_k, hp.n_experts, hp.n_embd, hp.moe_ff) && q4k_column_blocks(sw, hp, N) == 1;
}

// Of those, the shapes whose down products run by spans of (unit, tile) work
// (k_down_span.hip) with the combine launch after them: every activation row
// is read once per workgroup instead of once per 16 output rows (26.8 + 4.1
// against 36.0 us at the flash shape, 32 tokens; at 256 tokens the item
// kernel is faster, 98.6 against 107.2 us).  DMOE_DOWN_FUSED=1 selects the
// single fused launch (k_down_rows.hip) instead: the same bits.
bool use_down_span(const KernelSwitches &sw, const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared,
                   int N)
{
    if (sw.down_fused) return false;
    return use_down_rows(sw, hp, wtype, stype, shared, N) &&
           down_span_ok(N, hp.top_k, hp.n_experts, hp.n_embd, hp.moe_ff, shared);
}

// Q8_0 experts (and a Q8_0 shared expert of the same width) run on the int8
// MFMA kernels of k_expert_q80.hip.
bool use_q80_path(const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared)
{
    const int gu = expert_q80_rows_per_item(0), dn = expert_q80_rows_per_item(1);
    if (wtype != DMOE_TYPE_Q8_0 || hp.n_embd % 256 || hp.moe_ff % 256) return false;
    if (hp.moe_ff % gu || hp.n_embd % dn) return false;
    if (shared && (stype != DMOE_TYPE_Q8_0 || hp.shared_ff != hp.moe_ff)) return false;
    return true;
}

// F16 experts (and an F16 shared expert) run on the MFMA grouped-GEMM path.
bool use_gemm_path(const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared)
{
    if (wtype != DMOE_TYPE_F16 || (shared && stype != DMOE_TYPE_F16)) return false;
    return gemm_shapes_ok(hp.n_embd, hp.moe_ff, shared ? hp.shared_ff : 0, shared);
}

ActI8 take_act(const std::function<uint8_t *(size_t)> &take, int rows, int K, bool split,
               bool per32 = false)
{
    // split activations keep their a0 digit rows as rows rows..2*rows-1;
    // per32: one scale per 32 values and no sums (the Q8_0 kernels)
    const int r = split ? 2 * rows : rows;
    ActI8 a{};
    a.K = K;
    a.q = (int8_t *)take((size_t)r * K);
    a.bs = per32 ? nullptr : (uint16_t *)take((size_t)r * (K / 16) * 2);
    a.d = (float *)take((size_t)r * (K / (per32 ? 32 : 256)) * 4);
    return a;
}

// host_io: room for x and y (the host-buffer forward copies them through HBM).
// Buffers only one kernel family reads are planned only for that family.
size_t plan_workspace(const KernelSwitches &sw, const dmoe_hparams &hp, int32_t wtype, int32_t stype, bool shared, int N,
                      bool host_io, uint8_t *base, Workspace *w)
{
    const int H = hp.n_embd, E = hp.n_experts, K = hp.top_k, FF = hp.moe_ff;
    const int SF = shared ? hp.shared_ff : 0;
    const int P = N * K;
    const int B = hp.block_size > 0 ? (N + hp.block_size - 1) / hp.block_size : 1;
    // routing groups: block_size tokens with block routing, else 32
    const int gmin = hp.block_size > 1 ? std::min(hp.block_size, 32) : 32;
    const int groups = (N + gmin - 1) / gmin;
    const int32_t at = act_type_of(wtype);
    size_t off = 0;
    std::function<uint8_t *(size_t)> take = [&](size_t bytes) -> uint8_t * {
        uint8_t *p = base ? base + off : nullptr;
        off += align_up(bytes > 0 ? bytes : 1);
        return p;
    };
    Workspace t{};
    if (host_io) {
        t.x = (float *)take((size_t)N * H * 4);
        t.y = (float *)take((size_t)N * H * 4);
    }
    t.bias = (float *)take((size_t)E * 4);
    t.rb.logits = (float *)take((size_t)N * E * 4);
    t.rb.probs = (float *)take((size_t)N * E * 4);
    t.rb.sel = (float *)take((size_t)N * E * 4);
    t.rb.bmax = (float *)take((size_t)B * E * 4);
    t.rb.thr = (float *)take((size_t)B * 4);
    t.rb.allowed = (uint8_t *)take((size_t)B * E);
    t.rb.idx = (int32_t *)take((size_t)P * 4);
    t.rb.weights = (float *)take((size_t)P * 4);
    t.rb.counts = (int32_t *)take((size_t)E * 4);
    t.rb.offsets = (int32_t *)take((size_t)(E + 1) * 4);
    t.rb.perm = (int32_t *)take((size_t)P * 4);
    t.rb.hist = (int32_t *)take((size_t)groups * E * 4);
    t.rb.lrank = (int32_t *)take((size_t)P * 4);
    const bool gemm = use_gemm_path(hp, wtype, stype, shared);
    const bool gemv = !gemm && !use_mfma_path(hp, wtype, stype, shared) &&
                      !use_q80_path(hp, wtype, stype, shared);
    const bool tile = use_tile_path(sw, hp, wtype, stype, shared, N);
    t.wl.chunk = use_q4k_gemm(sw, hp, wtype, stype, shared, N) ? EXPERT_GEMM_CHUNK
                 : tile                                         ? expert_tile_chunk(wtype)
                 : gemm ? GM
                        : EXPERT_CHUNK * (use_mfma_path(hp, wtype, stype, shared) ? q4k_column_blocks(sw, hp, N) : 1);
    t.wl.n_ec = (int32_t *)take(4);
    t.wl.ec_expert = (int32_t *)take((size_t)(E + P / EXPERT_CHUNK + 1) * 4);
    t.wl.ec_chunk = (int32_t *)take((size_t)(E + P / EXPERT_CHUNK + 1) * 4);

    if (use_mfma_path(hp, wtype, stype, shared)) {
        t.ax = take_act(take, N, H, false);
        t.ah = take_act(take, P, FF, false);
        if (shared) {
            t.axs = take_act(take, N, H, true);
            t.ahs = take_act(take, N, SF, true);
        }
        if (tile || use_q4k_gemm(sw, hp, wtype, stype, shared, N)) {
            // the tile kernels' and the grouped GEMM's f32 h, converted by one launch
            t.h = (float *)take((size_t)P * FF * 4);
            if (shared) t.hs = (float *)take((size_t)N * SF * 4);
        }
    }
    if (use_q80_path(hp, wtype, stype, shared)) {
        t.ax = take_act(take, N, H, false, true);
        t.ah = take_act(take, P, FF, false, true);
        if (shared) {
            t.axs = take_act(take, N, H, true, true);
            t.ahs = take_act(take, N, SF, true, true);
        }
        if (tile) {
            t.h = (float *)take((size_t)P * FF * 4);
            if (shared) t.hs = (float *)take((size_t)N * SF * 4);
        }
    }
    if (gemm) {
        // with a shared expert, the hi rows of its split x (f16(x)) are the
        // routed experts' f16 x as well: no separate copy
        if (shared) {
            t.xs16 = (uint16_t *)take((size_t)2 * N * H * 2);
            t.hs16 = (uint16_t *)take((size_t)2 * N * SF * 2);
            t.x16 = t.xs16;
        } else {
            t.x16 = (uint16_t *)take((size_t)N * H * 2);
        }
        t.h16 = (uint16_t *)take((size_t)P * FF * 2);
        if (tile) {
            t.h = (float *)take((size_t)P * FF * 4);
            if (shared) t.hs = (float *)take((size_t)N * SF * 4);
        }
    }
    if (gemv) {
        // activations of the GEMV kernels (k_gemv.hip) and their f32 h
        t.xq.type = at;
        t.xq.n = H;
        t.xq.vals = take((size_t)N * act_row_vals_bytes(at, H));
        t.xq.d = (float *)take((size_t)N * (H / 32) * 4);
        t.xq.bsums = (int16_t *)take((size_t)N * (H / 16) * 2);
        t.h = (float *)take((size_t)P * FF * 4);
        t.hq.type = at;
        t.hq.n = FF;
        t.hq.vals = take((size_t)P * act_row_vals_bytes(at, FF));
        t.hq.d = (float *)take((size_t)P * (FF / 32 + 1) * 4);
        t.hq.bsums = (int16_t *)take((size_t)P * (FF / 16 + 1) * 2);
        t.hs = (float *)take((size_t)N * (SF > 0 ? SF : 1) * 4);
    }
    if (!use_down_rows(sw, hp, wtype, stype, shared, N) || use_down_span(sw, hp, wtype, stype, shared, N)) {
        // per-pair and shared down results, folded by the combine launch
        t.ye = (float *)take((size_t)P * H * 4);
        t.ys = (float *)take((size_t)N * H * 4);
    }
    if (w) *w = t;
    return off;
}

int ensure_workspace(dmoe_ctx *ctx, const dmoe_layer *L, int N, bool host_io, Workspace *w)
{
    const size_t need =
        plan_workspace(ctx->sw, L->hp, L->eg.type, L->sg.type, L->has_shared, N, host_io, nullptr, nullptr);
    if (need > ctx->ws_bytes) {
        if (ctx->ws) {
            // work queued on any stream may still read the old workspace
            HIP_TRY(ctx, hipDeviceSynchronize());
            HIP_TRY(ctx, hipFree(ctx->ws));
            ctx->ws = nullptr;
            ctx->ws_bytes = 0;
        }
        if (getenv("DMOE_FAIL_ALLOC"))
            return set_err(ctx, DMOE_ERR_OOM, "workspace allocation of %zu bytes refused (DMOE_FAIL_ALLOC)", need);
        HIP_TRY(ctx, hipMalloc(&ctx->ws, need));
        ctx->ws_bytes = need;
    }
    plan_workspace(ctx->sw, L->hp, L->eg.type, L->sg.type, L->has_shared, N, host_io, (uint8_t *)ctx->ws, w);
    return DMOE_OK;
}

RouteParams route_params(const dmoe_layer *L, const dmoe_hparams &hp, int N)
{
    RouteParams rp{};
    rp.bias = L ? L->gate_bias : nullptr;
    rp.bias_small = L ? L->bias_small : 0;
    rp.n_tokens = N;
    rp.n_experts = hp.n_experts;
    rp.top_k = hp.top_k;
    rp.capacity = hp.capacity;
    rp.block_size = hp.block_size;
    // src/diffuse-moe-graph.cpp:215-216
    rp.use_block = hp.block_size > 1 && hp.capacity > 0 && hp.capacity < hp.n_experts &&
                   N % hp.block_size == 0;
    rp.norm_topk_prob = hp.norm_topk_prob;
    rp.routed_scaling = hp.routed_scaling;
    return rp;
}

const char *const kStageNames[DMOE_N_STAGES] = {
    "front", "route", "scores", "act_quant_x", "gateup_routed",
    "act_quant_h", "down_routed", "gateup_shared", "down_shared", "combine"};

enum { ST_FRONT, ST_ROUTE, ST_SCORES, ST_ACTQ_X, ST_GATEUP, ST_ACTQ_H, ST_DOWN, ST_SH_GATEUP,
       ST_SH_DOWN, ST_COMBINE };

hipEvent_t take_event(dmoe_ctx *ctx)
{
    if (!ctx->pool.empty()) {
        hipEvent_t e = ctx->pool.back();
        ctx->pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Runs one stage; with profiling on, brackets it with an event pair.
template <class F>
hipError_t stage(dmoe_ctx *ctx, bool prof, int id, hipStream_t s, F &&launch)
{
    if (!prof) return launch();
    hipEvent_t a = take_event(ctx), b = take_event(ctx);
    if (!a || !b) return hipErrorOutOfMemory;
    hipError_t e = hipEventRecord(a, s);
    if (e == hipSuccess) e = launch();
    if (e == hipSuccess) e = hipEventRecord(b, s);
    ctx->marks.push_back({id, a, b});
    return e;
}

#define LAUNCH_TRY(ctx, expr)                                                                      \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return set_err((ctx), DMOE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));           \
    } while (0)

// prof: bracket the stages with timing events (which may create events; the
// allocation-free forward passes false).
int enqueue_forward(dmoe_ctx *ctx, const dmoe_layer *L, const Workspace &w, const float *x,
                    int N, float *y, hipStream_t s, bool prof)
{
    const dmoe_hparams &hp = L->hp;
    const int H = hp.n_embd, E = hp.n_experts, K = hp.top_k, FF = hp.moe_ff;
    const RouteParams rp = route_params(L, hp, N);
    const bool q4 = use_mfma_path(hp, L->eg.type, L->sg.type, L->has_shared);
    const bool q8 = use_q80_path(hp, L->eg.type, L->sg.type, L->has_shared);
    const bool mfma = q4 || q8;
    const bool gemm = use_gemm_path(hp, L->eg.type, L->sg.type, L->has_shared);
    // activation layouts of the int8 MFMA kernels (routed, shared expert)
    const int mode_r = q8 ? ACT_Q80 : ACT_Q8K, mode_s = q8 ? ACT_SPLIT32 : ACT_SPLIT;
    const int nc = q4 ? q4k_column_blocks(ctx->sw, hp, N) : 1;
    auto expert = [&](int phase, const MoeJob &j) {
        return q8 ? launch_expert_q80(phase, j, s) : launch_expert_q4k(phase, j, s, nc, ctx->sw.gateup_lds);
    };
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    // router logits, sigmoid, selection scores (+ x in the MFMA operand layout)
    PrepJob xj[2];
    int nxj = 0;
    if (mfma) {
        xj[nxj++] = PrepJob{x, N, H, mode_r, w.ax};
        if (L->has_shared) xj[nxj++] = PrepJob{x, N, H, mode_s, w.axs};
    }
    // With one routing group the conversions run in the route launch, on the
    // compute units its one routing workgroup leaves idle, rather than in
    // the front, whose workgroups would run them before their logit products
    const bool conv_route = nxj > 0 && route_single(rp);
    STAGE(ST_FRONT, launch_front(L->gate_w, L->gate_bias, x, N, H, E, w.rb, xj, conv_route ? 0 : nxj, s));
    // block routing, top-k, gate weights and the dispatch
    STAGE(ST_ROUTE, launch_route(rp, w.rb, w.wl, s, xj, conv_route ? nxj : 0));
    if (mfma) {
        // Q4_K / Q8_0 experts on int8 MFMA: routed experts and the shared one
        // share a launch
        MoeJob job{};
        job.eg = L->eg;
        job.eu = L->eu;
        job.ed = L->ed;
        job.sg = L->sg;
        job.su = L->su;
        job.sd = L->sd;
        job.has_shared = L->has_shared;
        job.H = H;
        job.FF = FF;
        job.SF = hp.shared_ff;
        job.n_tokens = N;
        job.top_k = K;
        job.perm = w.rb.perm;
        job.offsets = w.rb.offsets;
        job.counts = w.rb.counts;
        job.E = E;
        job.ec_cap = E + N * K / EXPERT_CHUNK + 1;
        job.wl = w.wl;
        job.ax = w.ax;
        job.axs = w.axs;
        job.h = w.h;
        job.hs = w.hs;
        job.ah = w.ah;
        job.ahs = w.ahs;
        job.ye = w.ye;
        job.ys = w.ys;
        const bool xgemm = use_q4k_gemm(ctx->sw, hp, L->eg.type, L->sg.type, L->has_shared, N);
        if (xgemm || use_tile_path(ctx->sw, hp, L->eg.type, L->sg.type, L->has_shared, N)) {
            // many tokens per expert: the grouped GEMM or the tile kernels, h
            // converted between the two launches
            STAGE(ST_GATEUP, xgemm ? launch_expert_gemm_q4k(0, job, s) : launch_expert_tile(0, job, s));
            PrepJob hj[2];
            int nhj = 0;
            hj[nhj++] = PrepJob{w.h, N * K, FF, q8 ? ACT_Q80 : ACT_Q8K, w.ah};
            if (L->has_shared) hj[nhj++] = PrepJob{w.hs, N, hp.shared_ff, q8 ? ACT_SPLIT32 : ACT_SPLIT, w.ahs};
            STAGE(ST_ACTQ_H, launch_prep(hj, nhj, s));
            STAGE(ST_DOWN, xgemm ? launch_expert_gemm_q4k(1, job, s) : launch_expert_tile(1, job, s));
            STAGE(ST_COMBINE, launch_combine(w.ye, w.rb.weights, L->has_shared ? w.ys : nullptr, N,
                                             K, H, y, s));
            return DMOE_OK;
        }
        // the gate/up launch converts h to the down products' layout itself
        STAGE(ST_GATEUP, expert(0, job));
        const bool span = use_down_span(ctx->sw, hp, L->eg.type, L->sg.type, L->has_shared, N);
        if (span || use_down_rows(ctx->sw, hp, L->eg.type, L->sg.type, L->has_shared, N)) {
            // down products and the combine in one launch
            DownRowsJob dj{};
            dj.ed = L->ed;
            dj.sd = L->sd;
            dj.has_shared = L->has_shared;
            dj.N = N;
            dj.K = K;
            dj.E = E;
            dj.H = H;
            dj.FF = FF;
            dj.perm = w.rb.perm;
            dj.offsets = w.rb.offsets;
            dj.counts = w.rb.counts;
            dj.wl = w.wl;
            dj.ec_cap = E + N * K / EXPERT_CHUNK + 1;
            dj.ah = w.ah;
            dj.ahs = w.ahs;
            dj.weights = w.rb.weights;
            dj.y = y;
            if (span) {
                dj.ye = w.ye;
                dj.ys = w.ys;
                STAGE(ST_DOWN, launch_down_span(dj, s));
                STAGE(ST_COMBINE, launch_combine(w.ye, w.rb.weights, L->has_shared ? w.ys : nullptr, N,
                                                 K, H, y, s));
                return DMOE_OK;
            }
            STAGE(ST_DOWN, launch_down_rows(dj, s));
            return DMOE_OK;
        }
        STAGE(ST_DOWN, expert(1, job));
        STAGE(ST_COMBINE, launch_combine(w.ye, w.rb.weights, L->has_shared ? w.ys : nullptr, N,
                                         K, H, y, s));
        return DMOE_OK;
    }
    if (gemm && use_tile_path(ctx->sw, hp, L->eg.type, L->sg.type, L->has_shared, N)) {
        // F16 experts, few tokens per expert: the tile kernels on f16 x and h
        MoeJob job{};
        job.eg = L->eg;
        job.eu = L->eu;
        job.ed = L->ed;
        job.sg = L->sg;
        job.su = L->su;
        job.sd = L->sd;
        job.has_shared = L->has_shared;
        job.H = H;
        job.FF = FF;
        job.SF = hp.shared_ff;
        job.n_tokens = N;
        job.top_k = K;
        job.perm = w.rb.perm;
        job.offsets = w.rb.offsets;
        job.counts = w.rb.counts;
        job.E = E;
        job.ec_cap = E + N * K / EXPERT_CHUNK + 1;
        job.wl = w.wl;
        job.h = w.h;
        job.hs = w.hs;
        job.ye = w.ye;
        job.ys = w.ys;
        job.x16 = w.x16;
        job.xs16 = w.xs16;
        job.h16 = w.h16;
        job.hs16 = w.hs16;
        if (L->has_shared)
            STAGE(ST_ACTQ_X, launch_cvt_f16(x, N, H, 1, w.xs16, s));
        else
            STAGE(ST_ACTQ_X, launch_cvt_f16(x, N, H, 0, w.x16, s));
        STAGE(ST_GATEUP, launch_expert_tile(0, job, s));
        STAGE(ST_ACTQ_H, launch_cvt_f16(w.h, N * K, FF, 0, w.h16, s));
        if (L->has_shared) STAGE(ST_ACTQ_H, launch_cvt_f16(w.hs, N, hp.shared_ff, 1, w.hs16, s));
        STAGE(ST_DOWN, launch_expert_tile(1, job, s));
        STAGE(ST_COMBINE, launch_combine(w.ye, w.rb.weights, L->has_shared ? w.ys : nullptr, N,
                                         K, H, y, s));
        return DMOE_OK;
    }
    if (gemm) {
        // F16 experts on MFMA tiles (the prefill path)
        GemmJob job{};
        job.eg = L->eg;
        job.eu = L->eu;
        job.ed = L->ed;
        job.sg = L->sg;
        job.su = L->su;
        job.sd = L->sd;
        job.has_shared = L->has_shared;
        job.H = H;
        job.FF = FF;
        job.SF = hp.shared_ff;
        job.n_tokens = N;
        job.top_k = K;
        job.perm = w.rb.perm;
        job.offsets = w.rb.offsets;
        job.counts = w.rb.counts;
        job.wl = w.wl;
        job.x16 = w.x16;
        job.xs16 = w.xs16;
        job.h16 = w.h16;
        job.hs16 = w.hs16;
        job.ye = w.ye;
        job.ys = w.ys;
        // one conversion: f16(x), or with a shared expert its (hi, lo) pair,
        // whose hi rows are x16
        if (L->has_shared)
            STAGE(ST_ACTQ_X, launch_cvt_f16(x, N, H, 1, w.xs16, s));
        else
            STAGE(ST_ACTQ_X, launch_cvt_f16(x, N, H, 0, w.x16, s));
        STAGE(ST_GATEUP, launch_gemm_f16(0, job, s));
        STAGE(ST_DOWN, launch_gemm_f16(1, job, s));
        STAGE(ST_COMBINE, launch_combine(w.ye, w.rb.weights, L->has_shared ? w.ys : nullptr, N,
                                         K, H, y, s));
        return DMOE_OK;
    }
    STAGE(ST_ACTQ_X, launch_act_quant(x, N, H, w.xq, s));
    STAGE(ST_GATEUP, launch_gateup_routed(L->eg, L->eu, w.xq, rp, w.rb, FF, w.h, s));
    STAGE(ST_ACTQ_H, launch_act_quant(w.h, N * K, FF, w.hq, s));
    STAGE(ST_DOWN, launch_down_routed(L->ed, w.hq, rp, w.rb, H, w.ye, s));
    if (L->has_shared) {
        STAGE(ST_SH_GATEUP, launch_gateup_shared(L->sg, L->su, x, N, H, hp.shared_ff, w.hs, s));
        STAGE(ST_SH_DOWN, launch_down_shared(L->sd, w.hs, N, hp.shared_ff, H, w.ys, s));
    }
    STAGE(ST_COMBINE, launch_combine(w.ye, w.rb.weights, L->has_shared ? w.ys : nullptr, N, K,
                                     H, y, s));
#undef STAGE
    return DMOE_OK;
}

int copy_debug(dmoe_ctx *ctx, const dmoe_hparams &hp, const Workspace &w, int N,
               dmoe_debug *dbg, hipStream_t s)
{
    if (!dbg) return DMOE_OK;
    const int E = hp.n_experts, K = hp.top_k, P = N * K;
    const RouteParams rp = route_params(nullptr, hp, N);
    const int B = rp.use_block ? N / hp.block_size : 0;
    auto cp = [&](void *dst, const void *src, size_t bytes) -> hipError_t {
        if (!dst || bytes == 0) return hipSuccess;
        return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
    };
    HIP_TRY(ctx, cp(dbg->logits, w.rb.logits, (size_t)N * E * 4));
    HIP_TRY(ctx, cp(dbg->probs, w.rb.probs, (size_t)N * E * 4));
    HIP_TRY(ctx, cp(dbg->bmax, w.rb.bmax, (size_t)B * E * 4));
    HIP_TRY(ctx, cp(dbg->thr, w.rb.thr, (size_t)B * 4));
    HIP_TRY(ctx, cp(dbg->allowed, w.rb.allowed, (size_t)B * E));
    HIP_TRY(ctx, cp(dbg->idx, w.rb.idx, (size_t)P * 4));
    HIP_TRY(ctx, cp(dbg->weights, w.rb.weights, (size_t)P * 4));
    HIP_TRY(ctx, cp(dbg->counts, w.rb.counts, (size_t)E * 4));
    HIP_TRY(ctx, cp(dbg->offsets, w.rb.offsets, (size_t)E * 4));
    HIP_TRY(ctx, cp(dbg->perm, w.rb.perm, (size_t)P * 4));
    if (dbg->use_block_routing) *dbg->use_block_routing = rp.use_block;
    return DMOE_OK;
}

// Rewrites one Q4_K tensor into the tiled layout the MFMA kernels stream
// (16-row tiles, super-block-major) in a library-owned buffer; a previous
// library-owned copy is released.
int tile_tensor(dmoe_ctx *ctx, dmoe_layer *L, WTensor &t, int rows, int K, int mats)
{
    const size_t bytes = (size_t)rows * (K / 256) * Q4K_BYTES * mats;
    void *dev = nullptr;
    HIP_TRY(ctx, hipMalloc(&dev, bytes));
    L->owned.push_back(dev);
    HIP_TRY(ctx, launch_tile_q4k(t.data, t.nb1, t.nb2, rows, K, mats, (uint8_t *)dev, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    auto it = std::find(L->owned.begin(), L->owned.end(), (void *)t.data);
    if (it != L->owned.end()) {
        HIP_TRY(ctx, hipFree(*it));
        L->owned.erase(it);
    }
    t.data = (const uint8_t *)dev;
    t.nb1 = Q4K_BYTES;
    t.nb2 = (size_t)rows * (K / 256) * Q4K_BYTES;
    return DMOE_OK;
}

// Q6_K [mats][rows][K] -> the tiled layout of the Q6_K projections
// (k_tile_q6k), in a library-owned copy (a library-owned original is freed).
int tile_tensor_q6k(dmoe_ctx *ctx, dmoe_layer *L, WTensor &t, int rows, int K, int mats)
{
    const size_t bytes = (size_t)rows * (K / 256) * Q6K_BYTES * mats;
    void *dev = nullptr;
    HIP_TRY(ctx, hipMalloc(&dev, bytes));
    L->owned.push_back(dev);
    HIP_TRY(ctx, launch_tile_q6k(t.data, t.nb1, t.nb2, rows, K, mats, (uint8_t *)dev, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    auto it = std::find(L->owned.begin(), L->owned.end(), (void *)t.data);
    if (it != L->owned.end()) {
        HIP_TRY(ctx, hipFree(*it));
        L->owned.erase(it);
    }
    t.data = (const uint8_t *)dev;
    t.nb1 = (size_t)(K / 256) * Q6K_BYTES;
    t.nb2 = (size_t)rows * (K / 256) * Q6K_BYTES;
    return DMOE_OK;
}

// Q8_0 [mats][rows][K] -> the tiled layout of k_expert_q80.hip, in a
// library-owned copy (a library-owned original is freed).
int tile_tensor_q80(dmoe_ctx *ctx, dmoe_layer *L, WTensor &t, int rows, int K, int mats)
{
    const size_t row_bytes = (size_t)(K / 32) * Q8_0_BYTES;
    const size_t bytes = (size_t)rows * row_bytes * mats;
    void *dev = nullptr;
    HIP_TRY(ctx, hipMalloc(&dev, bytes));
    L->owned.push_back(dev);
    HIP_TRY(ctx, launch_tile_q80(t.data, t.nb1, t.nb2, rows, K, mats, (uint8_t *)dev, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    auto it = std::find(L->owned.begin(), L->owned.end(), (void *)t.data);
    if (it != L->owned.end()) {
        HIP_TRY(ctx, hipFree(*it));
        L->owned.erase(it);
    }
    t.data = (const uint8_t *)dev;
    t.nb1 = row_bytes;
    t.nb2 = (size_t)rows * row_bytes;
    return DMOE_OK;
}

// F16 [mats][rows][K] -> the tiled layout of the grouped GEMM (k_gemm.hip), in
// a library-owned copy (a library-owned original is freed).
int tile_tensor_f16(dmoe_ctx *ctx, dmoe_layer *L, WTensor &t, int rows, int K, int mats)
{
    const size_t bytes = (size_t)rows * K * 2 * mats;
    void *dev = nullptr;
    HIP_TRY(ctx, hipMalloc(&dev, bytes));
    L->owned.push_back(dev);
    HIP_TRY(ctx, launch_tile_f16(t.data, t.nb1, t.nb2, rows, K, mats, (uint8_t *)dev, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    auto it = std::find(L->owned.begin(), L->owned.end(), (void *)t.data);
    if (it != L->owned.end()) {
        HIP_TRY(ctx, hipFree(*it));
        L->owned.erase(it);
    }
    t.data = (const uint8_t *)dev;
    t.nb1 = (size_t)K * 2;                          // bytes per row (blocks of 128 rows)
    t.nb2 = (size_t)rows * K * 2;
    return DMOE_OK;
}

int finish_layer(dmoe_ctx *ctx, dmoe_layer *L, const dmoe_hparams *hp, const dmoe_layer_desc *d)
{
    L->hp = *hp;
    // Routing keeps a per-token candidate list only when adding the -1e30
    // mask to a selection score cannot be absorbed by a huge bias.
    L->bias_small = 1;
    if (L->gate_bias) {
        std::vector<float> b(hp->n_experts);
        HIP_TRY(ctx, hipMemcpy(b.data(), L->gate_bias, b.size() * 4, hipMemcpyDeviceToHost));
        for (float v : b)
            if (!(std::fabs(v) < 1e19f)) L->bias_small = 0;
    }
    L->has_shared = hp->n_shared > 0 && d->sh_gate.data != nullptr;
    if (!L->has_shared) L->hp.shared_ff = 0;
    if (use_mfma_path(L->hp, L->eg.type, L->sg.type, L->has_shared)) {
        const int H = hp->n_embd, E = hp->n_experts, FF = hp->moe_ff, SF = L->hp.shared_ff;
        int rc;
        if ((rc = tile_tensor(ctx, L, L->eg, FF, H, E))) return rc;
        if ((rc = tile_tensor(ctx, L, L->eu, FF, H, E))) return rc;
        if ((rc = tile_tensor(ctx, L, L->ed, H, FF, E))) return rc;
        if (L->has_shared) {
            if ((rc = tile_tensor(ctx, L, L->sg, SF, H, 1))) return rc;
            if ((rc = tile_tensor(ctx, L, L->su, SF, H, 1))) return rc;
            if ((rc = tile_tensor(ctx, L, L->sd, H, SF, 1))) return rc;
        }
    }
    if (use_q80_path(L->hp, L->eg.type, L->sg.type, L->has_shared)) {
        const int H = hp->n_embd, E = hp->n_experts, FF = hp->moe_ff, SF = L->hp.shared_ff;
        int rc;
        if ((rc = tile_tensor_q80(ctx, L, L->eg, FF, H, E))) return rc;
        if ((rc = tile_tensor_q80(ctx, L, L->eu, FF, H, E))) return rc;
        if ((rc = tile_tensor_q80(ctx, L, L->ed, H, FF, E))) return rc;
        if (L->has_shared) {
            if ((rc = tile_tensor_q80(ctx, L, L->sg, SF, H, 1))) return rc;
            if ((rc = tile_tensor_q80(ctx, L, L->su, SF, H, 1))) return rc;
            if ((rc = tile_tensor_q80(ctx, L, L->sd, H, SF, 1))) return rc;
        }
    }
    if (use_gemm_path(L->hp, L->eg.type, L->sg.type, L->has_shared)) {
        const int H = hp->n_embd, E = hp->n_experts, FF = hp->moe_ff, SF = L->hp.shared_ff;
        int rc;
        if ((rc = tile_tensor_f16(ctx, L, L->eg, FF, H, E))) return rc;
        if ((rc = tile_tensor_f16(ctx, L, L->eu, FF, H, E))) return rc;
        if ((rc = tile_tensor_f16(ctx, L, L->ed, H, FF, E))) return rc;
        if (L->has_shared) {
            if ((rc = tile_tensor_f16(ctx, L, L->sg, SF, H, 1))) return rc;
            if ((rc = tile_tensor_f16(ctx, L, L->su, SF, H, 1))) return rc;
            if ((rc = tile_tensor_f16(ctx, L, L->sd, H, SF, 1))) return rc;
        }
    }
    return DMOE_OK;
}

// ---------------------------------------------------------------------------
// Dense MLP (src/diffuse-moe-graph.cpp:181-187): the shared expert's kernels
// with an empty routed work list; the down launch writes y directly.
enum DensePath { DP_GEMV = 0, DP_Q4K, DP_Q80, DP_F16, DP_Q6K };

int dense_path(int32_t type, int H, int FF)
{
    if (H % 256 == 0 && FF % 256 == 0) {
        if (type == DMOE_TYPE_Q4_K && FF % expert_rows_per_item(0) == 0 && H % expert_rows_per_item(1) == 0)
            return DP_Q4K;
        if (type == DMOE_TYPE_Q8_0 && FF % expert_q80_rows_per_item(0) == 0 &&
            H % expert_q80_rows_per_item(1) == 0)
            return DP_Q80;
        if (type == DMOE_TYPE_Q6_K) return DP_Q6K;
    }
    if (type == DMOE_TYPE_F16 && gemm_shapes_ok(H, FF, FF, true)) return DP_F16;
    return DP_GEMV;
}

int dense_validate(dmoe_ctx *ctx, int H, int FF, const dmoe_tensor *g, const dmoe_tensor *u,
                   const dmoe_tensor *d, bool device_mode)
{
    if (!g || !u || !d) return set_err(ctx, DMOE_ERR_INVALID_ARG, "dense: NULL tensor");
    if (H <= 0 || H % 256) return set_err(ctx, DMOE_ERR_SHAPE, "dense: n_embd = %d must be a positive multiple of 256", H);
    if (FF <= 0) return set_err(ctx, DMOE_ERR_SHAPE, "dense: n_ff = %d", FF);
    int rc;
    if ((rc = check_tensor(ctx, "ffn_gate", *g, H, FF, 0, device_mode))) return rc;
    if ((rc = check_tensor(ctx, "ffn_up", *u, H, FF, 0, device_mode))) return rc;
    if ((rc = check_tensor(ctx, "ffn_down", *d, FF, H, 0, device_mode))) return rc;
    if (u->type != g->type || d->type != g->type)
        return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "dense: ffn tensors differ in type");
    return DMOE_OK;
}

// hparams of a dense layer: the MLP as a lone shared expert
dmoe_hparams dense_hparams(int H, int FF)
{
    dmoe_hparams hp{};
    hp.n_embd = H;
    hp.moe_ff = FF;
    hp.shared_ff = FF;
    hp.n_shared = 1;
    return hp;
}

int dense_finish(dmoe_ctx *ctx, dmoe_layer *L)
{
    const int H = L->hp.n_embd, FF = L->hp.shared_ff;
    int rc;
    switch (dense_path(L->sg.type, H, FF)) {
    case DP_Q4K:
        if ((rc = tile_tensor(ctx, L, L->sg, FF, H, 1))) return rc;
        if ((rc = tile_tensor(ctx, L, L->su, FF, H, 1))) return rc;
        return tile_tensor(ctx, L, L->sd, H, FF, 1);
    case DP_Q80:
        if ((rc = tile_tensor_q80(ctx, L, L->sg, FF, H, 1))) return rc;
        if ((rc = tile_tensor_q80(ctx, L, L->su, FF, H, 1))) return rc;
        return tile_tensor_q80(ctx, L, L->sd, H, FF, 1);
    case DP_F16:
        if ((rc = tile_tensor_f16(ctx, L, L->sg, FF, H, 1))) return rc;
        if ((rc = tile_tensor_f16(ctx, L, L->su, FF, H, 1))) return rc;
        return tile_tensor_f16(ctx, L, L->sd, H, FF, 1);
    case DP_Q6K:
        if ((rc = tile_tensor_q6k(ctx, L, L->sg, FF, H, 1))) return rc;
        if ((rc = tile_tensor_q6k(ctx, L, L->su, FF, H, 1))) return rc;
        return tile_tensor_q6k(ctx, L, L->sd, H, FF, 1);
    default:
        return DMOE_OK;
    }
}

struct DenseWs {
    float *x, *y;
    int32_t *n_ec;                       // an empty routed work list
    ActI8 axs, ahs;                      // split x and h (int8 paths)
    uint16_t *xs16, *hs16;               // hi / lo f16 pairs (F16 path)
    float *hs;                           // f32 h (GEMV path)
    float *part_gu, *part_d;             // slice sums of the few-token Q4_K projections
};

// Few tokens of a Q4_K or Q6_K dense MLP: gate and up as one two-matrix
// projection, h formed and converted from their slice sums, down as a
// projection.  Q6_K weights take every token count this way, in chunks of up
// to PROJ_MAX_TOKENS tokens (dense_chunk).
bool dense_few(int path, int H, int FF, int N)
{
    return (path == DP_Q4K || path == DP_Q6K) && proj_ok(FF, H, N) && proj_ok(H, FF, N) && FF % 256 == 0;
}

int dense_chunk(int path, int N) { return path == DP_Q6K ? std::min(N, PROJ_MAX_TOKENS) : N; }

// Slice-sum floats the few-token projection of R x K (M matrices) needs at
// any token count 1 .. nmax (a smaller last chunk may split its reduction
// into more slices than a full one); with split_only, counting only launches
// whose reduction is split (KS > 1), 0 when none is.
// The scan costs a few thousand plan evaluations and every forward of a
// projection plans its workspace twice, so results are kept per thread for
// the last few shapes (the host enqueue of a 32-token dense MLP otherwise
// took longer than its kernels).
size_t proj_partial_max(int R, int K, int M, int nmax, bool split_only)
{
    struct Entry {
        int R, K, M, nmax, split;
        size_t v;
    };
    constexpr int kEntries = 16;
    thread_local Entry cache[kEntries];
    thread_local int used = 0, next = 0;
    for (int i = 0; i < used; i++) {
        const Entry &c = cache[i];
        if (c.R == R && c.K == K && c.M == M && c.nmax == nmax && c.split == (int)split_only) return c.v;
    }
    size_t best = 0;
    for (int n = 1; n <= nmax; n++) {
        if (split_only && proj_plan(R, K, M, n).KS <= 1) continue;
        best = std::max(best, proj_partial_floats(R, K, M, n));
    }
    cache[next] = Entry{R, K, M, nmax, (int)split_only, best};
    next = (next + 1) % kEntries;
    used = std::min(used + 1, kEntries);
    return best;
}

int dense_gemm_slices(const KernelSwitches &sw, int path, int H, int FF, int N);

size_t plan_dense(const KernelSwitches &sw, const dmoe_layer *L, int N, bool host_io, uint8_t *base, DenseWs *w)
{
    const int H = L->hp.n_embd, FF = L->hp.shared_ff;
    size_t off = 0;
    std::function<uint8_t *(size_t)> take = [&](size_t bytes) -> uint8_t * {
        uint8_t *p = base ? base + off : nullptr;
        off += align_up(bytes > 0 ? bytes : 1);
        return p;
    };
    DenseWs t{};
    if (host_io) {
        t.x = (float *)take((size_t)N * H * 4);
        t.y = (float *)take((size_t)N * H * 4);
    }
    t.n_ec = (int32_t *)take(4);
    const int path = dense_path(L->sg.type, H, FF);
    switch (path) {
    case DP_Q4K:
    case DP_Q6K: {
        // Q6_K: workspace for one chunk of tokens, reused chunk after chunk
        const int n = dense_chunk(path, N);
        t.axs = take_act(take, n, H, true);
        t.ahs = take_act(take, n, FF, true);
        if (dense_few(path, H, FF, n)) {
            t.part_gu = (float *)take(proj_partial_max(FF, H, 2, n, false) * 4);
            if (const size_t pd = proj_partial_max(H, FF, 1, n, true)) t.part_d = (float *)take(pd * 4);
        } else if (const int ks = dense_gemm_slices(sw, path, H, FF, N)) {
            // the grouped GEMM: f32 h, the down launch's slices
            t.hs = (float *)take((size_t)N * FF * 4);
            if (ks > 1) t.part_d = (float *)take((size_t)ks * N * H * 4);
        }
        break;
    }
    case DP_Q80:
        t.axs = take_act(take, N, H, true, true);
        t.ahs = take_act(take, N, FF, true, true);
        break;
    case DP_F16:
        t.xs16 = (uint16_t *)take((size_t)2 * N * H * 2);
        t.hs16 = (uint16_t *)take((size_t)2 * N * FF * 2);
        break;
    default:
        t.hs = (float *)take((size_t)N * FF * 4);
        break;
    }
    if (w) *w = t;
    return off;
}

int ensure_dense_workspace(dmoe_ctx *ctx, const dmoe_layer *L, int N, bool host_io, DenseWs *w)
{
    const size_t need = plan_dense(ctx->sw, L, N, host_io, nullptr, nullptr);
    if (need > ctx->ws_bytes) {
        if (ctx->ws) {
            HIP_TRY(ctx, hipDeviceSynchronize());
            HIP_TRY(ctx, hipFree(ctx->ws));
            ctx->ws = nullptr;
            ctx->ws_bytes = 0;
        }
        if (getenv("DMOE_FAIL_ALLOC"))
            return set_err(ctx, DMOE_ERR_OOM, "workspace allocation of %zu bytes refused (DMOE_FAIL_ALLOC)", need);
        HIP_TRY(ctx, hipMalloc(&ctx->ws, need));
        ctx->ws_bytes = need;
    }
    plan_dense(ctx->sw, L, N, host_io, (uint8_t *)ctx->ws, w);
    return DMOE_OK;
}

int enqueue_dense(dmoe_ctx *ctx, const dmoe_layer *L, const DenseWs &w, const float *x, int N,
                  float *y, hipStream_t s, bool prof)
{
    const int H = L->hp.n_embd, FF = L->hp.shared_ff;
    const int path = dense_path(L->sg.type, H, FF);
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    if (path == DP_GEMV) {
        STAGE(ST_SH_GATEUP, launch_gateup_shared(L->sg, L->su, x, N, H, FF, w.hs, s));
        STAGE(ST_SH_DOWN, launch_down_shared(L->sd, w.hs, N, FF, H, y, s));
        return DMOE_OK;
    }
    if (dense_few(path, H, FF, dense_chunk(path, N))) {
        // gate and up: one launch over both matrices, h from their slices;
        // tokens t0 .. t0 + n - 1 at a time (every token at once for Q4_K)
        const bool q6 = path == DP_Q6K;
        const int nc = dense_chunk(path, N);
        for (int t0 = 0; t0 < N; t0 += nc) {
            const int n = std::min(nc, N - t0);
            ProjJob gu{};
            gu.w[0] = L->sg.data;
            gu.w[1] = L->su.data;
            gu.M = 2;
            gu.R = FF;
            gu.K = H;
            gu.N = n;
            gu.KS = proj_plan(FF, H, 2, n).KS;
            gu.x = w.axs;
            gu.partial = 1;
            gu.out = w.part_gu;
            ProjJob dn{};
            dn.w[0] = L->sd.data;
            dn.M = 1;
            dn.R = H;
            dn.K = FF;
            dn.N = n;
            dn.KS = proj_plan(H, FF, 1, n).KS;
            dn.x = w.ahs;
            dn.partial = dn.KS > 1;
            dn.out = dn.partial ? w.part_d : y + (size_t)t0 * H;
            dn.ldo = H;
            PrepJob pj{x + (size_t)t0 * H, n, H, ACT_SPLIT, w.axs};
            STAGE(ST_ACTQ_X, launch_prep(&pj, 1, s));
            STAGE(ST_SH_GATEUP, q6 ? launch_proj_q6k(gu, s) : launch_proj_q4k(gu, s));
            STAGE(ST_ACTQ_H, launch_proj_swiglu(w.part_gu, gu.KS, n, FF, w.ahs, s));
            STAGE(ST_SH_DOWN, q6 ? launch_proj_q6k(dn, s) : launch_proj_q4k(dn, s));
            if (dn.partial) STAGE(ST_COMBINE, launch_proj_reduce(w.part_d, dn.KS, n, H, y + (size_t)t0 * H, H, s));
        }
        return DMOE_OK;
    }
    if (const int ks = dense_gemm_slices(ctx->sw, path, H, FF, N)) {
        // many tokens of Q4_K: the grouped GEMM's gate/up and down launches
        // over shared units (no routed work list), h converted between them,
        // the down reduction in slices added in order
        WorkList wl{};
        wl.chunk = EXPERT_GEMM_CHUNK;
        MoeJob job{};
        job.sg = L->sg;
        job.su = L->su;
        job.sd = L->sd;
        job.has_shared = 1;
        job.H = H;
        job.FF = FF;
        job.SF = FF;
        job.n_tokens = N;
        job.top_k = 1;
        job.wl = wl;
        job.axs = w.axs;
        job.hs = w.hs;
        job.ahs = w.ahs;
        job.ys = ks > 1 ? w.part_d : y;
        job.ks = ks;
        PrepJob pj{x, N, H, ACT_SPLIT, w.axs};
        STAGE(ST_ACTQ_X, launch_prep(&pj, 1, s));
        STAGE(ST_SH_GATEUP, launch_expert_gemm_q4k(0, job, s));
        PrepJob hj{w.hs, N, FF, ACT_SPLIT, w.ahs};
        STAGE(ST_ACTQ_H, launch_prep(&hj, 1, s));
        STAGE(ST_SH_DOWN, launch_expert_gemm_q4k(1, job, s));
        if (ks > 1) STAGE(ST_COMBINE, launch_proj_reduce(w.part_d, ks, N, H, y, H, s));
        return DMOE_OK;
    }
    // the expert kernels read an empty routed work list
    LAUNCH_TRY(ctx, launch_fill_i32(w.n_ec, 0, 1, s));
    WorkList wl{};
    wl.n_ec = w.n_ec;
    if (path == DP_F16) {
        wl.chunk = GM;
        GemmJob job{};
        job.sg = L->sg;
        job.su = L->su;
        job.sd = L->sd;
        job.has_shared = 1;
        job.H = H;
        job.FF = FF;
        job.SF = FF;
        job.n_tokens = N;
        job.top_k = 1;
        job.wl = wl;
        job.xs16 = w.xs16;
        job.x16 = w.xs16;
        job.hs16 = w.hs16;
        job.ys = y;
        STAGE(ST_ACTQ_X, launch_cvt_f16(x, N, H, 1, w.xs16, s));
        STAGE(ST_SH_GATEUP, launch_gemm_f16(0, job, s));
        STAGE(ST_SH_DOWN, launch_gemm_f16(1, job, s));
        return DMOE_OK;
    }
    const bool q8 = path == DP_Q80;
    wl.chunk = EXPERT_CHUNK;
    MoeJob job{};
    job.sg = L->sg;
    job.su = L->su;
    job.sd = L->sd;
    job.has_shared = 1;
    job.H = H;
    job.FF = FF;
    job.SF = FF;
    job.n_tokens = N;
    job.top_k = 1;
    job.wl = wl;
    job.ax.K = H;                        // no routed activations
    job.ah.K = FF;
    job.axs = w.axs;
    job.ahs = w.ahs;
    job.ys = y;                          // the shared expert's down output is the MLP's
    PrepJob pj{x, N, H, q8 ? ACT_SPLIT32 : ACT_SPLIT, w.axs};
    STAGE(ST_ACTQ_X, launch_prep(&pj, 1, s));
    STAGE(ST_SH_GATEUP, q8 ? launch_expert_q80(0, job, s) : launch_expert_q4k(0, job, s, 1, ctx->sw.gateup_lds));
    STAGE(ST_SH_DOWN, q8 ? launch_expert_q80(1, job, s) : launch_expert_q4k(1, job, s));
#undef STAGE
    return DMOE_OK;
}

// ---------------------------------------------------------------------------
// Step tail (src/diffuse-moe-graph.cpp:295-300 and the temperature-0 sampler,
// src/diffuse-sampler.cpp:29-49): rms_norm * output_norm, the LM head as a
// shared expert's down product of n_vocab rows (F32 weight semantics, as
// ensure_f32_moe gives the reference), then argmax and confidence per row.
int head_path(int32_t type, int V, int H)
{
    if (H % 256 == 0) {
        if (type == DMOE_TYPE_Q4_K && V % expert_rows_per_item(1) == 0 && V % 256 == 0) return DP_Q4K;
        if (type == DMOE_TYPE_Q8_0 && V % expert_q80_rows_per_item(1) == 0 && V % 256 == 0) return DP_Q80;
        if (type == DMOE_TYPE_Q6_K && V % 16 == 0) return DP_Q6K;
    }
    if (type == DMOE_TYPE_F16 && gemm_shapes_ok(V, H, H, true)) return DP_F16;
    return DP_GEMV;
}

// Output rows up to which a few-token Q4_K projection runs one workgroup per
// 16 rows (k_down_rows); above it (the LM head) the expert kernel's items.
constexpr int PROJ_ROWS_MAX = 32768;

// One projection y [N][rows] = W x with W's F32 semantics (x [N][K] f32):
// the shared-down product of the expert kernels (Q4_K / Q8_0 on int8 digits,
// F16 on hi / lo pairs) or the GEMV kernel.
struct ProjWs {
    int32_t *n_ec;                       // an empty routed work list
    ActI8 act;                           // split x (int8 paths)
    uint16_t *x16;                       // hi / lo f16 x (F16 path)
    float *part;                         // slice sums of the few-token Q4_K projection
};

// Tokens per launch of a projection: Q6_K runs only the few-token kernel,
// in chunks of up to PROJ_MAX_TOKENS tokens.
int proj_chunk(int path, int N) { return path == DP_Q6K ? std::min(N, PROJ_MAX_TOKENS) : N; }

// Q4_K projections of PROJ_GEMM_MIN_TOKENS or more tokens run on the grouped
// GEMM's down launch (k_expert_gemm.hip) with shared units only: 64 tokens
// (128 digit rows) per unit, 256 output rows per item, the reduction split
// into slices of 2 or more super-blocks, as many as minimise the static
// schedule's rounds x steps plus the slices' own traffic.  Returns the slice
// count, 0 where the GEMM does not take the shape.
constexpr int PROJ_GEMM_MIN_TOKENS = 33;

int proj_gemm_slices(const KernelSwitches &sw, int path, int rows, int K, int N)
{
    if (path != DP_Q4K || sw.proj_gemm == 0 || (sw.proj_gemm < 0 && N < PROJ_GEMM_MIN_TOKENS) ||
        !expert_gemm_q4k_ok(rows, K, K, true) || 2L * N * K >= (1L << 31))
        return 0;
    int n_cu = 0;
    if (device_cu_count(&n_cu) != hipSuccess || n_cu <= 0) n_cu = 256;
    const long items = (long)((N + 63) / 64) * (rows / 256);
    const int nsb = K / 256;
    const long grid = (n_cu + 7) / 8 * 8;
    // rounds of the static schedule x super-blocks per item at ~4.5 us per
    // step, plus the slices written and read again at ~4 TB/s
    int best = 1;
    double best_us = 0.0;
    for (int ks = 1; ks <= 16; ks *= 2) {
        if (nsb % ks || (ks > 1 && nsb / ks < 2)) continue;
        const long rounds = (items * ks + grid - 1) / grid;
        double us = 4.5 * (double)(rounds * (nsb / ks));
        if (ks > 1) us += (double)ks * N * rows * 8 / 4e6;
        if (ks == 1 || us < best_us) {
            best = ks;
            best_us = us;
        }
    }
    return best;
}

// The dense MLP past the few-token kernels on the same GEMM (gate/up, then
// down in proj_gemm_slices slices): 0 where it does not take the shape.
int dense_gemm_slices(const KernelSwitches &sw, int path, int H, int FF, int N)
{
    if (2L * N * H >= (1L << 31)) return 0;
    return proj_gemm_slices(sw, path, H, FF, N);
}

template <class Take>
ProjWs plan_proj(const KernelSwitches &sw, int path, int N, int K, int rows, Take &&take)
{
    ProjWs p{};
    p.n_ec = (int32_t *)take(4);
    switch (path) {
    case DP_Q4K:
    case DP_Q6K: {
        const int n = proj_chunk(path, N);
        p.act = take_act(take, n, K, true);
        if (proj_ok(rows, K, n)) {
            if (const size_t pf = proj_partial_max(rows, K, 1, n, true)) p.part = (float *)take(pf * 4);
        } else if (const int ks = proj_gemm_slices(sw, path, rows, K, N); ks > 1) {
            p.part = (float *)take((size_t)ks * N * rows * 4);
        }
        break;
    }
    case DP_Q80: p.act = take_act(take, N, K, true, true); break;
    case DP_F16: p.x16 = (uint16_t *)take((size_t)2 * N * K * 2); break;
    default: break;
    }
    return p;
}

// Few tokens of Q4_K or Q6_K weights: k_proj.hip on x already converted to
// p.act.
bool proj_few(int path, int rows, int K, int N)
{
    return (path == DP_Q4K || path == DP_Q6K) && proj_ok(rows, K, N);
}

// y [N][rows] = W x from p.act: 128 T-row tiles x reduction slices over every
// CU.  With ks_out the slices are left for the consumer to add in order
// (*src_out: the slices, *ks_out of them, N rows apart); else they are added
// into y here.
int enqueue_proj_few(dmoe_ctx *ctx, bool prof, int st_prod, const WTensor &W, int rows, int K, int N,
                     const ProjWs &p, float *y, int *ks_out, const float **src_out, hipStream_t s)
{
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    ProjJob j{};
    j.w[0] = W.data;
    j.M = 1;
    j.R = rows;
    j.K = K;
    j.N = N;
    j.KS = proj_plan(rows, K, 1, N).KS;
    j.x = p.act;
    j.partial = j.KS > 1;
    j.out = j.partial ? p.part : y;
    j.ldo = rows;
    STAGE(st_prod, W.type == DMOE_TYPE_Q6_K ? launch_proj_q6k(j, s) : launch_proj_q4k(j, s));
    if (ks_out) {
        *ks_out = j.KS;
        *src_out = j.out;
    } else if (j.partial) {
        STAGE(ST_COMBINE, launch_proj_reduce(p.part, j.KS, N, rows, y, rows, s));
    }
#undef STAGE
    return DMOE_OK;
}

// y [N][rows] = W x from p.act on the grouped GEMM's down launch over
// shared units (no routed work list), in ks reduction slices; with ks_out the
// slices are left to the consumer as in enqueue_proj_few, else added into y.
int enqueue_proj_gemm(dmoe_ctx *ctx, bool prof, int st_prod, const WTensor &W, int rows, int K, int N, int ks,
                      const ProjWs &p, float *y, int *ks_out, const float **src_out, hipStream_t s)
{
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    MoeJob job{};
    job.sd = W;
    job.has_shared = 1;
    job.H = rows;
    job.FF = K;
    job.SF = K;
    job.n_tokens = N;
    job.top_k = 1;
    job.wl.chunk = EXPERT_GEMM_CHUNK;
    job.ahs = p.act;
    job.ys = ks > 1 ? p.part : y;
    job.ks = ks;
    STAGE(st_prod, launch_expert_gemm_q4k(1, job, s));
    if (ks_out) {
        *ks_out = ks;
        *src_out = job.ys;
    } else if (ks > 1) {
        STAGE(ST_COMBINE, launch_proj_reduce(p.part, ks, N, rows, y, rows, s));
    }
#undef STAGE
    return DMOE_OK;
}

// Projections that take p.act's digits from the caller (k_norm_fused writes
// them beside its RMSNorm): the few-token kernel or, for many tokens of Q4_K,
// the GEMM (*gemm_ks its slice count, else 0).
bool proj_takes_digits(const KernelSwitches &sw, int path, int rows, int K, int N, int *gemm_ks)
{
    *gemm_ks = 0;
    if (proj_few(path, rows, K, N)) return true;
    *gemm_ks = proj_gemm_slices(sw, path, rows, K, N);
    return *gemm_ks > 0;
}

int enqueue_proj_digits(dmoe_ctx *ctx, bool prof, int st_prod, const WTensor &W, int rows, int K, int N, int gemm_ks,
                        const ProjWs &p, float *y, int *ks_out, const float **src_out, hipStream_t s)
{
    return gemm_ks ? enqueue_proj_gemm(ctx, prof, st_prod, W, rows, K, N, gemm_ks, p, y, ks_out, src_out, s)
                   : enqueue_proj_few(ctx, prof, st_prod, W, rows, K, N, p, y, ks_out, src_out, s);
}

int enqueue_proj(dmoe_ctx *ctx, bool prof, int st_conv, int st_prod, const WTensor &W, int rows, int K,
                 const float *x, int N, float *y, const ProjWs &p, hipStream_t s)
{
    const int path = head_path(W.type, rows, K);
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    if (path == DP_GEMV) {
        STAGE(st_prod, launch_down_shared(W, x, N, K, rows, y, s));
        return DMOE_OK;
    }
    if (proj_few(path, rows, K, proj_chunk(path, N))) {
        // every token at once, or (Q6_K) chunks of up to PROJ_MAX_TOKENS
        const int nc = proj_chunk(path, N);
        for (int t0 = 0; t0 < N; t0 += nc) {
            const int n = std::min(nc, N - t0);
            PrepJob pj{x + (size_t)t0 * K, n, K, ACT_SPLIT, p.act};
            STAGE(st_conv, launch_prep(&pj, 1, s));
            int rc = enqueue_proj_few(ctx, prof, st_prod, W, rows, K, n, p, y + (size_t)t0 * rows, nullptr, nullptr, s);
            if (rc) return rc;
        }
        return DMOE_OK;
    }
    if (const int ks = proj_gemm_slices(ctx->sw, path, rows, K, N)) {
        // many tokens of Q4_K: the grouped GEMM's down launch over shared
        // units, its reduction slices added in order
        PrepJob pj{x, N, K, ACT_SPLIT, p.act};
        STAGE(st_conv, launch_prep(&pj, 1, s));
        return enqueue_proj_gemm(ctx, prof, st_prod, W, rows, K, N, ks, p, y, nullptr, nullptr, s);
    }
    LAUNCH_TRY(ctx, launch_fill_i32(p.n_ec, 0, 1, s));
    WorkList wl{};
    wl.n_ec = p.n_ec;
    if (path == DP_F16) {
        wl.chunk = GM;
        GemmJob job{};
        job.sd = W;
        job.has_shared = 1;
        job.H = rows;
        job.FF = K;
        job.SF = K;
        job.n_tokens = N;
        job.top_k = 1;
        job.wl = wl;
        job.hs16 = p.x16;
        job.ys = y;
        STAGE(st_conv, launch_cvt_f16(x, N, K, 1, p.x16, s));
        STAGE(st_prod, launch_gemm_f16(1, job, s));
        return DMOE_OK;
    }
    const bool q8 = path == DP_Q80;
    if (!q8 && N <= DR_MAX_TOKENS && rows <= PROJ_ROWS_MAX) {
        // few tokens, up to a few thousand rows: one workgroup per 16 output
        // rows over every token (k_down_rows with the shared slot only), so
        // the weights stream once from as many compute units as there are
        // 16-row tiles
        DownRowsJob dj{};
        dj.sd = W;
        dj.has_shared = 1;
        dj.N = N;
        dj.K = 0;
        dj.E = 0;
        dj.H = rows;
        dj.FF = K;
        dj.wl = wl;
        dj.wl.chunk = EXPERT_CHUNK;
        dj.ec_cap = 0;
        dj.ahs = p.act;
        dj.y = y;
        PrepJob pj{x, N, K, ACT_SPLIT, p.act};
        STAGE(st_conv, launch_prep(&pj, 1, s));
        STAGE(st_prod, launch_down_rows(dj, s));
        return DMOE_OK;
    }
    // more rows or tokens: items of up to 32 tokens (4 column blocks of 8
    // tokens' two digit rows) per weight-tile read
    const int nc = q8 ? 1 : (N >= 32 ? 4 : N >= 16 ? 2 : 1);
    wl.chunk = EXPERT_CHUNK * nc;
    MoeJob job{};
    job.sd = W;
    job.has_shared = 1;
    job.H = rows;                        // output rows
    job.FF = K;                          // reduction length
    job.SF = K;
    job.n_tokens = N;
    job.top_k = 1;
    job.wl = wl;
    job.ax.K = rows;
    job.ah.K = K;
    job.ahs = p.act;
    job.ys = y;
    PrepJob pj{x, N, K, q8 ? ACT_SPLIT32 : ACT_SPLIT, p.act};
    STAGE(st_conv, launch_prep(&pj, 1, s));
    STAGE(st_prod, q8 ? launch_expert_q80(1, job, s) : launch_expert_q4k(1, job, s, nc));
#undef STAGE
    return DMOE_OK;
}

// Tiles a projection weight for its path (library-owned copy).
int tile_proj(dmoe_ctx *ctx, dmoe_layer *L, WTensor &W, int rows, int K)
{
    switch (head_path(W.type, rows, K)) {
    case DP_Q4K: return tile_tensor(ctx, L, W, rows, K, 1);
    case DP_Q6K: return tile_tensor_q6k(ctx, L, W, rows, K, 1);
    case DP_Q80: return tile_tensor_q80(ctx, L, W, rows, K, 1);
    case DP_F16: return tile_tensor_f16(ctx, L, W, rows, K, 1);
    default: return DMOE_OK;
    }
}

// Grows the context workspace to `need` bytes (synchronising before a free).
int grow_workspace(dmoe_ctx *ctx, size_t need)
{
    if (need <= ctx->ws_bytes) return DMOE_OK;
    if (ctx->ws) {
        HIP_TRY(ctx, hipDeviceSynchronize());
        HIP_TRY(ctx, hipFree(ctx->ws));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    if (getenv("DMOE_FAIL_ALLOC"))
        return set_err(ctx, DMOE_ERR_OOM, "workspace allocation of %zu bytes refused (DMOE_FAIL_ALLOC)", need);
    HIP_TRY(ctx, hipMalloc(&ctx->ws, need));
    ctx->ws_bytes = need;
    return DMOE_OK;
}

struct HeadWs {
    float *h;                            // host input copy
    int32_t *tokens;                     // host output staging
    float *probs;
    float *xn;                           // rms_norm(h) * output_norm
    float *logits;                       // [N][V] (unless the caller's)
    ArgmaxPart *part;                    // per-chunk argmax / exp-sum partials
    ProjWs proj;
};

size_t plan_head(const KernelSwitches &sw, const dmoe_layer *L, int N, bool host_io, bool own_logits, uint8_t *base,
                 HeadWs *w)
{
    const int H = L->hp.n_embd, V = L->n_vocab;
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t * {
        uint8_t *p = base ? base + off : nullptr;
        off += align_up(bytes > 0 ? bytes : 1);
        return p;
    };
    HeadWs t{};
    if (host_io) {
        t.h = (float *)take((size_t)N * H * 4);
        t.tokens = (int32_t *)take((size_t)N * 4);
        t.probs = (float *)take((size_t)N * 4);
    }
    t.xn = (float *)take((size_t)N * H * 4);
    if (own_logits) t.logits = (float *)take((size_t)N * V * 4);
    t.part = (ArgmaxPart *)take(argmax_partials_bytes(N, V));
    t.proj = plan_proj(sw, head_path(L->sd.type, V, H), N, H, V, take);
    if (w) *w = t;
    return off;
}

int ensure_head_workspace(dmoe_ctx *ctx, const dmoe_layer *L, int N, bool host_io, bool own_logits,
                          HeadWs *w)
{
    int rc = grow_workspace(ctx, plan_head(ctx->sw, L, N, host_io, own_logits, nullptr, nullptr));
    if (rc) return rc;
    plan_head(ctx->sw, L, N, host_io, own_logits, (uint8_t *)ctx->ws, w);
    return DMOE_OK;
}

int enqueue_head(dmoe_ctx *ctx, const dmoe_layer *L, const HeadWs &w, const float *h, int N, float eps,
                 int32_t *tokens, float *probs, float *logits, hipStream_t s)
{
    const int H = L->hp.n_embd, V = L->n_vocab;
    const bool prof = ctx->prof;
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    // :296-297 rms_norm(cur) * output_norm (h is only read: no residual add);
    // :299 the LM head.  On the few-token kernel or the GEMM the norm hands
    // the head its int8 digits directly.
    int rc, gh = 0;
    if (proj_takes_digits(ctx->sw, head_path(L->sd.type, V, H), V, H, N, &gh) && H <= 8192) {
        NormArgs na{};
        na.h_in = h;
        na.gain = L->gate_w;
        na.act = w.proj.act;
        na.rows = N;
        na.H = H;
        na.eps = eps;
        STAGE(ST_FRONT, launch_norm_fused(na, s));
        rc = enqueue_proj_digits(ctx, prof, ST_SH_DOWN, L->sd, V, H, N, gh, w.proj, logits, nullptr, nullptr, s);
    } else {
        STAGE(ST_FRONT, launch_residual_rmsnorm(const_cast<float *>(h), nullptr, L->gate_w, w.xn, N, H, eps, s));
        rc = enqueue_proj(ctx, prof, ST_ACTQ_H, ST_SH_DOWN, L->sd, V, H, w.xn, N, logits, w.proj, s);
    }
    if (rc) return rc;
    STAGE(ST_COMBINE, launch_argmax_prob(logits, N, V, w.part, tokens, probs, s));
#undef STAGE
    return DMOE_OK;
}

// ---------------------------------------------------------------------------
// Attention half of the layer (src/diffuse-moe-graph.cpp:116-178).
struct AttnWs {
    float *h, *h_out, *moe_in;           // host io copies
    float *xn;                           // rms_norm(h) * attn_norm       [N][H]
    float *qkv;                          // fused projection              [N][QKV]
    float *Qh, *Kh, *Vh;                 // head-major after norm / RoPE
    float *att;                          // attention output              [N][nh hd]
    float *proj;                         // output projection             [N][H]
    float *scratch;                      // post-norm output when not wanted [N][H]
    ProjWs pq, po;
};

size_t plan_attn(const KernelSwitches &sw, const dmoe_layer *L, int N, bool host_io, uint8_t *base, AttnWs *w)
{
    const dmoe_attn_hparams &a = L->ahp;
    const int H = a.n_embd, QD = a.n_head * a.head_dim, KD = a.n_head_kv * a.head_dim, QKV = QD + 2 * KD;
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t * {
        uint8_t *p = base ? base + off : nullptr;
        off += align_up(bytes > 0 ? bytes : 1);
        return p;
    };
    AttnWs t{};
    if (host_io) {
        t.h = (float *)take((size_t)N * H * 4);
        t.h_out = (float *)take((size_t)N * H * 4);
        t.moe_in = (float *)take((size_t)N * H * 4);
    }
    t.xn = (float *)take((size_t)N * H * 4);
    t.qkv = (float *)take((size_t)N * QKV * 4);
    t.Qh = (float *)take((size_t)N * QD * 4);
    t.Kh = (float *)take((size_t)N * KD * 4);
    t.Vh = (float *)take((size_t)N * KD * 4);
    t.att = (float *)take((size_t)N * QD * 4);
    t.proj = (float *)take((size_t)N * H * 4);
    t.scratch = (float *)take((size_t)N * H * 4);
    t.pq = plan_proj(sw, head_path(L->aqkv.type, QKV, H), N, H, QKV, take);
    t.po = plan_proj(sw, head_path(L->awo.type, H, QD), N, QD, H, take);
    if (w) *w = t;
    return off;
}

int enqueue_attn(dmoe_ctx *ctx, const dmoe_layer *L, const AttnWs &w, const float *h, int N, float *h_out,
                 float *moe_in, hipStream_t s)
{
    const dmoe_attn_hparams &a = L->ahp;
    const int H = a.n_embd, QD = a.n_head * a.head_dim, KD = a.n_head_kv * a.head_dim, QKV = QD + 2 * KD;
    const bool prof = ctx->prof;
    // Q4_K / Q6_K projections on the few-token kernel or the GEMM: the norms
    // hand them int8 digits and take their reduction slices directly
    // (k_norm_fused, k_qk_rope)
    int gq = 0, go = 0;
    const bool fq = proj_takes_digits(ctx->sw, head_path(L->aqkv.type, QKV, H), QKV, H, N, &gq) && H <= 8192;
    const bool fo = proj_takes_digits(ctx->sw, head_path(L->awo.type, H, QD), H, QD, N, &go) && H <= 8192;
#define STAGE(id, call) LAUNCH_TRY(ctx, stage(ctx, prof, id, s, [&] { return call; }))
    // :120-121 input layernorm; :124 fused QKV
    const float *qkv = w.qkv;
    int qks = 1;
    int rc;
    if (fq) {
        NormArgs na{};
        na.h_in = h;
        na.gain = L->attn_norm;
        na.act = w.pq.act;
        na.rows = N;
        na.H = H;
        na.eps = a.rms_eps;
        STAGE(ST_FRONT, launch_norm_fused(na, s));
        if ((rc = enqueue_proj_digits(ctx, prof, ST_SH_GATEUP, L->aqkv, QKV, H, N, gq, w.pq, w.qkv, &qks, &qkv, s)))
            return rc;
    } else {
        STAGE(ST_FRONT, launch_residual_rmsnorm(const_cast<float *>(h), nullptr, L->attn_norm, w.xn, N, H,
                                                a.rms_eps, s));
        if ((rc = enqueue_proj(ctx, prof, ST_ACTQ_X, ST_SH_GATEUP, L->aqkv, QKV, H, w.xn, N, w.qkv, w.pq, s)))
            return rc;
    }
    AttnDims d{};
    d.n = N;
    d.nh = a.n_head;
    d.nkv = a.n_head_kv;
    d.hd = a.head_dim;
    d.rd = a.rotary_dim;
    d.qk_norm = a.use_qk_norm;
    d.block = a.block_length;
    d.eps = a.rms_eps;
    // the rope cache's angle step, as ggml computes it on the host
    d.theta_scale = a.rotary_dim > 0 ? powf(a.rope_base, -2.0f / (float)a.rotary_dim) : 1.0f;
    d.scale = 1.0f / sqrtf((float)a.head_dim);
    d.waves = ctx->sw.attn_waves;
    STAGE(ST_ROUTE, launch_qk_rope(qkv, qks, (size_t)N * QKV, L->qn, L->kn, d, w.Qh, w.Kh, w.Vh, s));
    STAGE(ST_SCORES, launch_attn(w.Qh, w.Kh, w.Vh, d, w.att, s));
    // :172 output projection; :175-178 residual, then the post-attention
    // layernorm (the MoE input)
    if (fo) {
        PrepJob pj{w.att, N, QD, ACT_SPLIT, w.po.act};
        STAGE(ST_ACTQ_H, launch_prep(&pj, 1, s));
        const float *o = w.proj;
        int oks = 1;
        if ((rc = enqueue_proj_digits(ctx, prof, ST_SH_DOWN, L->awo, H, QD, N, go, w.po, w.proj, &oks, &o, s)))
            return rc;
        NormArgs na{};
        na.h_in = h;
        na.h_out = h_out;
        na.y = o;
        na.ks = oks;
        na.kstride = (size_t)N * H;
        na.gain = L->post_norm;
        na.x = moe_in;
        na.rows = N;
        na.H = H;
        na.eps = a.rms_eps;
        STAGE(ST_COMBINE, launch_norm_fused(na, s));
    } else {
        if ((rc = enqueue_proj(ctx, prof, ST_ACTQ_H, ST_SH_DOWN, L->awo, H, QD, w.att, N, w.proj, w.po, s)))
            return rc;
        if (h_out != h) HIP_TRY(ctx, hipMemcpyAsync(h_out, h, (size_t)N * H * 4, hipMemcpyDeviceToDevice, s));
        STAGE(ST_COMBINE, launch_residual_rmsnorm(h_out, w.proj, L->post_norm, moe_in ? moe_in : w.scratch, N, H,
                                                  a.rms_eps, s));
    }
#undef STAGE
    return DMOE_OK;
}

} // namespace

KernelSwitches read_kernel_switches()
{
    KernelSwitches sw;
    auto flag = [](const char *name) {
        const char *v = getenv(name);
        return v && atoi(v) == 1;
    };
    if (const char *v = getenv("DMOE_Q4K_COLUMN_BLOCKS")) {
        const int n = atoi(v);
        if (n == 1 || n == 2 || n == 4) sw.q4k_column_blocks = n;
    }
    sw.down_fused = flag("DMOE_DOWN_FUSED");
    sw.gateup_lds = flag("DMOE_GATEUP_LDS");
    if (const char *v = getenv("DMOE_EXPERT_TILE")) {
        const int n = atoi(v);
        if (n == 0 || n == 1) sw.expert_tile = n;
    }
    if (const char *v = getenv("DMOE_EXPERT_GEMM")) {
        const int n = atoi(v);
        if (n == 0 || n == 1) sw.expert_gemm = n;
    }
    if (const char *v = getenv("DMOE_PROJ_GEMM")) {
        const int n = atoi(v);
        if (n == 0 || n == 1) sw.proj_gemm = n;
    }
    if (const char *v = getenv("DMOE_ATTN_WAVES")) {
        const int n = atoi(v);
        if (n == 4 || n == 8) sw.attn_waves = n;
    }
    return sw;
}

// ===========================================================================
extern "C" {

int dmoe_create(int hip_device, dmoe_ctx **out)
{
    if (!out) return DMOE_ERR_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || hip_device < 0 || hip_device >= n)
        return DMOE_ERR_HIP;
    dmoe_ctx *ctx = new (std::nothrow) dmoe_ctx();
    if (!ctx) return DMOE_ERR_OOM;
    ctx->device = hip_device;
    ctx->sw = read_kernel_switches();
    if (hip_device >= kMaxDevices || hipSetDevice(hip_device) != hipSuccess ||
        scratch_address(hip_device, &ctx->scratch) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return DMOE_ERR_HIP;
    }
    *out = ctx;
    return DMOE_OK;
}

void dmoe_destroy(dmoe_ctx *ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    for (auto &m : ctx->marks) {
        (void)hipEventDestroy(m.a);
        (void)hipEventDestroy(m.b);
    }
    for (hipEvent_t e : ctx->pool) (void)hipEventDestroy(e);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char *dmoe_last_error(const dmoe_ctx *ctx)
{
    return ctx ? ctx->err.c_str() : "null context";
}

size_t dmoe_row_size(int32_t type, int64_t n)
{
    return n > 0 ? row_bytes(type, n) : 0;
}

int dmoe_layer_upload(dmoe_ctx *ctx, const dmoe_hparams *hp, const dmoe_layer_desc *d,
                      dmoe_layer **out)
{
    if (!ctx || !out) return DMOE_ERR_INVALID_ARG;
    *out = nullptr;
    int rc = validate(ctx, hp, d, false);
    if (rc) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    dmoe_layer *L = new (std::nothrow) dmoe_layer();
    if (!L) return set_err(ctx, DMOE_ERR_OOM, "host allocation failed");
    L->ctx = ctx;
    L->device = ctx->device;
    const int H = hp->n_embd, E = hp->n_experts, FF = hp->moe_ff;
    auto fail = [&](int code) {
        dmoe_layer_free(L);
        return code;
    };
    // router -> f32 [E][H]  (ensure_f32_moe, diffuse-moe-graph.cpp:8-12, :203)
    {
        std::vector<float> w((size_t)E * H);
        const dmoe_tensor &gw = d->gate_w;
        for (int e = 0; e < E; e++) {
            const uint8_t *row = (const uint8_t *)gw.data + (size_t)e * gw.nb[1];
            if (gw.type == DMOE_TYPE_F32)
                memcpy(&w[(size_t)e * H], row, (size_t)H * 4);
            else
                for (int k = 0; k < H; k++)
                    w[(size_t)e * H + k] = f16_to_f32_host(((const uint16_t *)row)[k]);
        }
        void *dev = nullptr;
        hipError_t he = hipMalloc(&dev, w.size() * 4);
        if (he != hipSuccess) return fail(set_err(ctx, DMOE_ERR_OOM, "hipMalloc router: %s", hipGetErrorString(he)));
        L->owned.push_back(dev);
        he = hipMemcpy(dev, w.data(), w.size() * 4, hipMemcpyHostToDevice);
        if (he != hipSuccess) return fail(set_err(ctx, DMOE_ERR_HIP, "router copy: %s", hipGetErrorString(he)));
        L->gate_w = (float *)dev;
    }
    if (d->gate_bias.data) {
        void *dev = nullptr;
        hipError_t he = hipMalloc(&dev, (size_t)E * 4);
        if (he != hipSuccess) return fail(set_err(ctx, DMOE_ERR_OOM, "hipMalloc bias: %s", hipGetErrorString(he)));
        L->owned.push_back(dev);
        he = hipMemcpy(dev, d->gate_bias.data, (size_t)E * 4, hipMemcpyHostToDevice);
        if (he != hipSuccess) return fail(set_err(ctx, DMOE_ERR_HIP, "bias copy: %s", hipGetErrorString(he)));
        L->gate_bias = (float *)dev;
    }
    if ((rc = upload_tensor(ctx, L, d->exp_gate, FF, E, L->eg))) return fail(rc);
    if ((rc = upload_tensor(ctx, L, d->exp_up, FF, E, L->eu))) return fail(rc);
    if ((rc = upload_tensor(ctx, L, d->exp_down, H, E, L->ed))) return fail(rc);
    if (hp->n_shared > 0 && d->sh_gate.data) {
        if ((rc = upload_tensor(ctx, L, d->sh_gate, hp->shared_ff, 1, L->sg))) return fail(rc);
        if ((rc = upload_tensor(ctx, L, d->sh_up, hp->shared_ff, 1, L->su))) return fail(rc);
        if ((rc = upload_tensor(ctx, L, d->sh_down, H, 1, L->sd))) return fail(rc);
    }
    if ((rc = finish_layer(ctx, L, hp, d))) return fail(rc);
    *out = L;
    return DMOE_OK;
}

int dmoe_layer_wrap_device(dmoe_ctx *ctx, const dmoe_hparams *hp, const dmoe_layer_desc *d,
                           dmoe_layer **out)
{
    if (!ctx || !out) return DMOE_ERR_INVALID_ARG;
    *out = nullptr;
    int rc = validate(ctx, hp, d, true);
    if (rc) return rc;
    dmoe_layer *L = new (std::nothrow) dmoe_layer();
    if (!L) return set_err(ctx, DMOE_ERR_OOM, "host allocation failed");
    L->ctx = ctx;
    L->device = ctx->device;
    L->gate_w = (float *)d->gate_w.data;
    L->gate_bias = (float *)d->gate_bias.data;
    L->eg = wrap_tensor(d->exp_gate);
    L->eu = wrap_tensor(d->exp_up);
    L->ed = wrap_tensor(d->exp_down);
    if (hp->n_shared > 0 && d->sh_gate.data) {
        L->sg = wrap_tensor(d->sh_gate);
        L->su = wrap_tensor(d->sh_up);
        L->sd = wrap_tensor(d->sh_down);
    }
    if ((rc = finish_layer(ctx, L, hp, d))) {
        dmoe_layer_free(L);
        return rc;
    }
    *out = L;
    return DMOE_OK;
}

static int dense_create(dmoe_ctx *ctx, int32_t n_embd, int32_t n_ff, const dmoe_tensor *gate,
                        const dmoe_tensor *up, const dmoe_tensor *down, bool device_mode,
                        dmoe_layer **out)
{
    if (!ctx || !out) return DMOE_ERR_INVALID_ARG;
    *out = nullptr;
    int rc = dense_validate(ctx, n_embd, n_ff, gate, up, down, device_mode);
    if (rc) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    dmoe_layer *L = new (std::nothrow) dmoe_layer();
    if (!L) return set_err(ctx, DMOE_ERR_OOM, "host allocation failed");
    L->ctx = ctx;
    L->device = ctx->device;
    L->dense = true;
    L->has_shared = true;
    L->hp = dense_hparams(n_embd, n_ff);
    if (device_mode) {
        L->sg = wrap_tensor(*gate);
        L->su = wrap_tensor(*up);
        L->sd = wrap_tensor(*down);
    } else if ((rc = upload_tensor(ctx, L, *gate, n_ff, 1, L->sg)) ||
               (rc = upload_tensor(ctx, L, *up, n_ff, 1, L->su)) ||
               (rc = upload_tensor(ctx, L, *down, n_embd, 1, L->sd))) {
        dmoe_layer_free(L);
        return rc;
    }
    if ((rc = dense_finish(ctx, L))) {
        dmoe_layer_free(L);
        return rc;
    }
    *out = L;
    return DMOE_OK;
}

static int f32_vector(dmoe_ctx *ctx, dmoe_layer *L, const dmoe_tensor &t, int n, bool device_mode,
                      const char *name, float **out)
{
    if (!t.data) return set_err(ctx, DMOE_ERR_INVALID_ARG, "%s: data is NULL", name);
    if (t.ne[0] != n || t.ne[1] > 1)
        return set_err(ctx, DMOE_ERR_SHAPE, "%s: ne0 = %lld, expected %d", name, (long long)t.ne[0], n);
    if (t.type != DMOE_TYPE_F32 && !(t.type == DMOE_TYPE_F16 && !device_mode))
        return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "%s: type %d", name, t.type);
    if (device_mode) {
        if ((uintptr_t)t.data % 16) return set_err(ctx, DMOE_ERR_SHAPE, "%s: device data not 16-byte aligned", name);
        *out = (float *)t.data;
        return DMOE_OK;
    }
    std::vector<float> w((size_t)n);
    for (int k = 0; k < n; k++)
        w[k] = t.type == DMOE_TYPE_F32 ? ((const float *)t.data)[k] : f16_to_f32_host(((const uint16_t *)t.data)[k]);
    void *dev = nullptr;
    hipError_t he = hipMalloc(&dev, (size_t)n * 4);
    if (he != hipSuccess) return set_err(ctx, DMOE_ERR_OOM, "hipMalloc %s: %s", name, hipGetErrorString(he));
    L->owned.push_back(dev);
    he = hipMemcpy(dev, w.data(), (size_t)n * 4, hipMemcpyHostToDevice);
    if (he != hipSuccess) return set_err(ctx, DMOE_ERR_HIP, "%s copy: %s", name, hipGetErrorString(he));
    *out = (float *)dev;
    return DMOE_OK;
}

static int head_create(dmoe_ctx *ctx, int32_t n_embd, int32_t n_vocab, const dmoe_tensor *norm,
                       const dmoe_tensor *output, bool device_mode, dmoe_layer **out)
{
    if (!ctx || !out) return DMOE_ERR_INVALID_ARG;
    *out = nullptr;
    if (!norm || !output) return set_err(ctx, DMOE_ERR_INVALID_ARG, "head: NULL tensor");
    const int H = n_embd, V = n_vocab;
    if (H <= 0 || H % 256) return set_err(ctx, DMOE_ERR_SHAPE, "head: n_embd = %d must be a positive multiple of 256", H);
    if (V <= 0) return set_err(ctx, DMOE_ERR_SHAPE, "head: n_vocab = %d", V);
    int rc;
    if ((rc = check_tensor(ctx, "output", *output, H, V, 0, device_mode))) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    dmoe_layer *L = new (std::nothrow) dmoe_layer();
    if (!L) return set_err(ctx, DMOE_ERR_OOM, "host allocation failed");
    L->ctx = ctx;
    L->device = ctx->device;
    L->head = true;
    L->n_vocab = V;
    L->hp.n_embd = H;
    auto fail = [&](int code) {
        dmoe_layer_free(L);
        return code;
    };
    if ((rc = f32_vector(ctx, L, *norm, H, device_mode, "output_norm", &L->gate_w))) return fail(rc);
    if (device_mode)
        L->sd = wrap_tensor(*output);
    else if ((rc = upload_tensor(ctx, L, *output, V, 1, L->sd)))
        return fail(rc);
    if ((rc = tile_proj(ctx, L, L->sd, V, H))) return fail(rc);
    *out = L;
    return DMOE_OK;
}

int dmoe_head_upload(dmoe_ctx *ctx, int32_t n_embd, int32_t n_vocab, const dmoe_tensor *output_norm,
                     const dmoe_tensor *output, dmoe_layer **out)
{
    return head_create(ctx, n_embd, n_vocab, output_norm, output, false, out);
}

int dmoe_head_wrap_device(dmoe_ctx *ctx, int32_t n_embd, int32_t n_vocab, const dmoe_tensor *output_norm,
                          const dmoe_tensor *output, dmoe_layer **out)
{
    return head_create(ctx, n_embd, n_vocab, output_norm, output, true, out);
}

static int head_args(dmoe_ctx *ctx, const dmoe_layer *L, const void *h, int32_t n_tokens, const void *tokens,
                     const void *probs, float eps)
{
    if (!L || !L->head) return set_err(ctx, DMOE_ERR_INVALID_ARG, "not a head layer (dmoe_head_upload)");
    if (!h || !tokens || !probs || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "h/tokens/probs NULL or n_tokens = %d", n_tokens);
    if (!(eps >= 0.0f) || eps > 1.0f) return set_err(ctx, DMOE_ERR_INVALID_ARG, "eps = %g outside [0, 1]", (double)eps);
    return DMOE_OK;
}

int dmoe_head_forward(dmoe_ctx *ctx, const dmoe_layer *L, const float *h, int32_t n_tokens, float eps,
                      int32_t *tokens, float *probs, float *logits)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    int rc = head_args(ctx, L, h, n_tokens, tokens, probs, eps);
    if (rc) return rc;
    const int H = L->hp.n_embd, V = L->n_vocab;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    HeadWs w;
    if ((rc = ensure_head_workspace(ctx, L, n_tokens, true, true, &w))) return rc;
    hipStream_t s = ctx->stream;
    HIP_TRY(ctx, hipMemcpyAsync(w.h, h, (size_t)n_tokens * H * 4, hipMemcpyHostToDevice, s));
    if ((rc = enqueue_head(ctx, L, w, w.h, n_tokens, eps, w.tokens, w.probs, w.logits, s))) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(tokens, w.tokens, (size_t)n_tokens * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipMemcpyAsync(probs, w.probs, (size_t)n_tokens * 4, hipMemcpyDeviceToHost, s));
    if (logits)
        HIP_TRY(ctx, hipMemcpyAsync(logits, w.logits, (size_t)n_tokens * V * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return DMOE_OK;
}

int dmoe_head_forward_device(dmoe_ctx *ctx, const dmoe_layer *L, const float *h_dev, int32_t n_tokens,
                             float eps, int32_t *tokens_dev, float *probs_dev, float *logits_dev,
                             void *stream)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    int rc = head_args(ctx, L, h_dev, n_tokens, tokens_dev, probs_dev, eps);
    if (rc) return rc;
    if ((uintptr_t)h_dev % 16) return set_err(ctx, DMOE_ERR_INVALID_ARG, "h_dev must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    HeadWs w;
    if ((rc = ensure_head_workspace(ctx, L, n_tokens, false, logits_dev == nullptr, &w))) return rc;
    return enqueue_head(ctx, L, w, h_dev, n_tokens, eps, tokens_dev, probs_dev,
                        logits_dev ? logits_dev : w.logits, (hipStream_t)stream);
}

static int attn_create(dmoe_ctx *ctx, const dmoe_attn_hparams *ap, const dmoe_attn_desc *d, bool device_mode,
                       dmoe_layer **out)
{
    if (!ctx || !out) return DMOE_ERR_INVALID_ARG;
    *out = nullptr;
    if (!ap || !d) return set_err(ctx, DMOE_ERR_INVALID_ARG, "attn: hparams / desc is NULL");
    const dmoe_attn_hparams a = *ap;
    if (a.n_embd <= 0 || a.n_embd % 256) return set_err(ctx, DMOE_ERR_SHAPE, "attn: n_embd = %d must be a positive multiple of 256", a.n_embd);
    if (a.n_head <= 0 || a.n_head_kv <= 0 || a.n_head % a.n_head_kv)
        return set_err(ctx, DMOE_ERR_SHAPE, "attn: n_head = %d, n_head_kv = %d", a.n_head, a.n_head_kv);
    if (a.head_dim != 64 && a.head_dim != 128)
        return set_err(ctx, DMOE_ERR_SHAPE, "attn: head_dim = %d (64 or 128 supported)", a.head_dim);
    if (a.rotary_dim < 0 || a.rotary_dim > a.head_dim || a.rotary_dim % 2)
        return set_err(ctx, DMOE_ERR_SHAPE, "attn: rotary_dim = %d", a.rotary_dim);
    if (!(a.rms_eps >= 0.0f) || !(a.rope_base > 0.0f))
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "attn: rms_eps / rope_base out of range");
    const int H = a.n_embd, QD = a.n_head * a.head_dim, QKV = QD + 2 * a.n_head_kv * a.head_dim;
    if (QD % 256) return set_err(ctx, DMOE_ERR_SHAPE, "attn: n_head * head_dim = %d not a multiple of 256", QD);
    int rc;
    if ((rc = check_tensor(ctx, "attn_qkv", d->qkv, H, QKV, 0, device_mode))) return rc;
    if ((rc = check_tensor(ctx, "attn_output", d->wo, QD, H, 0, device_mode))) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    dmoe_layer *L = new (std::nothrow) dmoe_layer();
    if (!L) return set_err(ctx, DMOE_ERR_OOM, "host allocation failed");
    L->ctx = ctx;
    L->device = ctx->device;
    L->attn = true;
    L->ahp = a;
    L->hp.n_embd = H;
    auto fail = [&](int code) {
        dmoe_layer_free(L);
        return code;
    };
    if ((rc = f32_vector(ctx, L, d->attn_norm, H, device_mode, "attn_norm", &L->attn_norm))) return fail(rc);
    if (d->post_attn_norm.data &&
        (rc = f32_vector(ctx, L, d->post_attn_norm, H, device_mode, "post_attn_norm", &L->post_norm)))
        return fail(rc);
    if (a.use_qk_norm) {
        if ((rc = f32_vector(ctx, L, d->q_norm, a.head_dim, device_mode, "attn_q_norm", &L->qn))) return fail(rc);
        if ((rc = f32_vector(ctx, L, d->k_norm, a.head_dim, device_mode, "attn_k_norm", &L->kn))) return fail(rc);
    }
    if (device_mode) {
        L->aqkv = wrap_tensor(d->qkv);
        L->awo = wrap_tensor(d->wo);
    } else if ((rc = upload_tensor(ctx, L, d->qkv, QKV, 1, L->aqkv)) ||
               (rc = upload_tensor(ctx, L, d->wo, H, 1, L->awo))) {
        return fail(rc);
    }
    if ((rc = tile_proj(ctx, L, L->aqkv, QKV, H)) || (rc = tile_proj(ctx, L, L->awo, H, QD))) return fail(rc);
    *out = L;
    return DMOE_OK;
}

int dmoe_attn_upload(dmoe_ctx *ctx, const dmoe_attn_hparams *ap, const dmoe_attn_desc *desc, dmoe_layer **out)
{
    return attn_create(ctx, ap, desc, false, out);
}

int dmoe_attn_wrap_device(dmoe_ctx *ctx, const dmoe_attn_hparams *ap, const dmoe_attn_desc *desc,
                          dmoe_layer **out)
{
    return attn_create(ctx, ap, desc, true, out);
}

int dmoe_attn_forward(dmoe_ctx *ctx, const dmoe_layer *L, const float *h, int32_t n_tokens, float *h_out,
                      float *moe_in)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (!L || !L->attn) return set_err(ctx, DMOE_ERR_INVALID_ARG, "not an attention layer (dmoe_attn_upload)");
    if (!h || !h_out || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "h/h_out NULL or n_tokens = %d", n_tokens);
    const int H = L->ahp.n_embd;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    int rc = grow_workspace(ctx, plan_attn(ctx->sw, L, n_tokens, true, nullptr, nullptr));
    if (rc) return rc;
    AttnWs w;
    plan_attn(ctx->sw, L, n_tokens, true, (uint8_t *)ctx->ws, &w);
    hipStream_t s = ctx->stream;
    HIP_TRY(ctx, hipMemcpyAsync(w.h, h, (size_t)n_tokens * H * 4, hipMemcpyHostToDevice, s));
    if ((rc = enqueue_attn(ctx, L, w, w.h, n_tokens, w.h_out, moe_in ? w.moe_in : nullptr, s))) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(h_out, w.h_out, (size_t)n_tokens * H * 4, hipMemcpyDeviceToHost, s));
    if (moe_in) HIP_TRY(ctx, hipMemcpyAsync(moe_in, w.moe_in, (size_t)n_tokens * H * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return DMOE_OK;
}

int dmoe_attn_forward_device(dmoe_ctx *ctx, const dmoe_layer *L, const float *h_dev, int32_t n_tokens,
                             float *h_out_dev, float *moe_in_dev, void *stream)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (!L || !L->attn) return set_err(ctx, DMOE_ERR_INVALID_ARG, "not an attention layer (dmoe_attn_upload)");
    if (!h_dev || !h_out_dev || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "h/h_out NULL or n_tokens = %d", n_tokens);
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(h_dev) || !al16(h_out_dev) || (moe_in_dev && !al16(moe_in_dev)))
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "device buffers must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    int rc = grow_workspace(ctx, plan_attn(ctx->sw, L, n_tokens, false, nullptr, nullptr));
    if (rc) return rc;
    AttnWs w;
    plan_attn(ctx->sw, L, n_tokens, false, (uint8_t *)ctx->ws, &w);
    return enqueue_attn(ctx, L, w, h_dev, n_tokens, h_out_dev, moe_in_dev, (hipStream_t)stream);
}

int dmoe_dense_upload(dmoe_ctx *ctx, int32_t n_embd, int32_t n_ff, const dmoe_tensor *gate,
                      const dmoe_tensor *up, const dmoe_tensor *down, dmoe_layer **out)
{
    return dense_create(ctx, n_embd, n_ff, gate, up, down, false, out);
}

int dmoe_dense_wrap_device(dmoe_ctx *ctx, int32_t n_embd, int32_t n_ff, const dmoe_tensor *gate,
                           const dmoe_tensor *up, const dmoe_tensor *down, dmoe_layer **out)
{
    return dense_create(ctx, n_embd, n_ff, gate, up, down, true, out);
}

void dmoe_layer_free(dmoe_layer *L)
{
    if (!L) return;
    // the layer keeps its own device id: freeing it after its context was
    // destroyed touches nothing of the context
    (void)hipSetDevice(L->device);
    for (void *p : L->owned) (void)hipFree(p);
    delete L;
}

int dmoe_layer_kernel_path(const dmoe_layer *L)
{
    if (!L) return -1;
    static const int kmap[] = {DMOE_PATH_GEMV, DMOE_PATH_Q4K_MFMA, DMOE_PATH_Q80_MFMA, DMOE_PATH_F16_GEMM,
                               DMOE_PATH_Q6K_MFMA};
    if (L->dense) return kmap[dense_path(L->sg.type, L->hp.n_embd, L->hp.shared_ff)];
    if (L->head) return kmap[head_path(L->sd.type, L->n_vocab, L->hp.n_embd)];
    if (L->attn) {
        const int QD = L->ahp.n_head * L->ahp.head_dim, QKV = QD + 2 * L->ahp.n_head_kv * L->ahp.head_dim;
        return kmap[head_path(L->aqkv.type, QKV, L->ahp.n_embd)];
    }
    if (use_mfma_path(L->hp, L->eg.type, L->sg.type, L->has_shared)) return DMOE_PATH_Q4K_MFMA;
    if (use_q80_path(L->hp, L->eg.type, L->sg.type, L->has_shared)) return DMOE_PATH_Q80_MFMA;
    if (use_gemm_path(L->hp, L->eg.type, L->sg.type, L->has_shared)) return DMOE_PATH_F16_GEMM;
    return DMOE_PATH_GEMV;
}

int dmoe_layer_forward(dmoe_ctx *ctx, const dmoe_layer *L, const float *x, int32_t n_tokens,
                       float *y, dmoe_debug *dbg)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (L && (L->head || L->attn))
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "not a MoE / dense layer (a step-tail or attention layer)");
    if (!L || !x || !y || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "layer/x/y NULL or n_tokens = %d", n_tokens);
    const int H = L->hp.n_embd;
    for (size_t i = 0; i < (size_t)n_tokens * H; i++)
        if (!std::isfinite(x[i]))
            return set_err(ctx, DMOE_ERR_NONFINITE, "x[%zu] = %g is not finite", i, (double)x[i]);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (L->dense) {
        DenseWs dw;
        int rc = ensure_dense_workspace(ctx, L, n_tokens, true, &dw);
        if (rc) return rc;
        hipStream_t s = ctx->stream;
        HIP_TRY(ctx, hipMemcpyAsync(dw.x, x, (size_t)n_tokens * H * 4, hipMemcpyHostToDevice, s));
        if ((rc = enqueue_dense(ctx, L, dw, dw.x, n_tokens, dw.y, s, ctx->prof))) return rc;
        HIP_TRY(ctx, hipMemcpyAsync(y, dw.y, (size_t)n_tokens * H * 4, hipMemcpyDeviceToHost, s));
        if (dbg && dbg->use_block_routing) *dbg->use_block_routing = 0;
        HIP_TRY(ctx, hipStreamSynchronize(s));
        return DMOE_OK;
    }
    Workspace w;
    int rc = ensure_workspace(ctx, L, n_tokens, true, &w);
    if (rc) return rc;
    hipStream_t s = ctx->stream;
    HIP_TRY(ctx, hipMemcpyAsync(w.x, x, (size_t)n_tokens * H * 4, hipMemcpyHostToDevice, s));
    if ((rc = enqueue_forward(ctx, L, w, w.x, n_tokens, w.y, s, ctx->prof))) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(y, w.y, (size_t)n_tokens * H * 4, hipMemcpyDeviceToHost, s));
    if ((rc = copy_debug(ctx, L->hp, w, n_tokens, dbg, s))) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return DMOE_OK;
}

int dmoe_layer_forward_device(dmoe_ctx *ctx, const dmoe_layer *L, const float *x_dev,
                              int32_t n_tokens, float *y_dev, void *stream)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (L && (L->head || L->attn))
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "not a MoE / dense layer (a step-tail or attention layer)");
    if (!L || !x_dev || !y_dev || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "layer/x/y NULL or n_tokens = %d", n_tokens);
    if ((uintptr_t)x_dev % 16)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "x_dev must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (L->dense) {
        DenseWs dw;
        int rc = ensure_dense_workspace(ctx, L, n_tokens, false, &dw);
        if (rc) return rc;
        return enqueue_dense(ctx, L, dw, x_dev, n_tokens, y_dev, (hipStream_t)stream, ctx->prof);
    }
    Workspace w;
    int rc = ensure_workspace(ctx, L, n_tokens, false, &w);
    if (rc) return rc;
    return enqueue_forward(ctx, L, w, x_dev, n_tokens, y_dev, (hipStream_t)stream, ctx->prof);
}

int dmoe_layer_forward_device_noalloc(dmoe_ctx *ctx, const dmoe_layer *L, const float *x_dev,
                                      int32_t n_tokens, float *y_dev, void *stream)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (L && (L->head || L->attn))
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "not a MoE / dense layer (a step-tail or attention layer)");
    if (!L || !x_dev || !y_dev || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "layer/x/y NULL or n_tokens = %d", n_tokens);
    if ((uintptr_t)x_dev % 16)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "x_dev must be 16-byte aligned");
    if (L->device != ctx->device)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "layer lives on device %d, context on %d",
                       L->device, ctx->device);
    if (!ctx->scratch)
        return set_err(ctx, DMOE_ERR_HIP, "scratch address of device %d not resolved", ctx->device);
    const size_t need = L->dense ? plan_dense(ctx->sw, L, n_tokens, false, nullptr, nullptr)
                                 : plan_workspace(ctx->sw, L->hp, L->eg.type, L->sg.type, L->has_shared, n_tokens,
                                                  false, nullptr, nullptr);
    if (need > DMOE_NOALLOC_SCRATCH_BYTES)
        return set_err(ctx, DMOE_ERR_INVALID_ARG,
                       "n_tokens = %d needs %zu bytes of workspace, above the %zu-byte scratch of "
                       "the allocation-free forward (use dmoe_layer_forward_device)",
                       n_tokens, need, (size_t)DMOE_NOALLOC_SCRATCH_BYTES);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    // Every workspace buffer is written by the forward before it is read, so
    // what a previous call left in the scratch needs no clearing.
    if (L->dense) {
        DenseWs dw;
        plan_dense(ctx->sw, L, n_tokens, false, ctx->scratch, &dw);
        return enqueue_dense(ctx, L, dw, x_dev, n_tokens, y_dev, (hipStream_t)stream, false);
    }
    Workspace w;
    plan_workspace(ctx->sw, L->hp, L->eg.type, L->sg.type, L->has_shared, n_tokens, false, ctx->scratch, &w);
    return enqueue_forward(ctx, L, w, x_dev, n_tokens, y_dev, (hipStream_t)stream, false);
}

int dmoe_route_logits(dmoe_ctx *ctx, const dmoe_hparams *hp, const float *bias,
                      const float *logits, int32_t n_tokens, dmoe_debug *dbg)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (!hp || !logits || n_tokens <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "hparams/logits NULL or n_tokens = %d", n_tokens);
    const int E = hp->n_experts, K = hp->top_k;
    if (E <= 0 || E > 1024) return set_err(ctx, DMOE_ERR_SHAPE, "n_experts = %d outside 1..1024", E);
    if (K <= 0 || K > 32 || K > E)
        return set_err(ctx, DMOE_ERR_SHAPE, "top_k = %d outside 1..min(32, n_experts)", K);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    // a routing-only pseudo layer: smallest valid sizes for the expert buffers
    dmoe_layer L;
    L.hp = *hp;
    L.hp.n_embd = 256;
    L.hp.moe_ff = 32;
    L.eg.type = DMOE_TYPE_F32;
    Workspace w;
    int rc = ensure_workspace(ctx, &L, n_tokens, false, &w);
    if (rc) return rc;
    hipStream_t s = ctx->stream;
    HIP_TRY(ctx, hipMemcpyAsync(w.rb.logits, logits, (size_t)n_tokens * E * 4,
                                hipMemcpyHostToDevice, s));
    const float *dbias = nullptr;
    if (bias) {
        HIP_TRY(ctx, hipMemcpyAsync(w.bias, bias, (size_t)E * 4, hipMemcpyHostToDevice, s));
        dbias = w.bias;
    }
    RouteParams rp = route_params(nullptr, *hp, n_tokens);
    rp.bias = dbias;
    rp.bias_small = 1;
    if (bias)
        for (int e = 0; e < E; e++)
            if (!(std::fabs(bias[e]) < 1e19f)) rp.bias_small = 0;
    LAUNCH_TRY(ctx, launch_scores(w.rb.logits, dbias, n_tokens, E, w.rb, s));
    LAUNCH_TRY(ctx, launch_route(rp, w.rb, w.wl, s));
    dmoe_debug d2 = dbg ? *dbg : dmoe_debug{};
    d2.logits = nullptr;
    if ((rc = copy_debug(ctx, *hp, w, n_tokens, &d2, s))) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return DMOE_OK;
}

int dmoe_quantize_device(dmoe_ctx *ctx, int32_t type, const float *src_dev, void *dst_dev,
                         int64_t nrows, int64_t n_per_row, void *stream)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (!src_dev || !dst_dev || nrows <= 0 || n_per_row <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "quantize: NULL pointer or empty shape");
    if (!type_supported(type))
        return set_err(ctx, DMOE_ERR_UNSUPPORTED_TYPE, "quantize: unsupported type %d", type);
    if (row_bytes(type, n_per_row) == 0)
        return set_err(ctx, DMOE_ERR_SHAPE, "quantize: n_per_row = %lld not a block multiple",
                       (long long)n_per_row);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    LAUNCH_TRY(ctx, launch_quantize_weights(type, src_dev, dst_dev, nrows, n_per_row,
                                            (hipStream_t)stream));
    return DMOE_OK;
}

int dmoe_residual_rmsnorm(dmoe_ctx *ctx, float *h_dev, const float *y_dev, const float *gain_dev,
                          float *x_dev, int32_t n_rows, int32_t n_embd, float eps, void *stream)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    if (!h_dev || !x_dev || n_rows < 0 || n_embd <= 0)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "residual_rmsnorm: NULL pointer or empty shape");
    if (n_embd % 4)
        return set_err(ctx, DMOE_ERR_SHAPE, "residual_rmsnorm: n_embd = %d not a multiple of 4", n_embd);
    auto misaligned = [](const void *p) { return p && ((uintptr_t)p & 15) != 0; };
    if (misaligned(h_dev) || misaligned(y_dev) || misaligned(gain_dev) || misaligned(x_dev))
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "residual_rmsnorm: pointers must be 16-byte aligned");
    const size_t bytes = (size_t)n_rows * n_embd * 4;
    const uintptr_t h0 = (uintptr_t)h_dev, x0 = (uintptr_t)x_dev;
    if (n_rows > 0 && h0 < x0 + bytes && x0 < h0 + bytes)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "residual_rmsnorm: h and x overlap");
    if (!(eps >= 0.0f) || eps > 1.0f)
        return set_err(ctx, DMOE_ERR_INVALID_ARG, "residual_rmsnorm: eps = %g outside [0, 1]", (double)eps);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    LAUNCH_TRY(ctx, launch_residual_rmsnorm(h_dev, y_dev, gain_dev, x_dev, n_rows, n_embd, eps,
                                            (hipStream_t)stream));
    return DMOE_OK;
}

int dmoe_profile_enable(dmoe_ctx *ctx, int enable)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    ctx->prof = enable != 0;
    return DMOE_OK;
}

int dmoe_profile_read(dmoe_ctx *ctx, float *total_ms, int32_t *calls)
{
    if (!ctx) return DMOE_ERR_INVALID_ARG;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (total_ms) for (int i = 0; i < DMOE_N_STAGES; i++) total_ms[i] = 0.0f;
    if (calls) for (int i = 0; i < DMOE_N_STAGES; i++) calls[i] = 0;
    int rc = DMOE_OK;
    for (auto &m : ctx->marks) {
        float ms = 0.0f;
        hipError_t e = hipEventSynchronize(m.b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, m.a, m.b);
        if (e != hipSuccess && rc == DMOE_OK)
            rc = set_err(ctx, DMOE_ERR_HIP, "profile event: %s", hipGetErrorString(e));
        if (total_ms) total_ms[m.stage] += ms;
        if (calls) calls[m.stage] += 1;
        ctx->pool.push_back(m.a);
        ctx->pool.push_back(m.b);
    }
    ctx->marks.clear();
    return rc;
}

const char *dmoe_stage_name(int stage)
{
    return (stage >= 0 && stage < DMOE_N_STAGES) ? kStageNames[stage] : "";
}

} // extern "C"
