"""Host-side Python mirror of the dmoe C ABI (include/dmoe.h).

The MoE segment of src/diffuse-moe-graph.cpp:188-289 runs in libdmoe.so (HIP
kernels for gfx950); this module only marshals pointers and shapes through
ctypes.  There is no Python or CPU compute path: if the library is missing
the import of the entry points fails loudly.

    ctx = dmoe.Context(0)
    layer = ctx.upload(weights)              # weights: LayerWeights (host)
    y, dbg = ctx.forward(layer, x, debug=True)
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np

from ._abi import (AttnDesc, AttnHParams, Debug, HParams, LayerDesc, Tensor, TYPE_F16, TYPE_F32, TYPE_Q4_K,
                   TYPE_Q8_0, TYPE_Q8_K, TYPE_NAMES, TYPE_BY_NAME, row_size, block_elems,
                   block_bytes)
from . import _abi

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "libdmoe.so"

EXPORTS = ("dmoe_create", "dmoe_destroy", "dmoe_last_error", "dmoe_layer_upload",
           "dmoe_layer_wrap_device", "dmoe_layer_free", "dmoe_layer_forward",
           "dmoe_layer_forward_device", "dmoe_route_logits", "dmoe_row_size",
           "dmoe_quantize_device", "dmoe_residual_rmsnorm", "dmoe_profile_enable",
           "dmoe_profile_read", "dmoe_stage_name", "dmoe_layer_kernel_path",
           "dmoe_layer_forward_device_noalloc", "dmoe_dense_upload", "dmoe_dense_wrap_device",
           "dmoe_gguf_open", "dmoe_gguf_close", "dmoe_gguf_get_u32", "dmoe_gguf_get_f32",
           "dmoe_gguf_find_tensor", "dmoe_gguf_tensor_count", "dmoe_gguf_tensor_name",
           "dmoe_gguf_moe_hparams", "dmoe_gguf_layer_desc", "dmoe_gguf_dense_desc",
           "dmoe_head_upload", "dmoe_head_wrap_device", "dmoe_head_forward", "dmoe_head_forward_device",
           "dmoe_attn_upload", "dmoe_attn_wrap_device", "dmoe_attn_forward", "dmoe_attn_forward_device",
           "dmoe_gguf_attn_hparams", "dmoe_gguf_attn_desc")
NOALLOC_SCRATCH_BYTES = 64 << 20
N_STAGES = 10
PATH_NAMES = {0: "gemv", 1: "q4k_mfma", 2: "q80_mfma", 3: "f16_gemm", 4: "q6k_mfma", -1: "none"}


class DmoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"dmoe error {code}: {msg}")
        self.code = code


_lib = None


def load() -> C.CDLL:
    """Load libdmoe.so (built in-tree by diffuse-cpp_amd/build.py)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} is not built; run diffuse-cpp_amd/build.py")
    # torch wheels ship their own HIP runtime (same soname libamdhip64.so.7 as
    # /opt/rocm's).  Loading torch first lets libdmoe bind to that already
    # loaded runtime; the other order would put two HIP/HSA runtimes in one
    # process and the second cannot open the device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(LIB_PATH))
    P = C.c_void_p
    lib.dmoe_create.argtypes = [C.c_int, C.POINTER(P)]
    lib.dmoe_destroy.argtypes = [P]
    lib.dmoe_destroy.restype = None
    lib.dmoe_last_error.argtypes = [P]
    lib.dmoe_last_error.restype = C.c_char_p
    lib.dmoe_layer_upload.argtypes = [P, C.POINTER(HParams), C.POINTER(LayerDesc), C.POINTER(P)]
    lib.dmoe_layer_wrap_device.argtypes = [P, C.POINTER(HParams), C.POINTER(LayerDesc),
                                           C.POINTER(P)]
    lib.dmoe_layer_free.argtypes = [P]
    lib.dmoe_layer_free.restype = None
    lib.dmoe_layer_kernel_path.argtypes = [P]
    lib.dmoe_dense_upload.argtypes = [P, C.c_int32, C.c_int32, C.POINTER(Tensor), C.POINTER(Tensor),
                                      C.POINTER(Tensor), C.POINTER(P)]
    lib.dmoe_dense_wrap_device.argtypes = lib.dmoe_dense_upload.argtypes
    lib.dmoe_head_upload.argtypes = [P, C.c_int32, C.c_int32, C.POINTER(Tensor), C.POINTER(Tensor),
                                     C.POINTER(P)]
    lib.dmoe_head_wrap_device.argtypes = lib.dmoe_head_upload.argtypes
    lib.dmoe_head_forward.argtypes = [P, P, P, C.c_int32, C.c_float, P, P, P]
    lib.dmoe_head_forward_device.argtypes = [P, P, P, C.c_int32, C.c_float, P, P, P, P]
    lib.dmoe_attn_upload.argtypes = [P, C.POINTER(AttnHParams), C.POINTER(AttnDesc), C.POINTER(P)]
    lib.dmoe_attn_wrap_device.argtypes = lib.dmoe_attn_upload.argtypes
    lib.dmoe_attn_forward.argtypes = [P, P, P, C.c_int32, P, P]
    lib.dmoe_attn_forward_device.argtypes = [P, P, P, C.c_int32, P, P, P]
    lib.dmoe_layer_forward.argtypes = [P, P, P, C.c_int32, P, C.POINTER(Debug)]
    lib.dmoe_layer_forward_device.argtypes = [P, P, P, C.c_int32, P, P]
    lib.dmoe_layer_forward_device_noalloc.argtypes = [P, P, P, C.c_int32, P, P]
    lib.dmoe_route_logits.argtypes = [P, C.POINTER(HParams), P, P, C.c_int32, C.POINTER(Debug)]
    lib.dmoe_row_size.argtypes = [C.c_int32, C.c_int64]
    lib.dmoe_row_size.restype = C.c_size_t
    lib.dmoe_quantize_device.argtypes = [P, C.c_int32, P, P, C.c_int64, C.c_int64, P]
    lib.dmoe_residual_rmsnorm.argtypes = [P, P, P, P, P, C.c_int32, C.c_int32, C.c_float, P]
    lib.dmoe_profile_enable.argtypes = [P, C.c_int]
    lib.dmoe_profile_read.argtypes = [P, P, P]
    lib.dmoe_stage_name.argtypes = [C.c_int]
    lib.dmoe_stage_name.restype = C.c_char_p
    _lib = lib
    return lib


def _ptr(a) -> int:
    if a is None:
        return 0
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return int(a.data_ptr())          # torch tensor


def tensor_view(ttype: int, data, ne, nb=None) -> Tensor:
    """dmoe_tensor for a contiguous tensor with ggml ne (ne[0] innermost)."""
    ne = list(ne) + [1] * (4 - len(ne))
    t = Tensor()
    t.type = ttype
    t.data = _ptr(data) or None
    for i in range(4):
        t.ne[i] = ne[i]
    if nb is None:
        shape = tuple(getattr(data, "shape", ()))
        is_bytes = str(getattr(data, "dtype", "")).endswith("uint8")
        # byte arrays carry their row size in the last dimension
        rs = int(shape[-1]) if is_bytes and shape else row_size(ttype, ne[0])
        b0 = block_bytes(ttype) if ttype in _abi.TYPE_NAMES else 1
        nb = [b0, rs, rs * ne[1], rs * ne[1] * ne[2]]
    for i in range(4):
        t.nb[i] = nb[i]
    return t


@dataclass
class LayerWeights:
    """One layer's MoE tensors as GGUF block bytes.

    Arrays are numpy (host) or torch (device) buffers:
      gate_w    f32 [E, H]                    (ggml ne [H, E])
      gate_bias f32 [E] or None
      exp_gate, exp_up  u8 [E, FF, row_size(T, H)]   (ne [H, FF, E])
      exp_down          u8 [E, H, row_size(T, FF)]   (ne [FF, H, E])
      sh_gate, sh_up    u8 [SF, row_size(Ts, H)] or None
      sh_down           u8 [H, row_size(Ts, SF)] or None
    """
    n_embd: int
    n_experts: int
    top_k: int
    capacity: int
    block_size: int
    moe_ff: int
    wtype: int
    gate_w: object
    exp_gate: object
    exp_up: object
    exp_down: object
    gate_bias: object = None
    n_shared: int = 0
    shared_ff: int = 0
    stype: int = TYPE_F32
    sh_gate: object = None
    sh_up: object = None
    sh_down: object = None
    norm_topk_prob: int = 1
    routed_scaling: float = 2.5
    extra: dict = field(default_factory=dict)

    def hparams(self) -> HParams:
        hp = HParams()
        hp.n_embd, hp.n_experts, hp.top_k = self.n_embd, self.n_experts, self.top_k
        hp.capacity, hp.block_size, hp.moe_ff = self.capacity, self.block_size, self.moe_ff
        hp.n_shared = self.n_shared if self.sh_gate is not None else 0
        hp.shared_ff = self.shared_ff
        hp.norm_topk_prob, hp.routed_scaling = self.norm_topk_prob, self.routed_scaling
        return hp

    def desc(self) -> LayerDesc:
        H, E, FF, SF = self.n_embd, self.n_experts, self.moe_ff, self.shared_ff
        d = LayerDesc()
        d.gate_w = tensor_view(TYPE_F32, self.gate_w, [H, E])
        if self.gate_bias is not None:
            d.gate_bias = tensor_view(TYPE_F32, self.gate_bias, [E])
        d.exp_gate = tensor_view(self.wtype, self.exp_gate, [H, FF, E])
        d.exp_up = tensor_view(self.wtype, self.exp_up, [H, FF, E])
        d.exp_down = tensor_view(self.wtype, self.exp_down, [FF, H, E])
        if self.sh_gate is not None:
            d.sh_gate = tensor_view(self.stype, self.sh_gate, [H, SF])
            d.sh_up = tensor_view(self.stype, self.sh_up, [H, SF])
            d.sh_down = tensor_view(self.stype, self.sh_down, [SF, H])
        return d

    def expert_bytes(self) -> int:
        """Bytes of gate+up+down of one routed expert."""
        return (2 * self.moe_ff * row_size(self.wtype, self.n_embd)
                + self.n_embd * row_size(self.wtype, self.moe_ff))

    def shared_bytes(self) -> int:
        if self.sh_gate is None:
            return 0
        return (2 * self.shared_ff * row_size(self.stype, self.n_embd)
                + self.n_embd * row_size(self.stype, self.shared_ff))


@dataclass
class DenseWeights:
    """The dense SwiGLU MLP of a first_k_dense layer (ffn_gate, ffn_up,
    ffn_down of diffuse_moe_layer, src/diffuse-common.h:67-70) as GGUF block
    bytes, numpy (host) or torch (device):
      gate, up  u8 [n_ff, row_size(T, n_embd)]   (ne [n_embd, n_ff])
      down      u8 [n_embd, row_size(T, n_ff)]   (ne [n_ff, n_embd])"""
    n_embd: int
    n_ff: int
    wtype: int
    gate: object
    up: object
    down: object

    def views(self):
        return (tensor_view(self.wtype, self.gate, [self.n_embd, self.n_ff]),
                tensor_view(self.wtype, self.up, [self.n_embd, self.n_ff]),
                tensor_view(self.wtype, self.down, [self.n_ff, self.n_embd]))

    def nbytes(self) -> int:
        return 2 * self.n_ff * row_size(self.wtype, self.n_embd) + self.n_embd * row_size(self.wtype, self.n_ff)


@dataclass
class HeadWeights:
    """The step tail's tensors (diffuse_model's output_norm and output,
    src/diffuse-common.h:94-96): norm f32 [n_embd] (numpy or torch), output
    GGUF block bytes u8 [n_vocab, row_size(T, n_embd)] (ne [n_embd, n_vocab])."""
    n_embd: int
    n_vocab: int
    wtype: int
    norm: object
    output: object

    def output_view(self) -> Tensor:
        return tensor_view(self.wtype, self.output, [self.n_embd, self.n_vocab])

    def norm_view(self) -> Tensor:
        return tensor_view(TYPE_F32, self.norm, [self.n_embd])


@dataclass
class AttnWeights:
    """The attention half of a layer (diffuse_moe_layer's attn_norm, wqkv,
    attn_q_norm, attn_k_norm, wo, attn_post_norm, src/diffuse-common.h:60-65)
    and its hyper-parameters.  Norms f32 (numpy or torch); qkv u8
    [(n_head + 2 n_head_kv) head_dim, row_size(T, n_embd)] (ne [n_embd,
    QKV]: rows Q then K then V); wo u8 [n_embd, row_size(T, n_head head_dim)]
    (ne [n_head head_dim, n_embd]).  q_norm / k_norm f32 [head_dim] or None."""
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    rotary_dim: int
    block_length: int
    rope_base: float
    rms_eps: float
    wtype: int
    attn_norm: object
    qkv: object
    wo: object
    post_norm: object
    q_norm: object = None
    k_norm: object = None

    @property
    def q_dim(self) -> int:
        return self.n_head * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return (self.n_head + 2 * self.n_head_kv) * self.head_dim

    def hparams(self) -> "AttnHParams":
        a = AttnHParams()
        a.n_embd, a.n_head, a.n_head_kv = self.n_embd, self.n_head, self.n_head_kv
        a.head_dim, a.rotary_dim = self.head_dim, self.rotary_dim
        a.use_qk_norm = int(self.q_norm is not None)
        a.block_length, a.rope_base, a.rms_eps = self.block_length, self.rope_base, self.rms_eps
        return a

    def desc(self) -> "AttnDesc":
        d = AttnDesc()
        d.attn_norm = tensor_view(TYPE_F32, self.attn_norm, [self.n_embd])
        d.qkv = tensor_view(self.wtype, self.qkv, [self.n_embd, self.qkv_dim])
        d.wo = tensor_view(self.wtype, self.wo, [self.q_dim, self.n_embd])
        if self.post_norm is not None:
            d.post_attn_norm = tensor_view(TYPE_F32, self.post_norm, [self.n_embd])
        if self.q_norm is not None:
            d.q_norm = tensor_view(TYPE_F32, self.q_norm, [self.head_dim])
            d.k_norm = tensor_view(TYPE_F32, self.k_norm, [self.head_dim])
        return d


def hparams_of(n_embd, n_experts, top_k, capacity, block_size, moe_ff=1, n_shared=0,
               shared_ff=0, norm_topk_prob=1, routed_scaling=2.5) -> HParams:
    hp = HParams()
    hp.n_embd, hp.n_experts, hp.top_k = n_embd, n_experts, top_k
    hp.capacity, hp.block_size, hp.moe_ff = capacity, block_size, moe_ff
    hp.n_shared, hp.shared_ff = n_shared, shared_ff
    hp.norm_topk_prob, hp.routed_scaling = norm_topk_prob, routed_scaling
    return hp


def use_block_routing(hp: HParams, n_tokens: int) -> bool:
    """src/diffuse-moe-graph.cpp:215-216"""
    return (hp.block_size > 1 and hp.capacity > 0 and hp.capacity < hp.n_experts
            and n_tokens % hp.block_size == 0)


class DebugOut:
    """Host buffers for dmoe_debug."""

    def __init__(self, hp: HParams, n_tokens: int):
        N, E, K = n_tokens, hp.n_experts, hp.top_k
        B = N // hp.block_size if use_block_routing(hp, N) else 0
        self.logits = np.zeros((N, E), np.float32)
        self.probs = np.zeros((N, E), np.float32)
        self.bmax = np.zeros((B, E), np.float32)
        self.thr = np.zeros((B,), np.float32)
        self.allowed = np.zeros((B, E), np.uint8)
        self.idx = np.zeros((N, K), np.int32)
        self.weights = np.zeros((N, K), np.float32)
        self.counts = np.zeros((E,), np.int32)
        self.offsets = np.zeros((E,), np.int32)
        self.perm = np.zeros((N * K,), np.int32)
        self.use_block = np.zeros((1,), np.int32)

    def struct(self) -> Debug:
        d = Debug()
        for name in ("logits", "probs", "bmax", "thr", "allowed", "idx", "weights", "counts",
                     "offsets", "perm"):
            a = getattr(self, name)
            setattr(d, name, a.ctypes.data if a.size else None)
        d.use_block_routing = self.use_block.ctypes.data
        return d

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k in ("logits", "probs", "bmax", "thr", "allowed", "idx",
                                              "weights", "counts", "offsets", "perm")} | {
            "use_block_routing": bool(self.use_block[0])}


class Layer:
    def __init__(self, ctx: "Context", handle: int, weights: LayerWeights):
        self.ctx, self.handle, self.weights = ctx, handle, weights
        self.hp = weights.hparams()

    def kernel_path(self) -> str:
        """Expert kernels this layer runs (dmoe_layer_kernel_path)."""
        return PATH_NAMES[load().dmoe_layer_kernel_path(self.handle)]

    def free(self):
        if self.handle:
            load().dmoe_layer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    def __init__(self, device: int = 0):
        lib = load()
        h = C.c_void_p()
        rc = lib.dmoe_create(device, C.byref(h))
        if rc:
            raise DmoeError(rc, f"dmoe_create({device}) failed")
        self.handle = h.value
        self.device = device

    def _check(self, rc: int):
        if rc:
            raise DmoeError(rc, load().dmoe_last_error(self.handle).decode())

    def last_error(self) -> str:
        return load().dmoe_last_error(self.handle).decode()

    def close(self):
        if getattr(self, "handle", None):
            load().dmoe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, w: LayerWeights, hp: Optional[HParams] = None,
               desc: Optional[LayerDesc] = None) -> Layer:
        """Copy w into HBM.  hp / desc override the structs built from w."""
        hp = w.hparams() if hp is None else hp
        d = w.desc() if desc is None else desc
        out = C.c_void_p()
        self._check(load().dmoe_layer_upload(self.handle, C.byref(hp), C.byref(d), C.byref(out)))
        return Layer(self, out.value, w)

    def wrap_device(self, w: LayerWeights) -> Layer:
        hp, d = w.hparams(), w.desc()
        out = C.c_void_p()
        self._check(load().dmoe_layer_wrap_device(self.handle, C.byref(hp), C.byref(d),
                                                  C.byref(out)))
        return Layer(self, out.value, w)

    def _dense(self, fn, w: DenseWeights) -> Layer:
        g, u, d = w.views()
        out = C.c_void_p()
        self._check(fn(self.handle, w.n_embd, w.n_ff, C.byref(g), C.byref(u), C.byref(d),
                       C.byref(out)))
        lw = LayerWeights(n_embd=w.n_embd, n_experts=0, top_k=0, capacity=0, block_size=0,
                          moe_ff=w.n_ff, wtype=w.wtype, gate_w=None, exp_gate=None, exp_up=None,
                          exp_down=None)
        layer = Layer(self, out.value, lw)
        # in device mode the library keeps pointers into w's tensors
        layer.src = w
        return layer

    def dense_upload(self, w: DenseWeights) -> Layer:
        """Copy a dense MLP (host arrays) into HBM (dmoe_dense_upload)."""
        return self._dense(load().dmoe_dense_upload, w)

    def dense_wrap_device(self, w: DenseWeights) -> Layer:
        """A dense MLP whose tensors already live on the GPU (dmoe_dense_wrap_device)."""
        return self._dense(load().dmoe_dense_wrap_device, w)

    def _head(self, fn, w: "HeadWeights") -> Layer:
        nv, ov = w.norm_view(), w.output_view()
        out = C.c_void_p()
        self._check(fn(self.handle, w.n_embd, w.n_vocab, C.byref(nv), C.byref(ov), C.byref(out)))
        lw = LayerWeights(n_embd=w.n_embd, n_experts=0, top_k=0, capacity=0, block_size=0,
                          moe_ff=0, wtype=w.wtype, gate_w=None, exp_gate=None, exp_up=None,
                          exp_down=None)
        layer = Layer(self, out.value, lw)
        layer.n_vocab = w.n_vocab
        # in device mode the library keeps pointers into w's tensors (the
        # output norm, untiled weight types)
        layer.src = w
        return layer

    def head_upload(self, w: "HeadWeights") -> Layer:
        """The step tail (final norm + LM head) from host arrays (dmoe_head_upload)."""
        return self._head(load().dmoe_head_upload, w)

    def head_wrap_device(self, w: "HeadWeights") -> Layer:
        return self._head(load().dmoe_head_wrap_device, w)

    def head_forward(self, layer: Layer, h: np.ndarray, eps: float, logits: bool = False):
        """(tokens i32 [N], probs f32 [N][, logits f32 [N][V]]) for h [N][n_embd]."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        N = h.shape[0]
        tok = np.zeros(N, np.int32)
        prob = np.zeros(N, np.float32)
        lg = np.zeros((N, layer.n_vocab), np.float32) if logits else None
        self._check(load().dmoe_head_forward(self.handle, layer.handle, h.ctypes.data, N, float(eps),
                                             tok.ctypes.data, prob.ctypes.data,
                                             lg.ctypes.data if logits else None))
        return (tok, prob, lg) if logits else (tok, prob)

    def head_forward_device(self, layer: Layer, h_dev, n_tokens: int, eps: float, tokens_dev, probs_dev,
                            logits_dev=None, stream=None):
        s = 0 if stream is None else int(stream)
        self._check(load().dmoe_head_forward_device(self.handle, layer.handle, _ptr(h_dev), n_tokens,
                                                    float(eps), _ptr(tokens_dev), _ptr(probs_dev),
                                                    _ptr(logits_dev) if logits_dev is not None else None,
                                                    s or None))

    def _attn(self, fn, w: AttnWeights) -> Layer:
        a, d = w.hparams(), w.desc()
        out = C.c_void_p()
        self._check(fn(self.handle, C.byref(a), C.byref(d), C.byref(out)))
        lw = LayerWeights(n_embd=w.n_embd, n_experts=0, top_k=0, capacity=0, block_size=0,
                          moe_ff=0, wtype=w.wtype, gate_w=None, exp_gate=None, exp_up=None,
                          exp_down=None)
        layer = Layer(self, out.value, lw)
        layer.attn = w
        return layer

    def attn_upload(self, w: AttnWeights) -> Layer:
        """The attention half of a layer from host arrays (dmoe_attn_upload)."""
        return self._attn(load().dmoe_attn_upload, w)

    def attn_wrap_device(self, w: AttnWeights) -> Layer:
        return self._attn(load().dmoe_attn_wrap_device, w)

    def attn_forward(self, layer: Layer, h: np.ndarray):
        """(h + attention(h), post-attention norm of it) for h [N][n_embd]."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        N = h.shape[0]
        h_out = np.empty_like(h)
        moe_in = np.empty_like(h)
        self._check(load().dmoe_attn_forward(self.handle, layer.handle, h.ctypes.data, N,
                                             h_out.ctypes.data, moe_in.ctypes.data))
        return h_out, moe_in

    def attn_forward_device(self, layer: Layer, h_dev, n_tokens: int, h_out_dev, moe_in_dev=None,
                            stream=None):
        s = 0 if stream is None else int(stream)
        self._check(load().dmoe_attn_forward_device(self.handle, layer.handle, _ptr(h_dev), n_tokens,
                                                    _ptr(h_out_dev),
                                                    _ptr(moe_in_dev) if moe_in_dev is not None else None,
                                                    s or None))

    def forward(self, layer: Layer, x: np.ndarray, debug: bool = False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        N = x.shape[0]
        y = np.empty_like(x)
        dbg = DebugOut(layer.hp, N) if debug else None
        ds = dbg.struct() if dbg else None
        self._check(load().dmoe_layer_forward(self.handle, layer.handle, x.ctypes.data, N,
                                              y.ctypes.data, C.byref(ds) if ds else None))
        return (y, dbg.as_dict()) if debug else y

    def forward_device(self, layer: Layer, x_dev, n_tokens: int, y_dev, stream=None):
        s = 0 if stream is None else int(stream)
        self._check(load().dmoe_layer_forward_device(self.handle, layer.handle, _ptr(x_dev),
                                                     n_tokens, _ptr(y_dev), s or None))

    def forward_device_noalloc(self, layer: Layer, x_dev, n_tokens: int, y_dev, stream=None):
        """dmoe_layer_forward_device_noalloc: the same forward on the GPU's
        fixed scratch array, without any device allocation."""
        s = 0 if stream is None else int(stream)
        self._check(load().dmoe_layer_forward_device_noalloc(self.handle, layer.handle,
                                                             _ptr(x_dev), n_tokens, _ptr(y_dev),
                                                             s or None))

    def route_logits(self, hp: HParams, logits: np.ndarray, bias: Optional[np.ndarray]):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        N = logits.shape[0]
        dbg = DebugOut(hp, N)
        ds = dbg.struct()
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._check(load().dmoe_route_logits(self.handle, C.byref(hp),
                                             b.ctypes.data if b is not None else None,
                                             logits.ctypes.data, N, C.byref(ds)))
        return dbg.as_dict()

    def profile(self, enable: bool):
        self._check(load().dmoe_profile_enable(self.handle, 1 if enable else 0))

    def profile_read(self) -> dict:
        """{stage name: (total ms, launches)} since the last read."""
        ms = np.zeros(N_STAGES, np.float32)
        calls = np.zeros(N_STAGES, np.int32)
        self._check(load().dmoe_profile_read(self.handle, ms.ctypes.data, calls.ctypes.data))
        return {load().dmoe_stage_name(i).decode(): (float(ms[i]), int(calls[i]))
                for i in range(N_STAGES) if calls[i]}

    def residual_rmsnorm(self, h_dev, y_dev, x_dev, n_rows: int, n_embd: int, eps: float,
                         gain_dev=None, stream=None):
        """h += y (y_dev may be None), then x = rms_norm(h, eps) [* gain], on
        device tensors (src/diffuse-moe-graph.cpp:292, :175-178); queued on
        `stream` (None: the null stream)."""
        s = 0 if stream is None else int(stream)
        self._check(load().dmoe_residual_rmsnorm(
            self.handle, _ptr(h_dev), _ptr(y_dev) if y_dev is not None else None,
            _ptr(gain_dev) if gain_dev is not None else None, _ptr(x_dev), n_rows, n_embd,
            float(eps), s or None))

    def quantize_device(self, ttype: int, src_dev, dst_dev, nrows: int, n_per_row: int,
                        stream=None):
        s = 0 if stream is None else int(stream)
        self._check(load().dmoe_quantize_device(self.handle, ttype, _ptr(src_dev), _ptr(dst_dev),
                                                nrows, n_per_row, s or None))


__all__ = ["Context", "Layer", "LayerWeights", "DenseWeights", "HeadWeights", "AttnWeights", "DmoeError", "load", "tensor_view", "hparams_of",
           "use_block_routing", "row_size", "TYPE_F32", "TYPE_F16", "TYPE_Q8_0", "TYPE_Q4_K",
           "TYPE_Q8_K", "TYPE_NAMES", "TYPE_BY_NAME", "EXPORTS", "LIB_PATH"]
