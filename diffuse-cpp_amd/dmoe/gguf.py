"""ctypes mirror of the GGUF entry points of include/dmoe.h (dmoe_gguf_*).

    g = dmoe.gguf.GGUF("model.gguf")
    hp, n_layer, first_k = g.moe_hparams()
    w = g.layer_weights(il)           # LayerWeights of numpy views onto the file
    layer = ctx.upload(w)             # dmoe_layer_upload straight from the mapping

The tensors stay memory-mapped (read-only) until close(); the arrays
layer_weights / dense_weights return are views of that mapping.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import AttnWeights, DenseWeights, DmoeError, LayerWeights, load
from ._abi import AttnDesc, AttnHParams, HParams, LayerDesc, Tensor, row_size


def _bind(lib):
    if getattr(lib, "_gguf_bound", False):
        return lib
    P = C.c_void_p
    lib.dmoe_gguf_open.argtypes = [C.c_char_p, C.POINTER(P), C.c_char_p, C.c_size_t]
    lib.dmoe_gguf_close.argtypes = [P]
    lib.dmoe_gguf_close.restype = None
    lib.dmoe_gguf_get_u32.argtypes = [P, C.c_char_p, C.POINTER(C.c_uint32)]
    lib.dmoe_gguf_get_f32.argtypes = [P, C.c_char_p, C.POINTER(C.c_float)]
    lib.dmoe_gguf_find_tensor.argtypes = [P, C.c_char_p, C.POINTER(Tensor)]
    lib.dmoe_gguf_tensor_count.argtypes = [P]
    lib.dmoe_gguf_tensor_name.argtypes = [P, C.c_int]
    lib.dmoe_gguf_tensor_name.restype = C.c_char_p
    lib.dmoe_gguf_moe_hparams.argtypes = [P, C.POINTER(HParams), C.POINTER(C.c_int32),
                                          C.POINTER(C.c_int32)]
    lib.dmoe_gguf_layer_desc.argtypes = [P, C.c_int32, C.POINTER(LayerDesc)]
    lib.dmoe_gguf_dense_desc.argtypes = [P, C.c_int32, C.POINTER(Tensor), C.POINTER(Tensor),
                                         C.POINTER(Tensor), C.POINTER(C.c_int32)]
    lib.dmoe_gguf_attn_hparams.argtypes = [P, C.POINTER(AttnHParams)]
    lib.dmoe_gguf_attn_desc.argtypes = [P, C.c_int32, C.c_int32, C.POINTER(AttnDesc)]
    lib._gguf_bound = True
    return lib


def _bytes_view(t: Tensor, rows: int) -> np.ndarray:
    """u8 [rows, row bytes] view of a tensor in the mapping."""
    rb = row_size(t.type, t.ne[0])
    n = rb * rows
    buf = (C.c_uint8 * n).from_address(t.data)
    return np.frombuffer(buf, dtype=np.uint8).reshape(rows, rb)


class GGUF:
    def __init__(self, path):
        self.lib = _bind(load())
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = self.lib.dmoe_gguf_open(str(path).encode(), C.byref(h), err, len(err))
        if rc:
            raise DmoeError(rc, err.value.decode())
        self.handle = h.value

    def close(self):
        if getattr(self, "handle", None):
            self.lib.dmoe_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc:
            raise DmoeError(rc, what)

    def get_u32(self, suffix: str):
        v = C.c_uint32()
        rc = self.lib.dmoe_gguf_get_u32(self.handle, suffix.encode(), C.byref(v))
        return None if rc == 8 else (self._check(rc, suffix) or v.value)

    def get_f32(self, suffix: str):
        v = C.c_float()
        rc = self.lib.dmoe_gguf_get_f32(self.handle, suffix.encode(), C.byref(v))
        return None if rc == 8 else (self._check(rc, suffix) or v.value)

    def tensor(self, name: str) -> Tensor:
        t = Tensor()
        self._check(self.lib.dmoe_gguf_find_tensor(self.handle, name.encode(), C.byref(t)), name)
        return t

    def tensor_names(self):
        n = self.lib.dmoe_gguf_tensor_count(self.handle)
        return [self.lib.dmoe_gguf_tensor_name(self.handle, i).decode() for i in range(n)]

    def moe_hparams(self):
        hp = HParams()
        nl, fk = C.c_int32(), C.c_int32()
        self._check(self.lib.dmoe_gguf_moe_hparams(self.handle, C.byref(hp), C.byref(nl), C.byref(fk)),
                    "moe hparams")
        return hp, nl.value, fk.value

    def layer_desc(self, il: int) -> LayerDesc:
        d = LayerDesc()
        self._check(self.lib.dmoe_gguf_layer_desc(self.handle, il, C.byref(d)), f"layer {il}")
        return d

    def layer_weights(self, il: int) -> LayerWeights:
        """The MoE tensors of layer il as a LayerWeights of views onto the file."""
        hp, _, _ = self.moe_hparams()
        d = self.layer_desc(il)
        H, E, FF = hp.n_embd, hp.n_experts, hp.moe_ff
        gw = d.gate_w
        if gw.type != 0:
            raise DmoeError(2, "router weight of type %d (F32 expected here)" % gw.type)
        gate_w = np.frombuffer((C.c_uint8 * (4 * H * E)).from_address(gw.data), np.float32).reshape(E, H)
        bias = None
        if d.gate_bias.data:
            bias = np.frombuffer((C.c_uint8 * (4 * E)).from_address(d.gate_bias.data), np.float32)
        w = LayerWeights(n_embd=H, n_experts=E, top_k=hp.top_k, capacity=hp.capacity,
                         block_size=hp.block_size, moe_ff=FF, wtype=d.exp_gate.type, gate_w=gate_w,
                         exp_gate=_bytes_view(d.exp_gate, E * FF).reshape(E, FF, -1),
                         exp_up=_bytes_view(d.exp_up, E * FF).reshape(E, FF, -1),
                         exp_down=_bytes_view(d.exp_down, E * H).reshape(E, H, -1), gate_bias=bias,
                         norm_topk_prob=hp.norm_topk_prob, routed_scaling=hp.routed_scaling)
        if d.sh_gate.data and hp.n_shared > 0:
            SF = hp.shared_ff
            w.n_shared, w.shared_ff, w.stype = 1, SF, d.sh_gate.type
            w.sh_gate = _bytes_view(d.sh_gate, SF)
            w.sh_up = _bytes_view(d.sh_up, SF)
            w.sh_down = _bytes_view(d.sh_down, H)
        return w

    def dense_weights(self, il: int) -> DenseWeights:
        g, u, dn = Tensor(), Tensor(), Tensor()
        nff = C.c_int32()
        self._check(self.lib.dmoe_gguf_dense_desc(self.handle, il, C.byref(g), C.byref(u), C.byref(dn),
                                                  C.byref(nff)), f"dense layer {il}")
        H, FF = int(g.ne[0]), nff.value
        return DenseWeights(n_embd=H, n_ff=FF, wtype=g.type, gate=_bytes_view(g, FF),
                            up=_bytes_view(u, FF), down=_bytes_view(dn, H))

    def attn_hparams(self) -> AttnHParams:
        a = AttnHParams()
        self._check(self.lib.dmoe_gguf_attn_hparams(self.handle, C.byref(a)), "attention hparams")
        return a

    def attn_desc(self, il: int, use_qk_norm: bool) -> AttnDesc:
        d = AttnDesc()
        self._check(self.lib.dmoe_gguf_attn_desc(self.handle, il, int(use_qk_norm), C.byref(d)),
                    f"attention layer {il}")
        return d

    def attn_weights(self, il: int) -> AttnWeights:
        """The attention tensors of layer il as an AttnWeights of views onto the file."""
        a = self.attn_hparams()
        d = self.attn_desc(il, bool(a.use_qk_norm))
        QD, QKV = a.n_head * a.head_dim, (a.n_head + 2 * a.n_head_kv) * a.head_dim

        def f32(t, n):
            if t.type != 0:
                raise DmoeError(2, "norm weight of type %d (F32 expected here)" % t.type)
            return np.frombuffer((C.c_uint8 * (4 * n)).from_address(t.data), np.float32)
        return AttnWeights(n_embd=a.n_embd, n_head=a.n_head, n_head_kv=a.n_head_kv, head_dim=a.head_dim,
                           rotary_dim=a.rotary_dim, block_length=a.block_length, rope_base=a.rope_base,
                           rms_eps=a.rms_eps, wtype=d.qkv.type, attn_norm=f32(d.attn_norm, a.n_embd),
                           qkv=_bytes_view(d.qkv, QKV), wo=_bytes_view(d.wo, a.n_embd),
                           post_norm=f32(d.post_attn_norm, a.n_embd),
                           q_norm=f32(d.q_norm, a.head_dim) if a.use_qk_norm else None,
                           k_norm=f32(d.k_norm, a.head_dim) if a.use_qk_norm else None)
