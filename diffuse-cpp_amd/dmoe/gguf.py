"""ctypes mirror of the GGUF entry points of include/dmoe.h (dmoe_gguf_*).

    g = dmoe.gguf.GGUF("model.gguf")
    hp, n_layer, first_k = g.moe_hparams()
    w = g.layer_weights(il)           # LayerWeights of numpy views onto the file
    layer = ctx.upload(w)             # dmoe_layer_upload straight from the mapping

The tensors are memory-mapped read-only.  The arrays layer_weights,
dense_weights and attn_weights return are views of that mapping, and each
view keeps the mapping alive: close() (or dropping the GGUF object) releases
the file once no view of it remains.  Every view is sized from its tensor's
own ne (bounds-checked against the file by the C reader) and must agree with
the hyper-parameters, or DmoeError(DMOE_ERR_SHAPE) is raised.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import AttnWeights, DenseWeights, DmoeError, HeadWeights, LayerWeights, load
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


class _Mapping:
    """Owner of one dmoe_gguf handle: the file stays mapped while this object
    lives, and the views hold a reference to it."""

    def __init__(self, lib, handle):
        self.lib, self.handle = lib, handle

    def __del__(self):
        h, self.handle = self.handle, None
        if h:
            self.lib.dmoe_gguf_close(h)


def _ne(t: Tensor, nd: int):
    return tuple(int(t.ne[i]) for i in range(nd))


def _expect(name: str, t: Tensor, ne: tuple):
    """Refuse a tensor whose own ne disagrees with what the hyper-parameters
    say it holds (the view would otherwise reach past the tensor)."""
    got = _ne(t, 4)
    want = tuple(ne) + (1,) * (4 - len(ne))
    if got != want:
        raise DmoeError(3, "%s: ne %s in the file, %s expected from the hyper-parameters" % (name, list(got), list(want)))


def _view(owner: _Mapping, t: Tensor, nbytes: int) -> np.ndarray:
    """u8 view of nbytes at the tensor's data, keeping the mapping alive."""
    buf = (C.c_uint8 * nbytes).from_address(t.data)
    buf._owner = owner          # np.frombuffer keeps buf, buf keeps the mapping
    return np.frombuffer(buf, dtype=np.uint8)


def _bytes_view(owner: _Mapping, t: Tensor) -> np.ndarray:
    """u8 [rows, row bytes] view of a tensor, rows = ne1 ne2 ne3 of its own ne."""
    rb = row_size(t.type, t.ne[0])
    rows = int(t.ne[1]) * int(t.ne[2]) * int(t.ne[3])
    return _view(owner, t, rb * rows).reshape(rows, rb)


def _f32_view(owner: _Mapping, t: Tensor, what: str) -> np.ndarray:
    if t.type != 0:
        raise DmoeError(2, "%s of type %d (F32 expected here)" % (what, t.type))
    n = int(t.ne[0]) * int(t.ne[1]) * int(t.ne[2]) * int(t.ne[3])
    return _view(owner, t, 4 * n).view(np.float32)


class GGUF:
    def __init__(self, path):
        self.lib = _bind(load())
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = self.lib.dmoe_gguf_open(str(path).encode(), C.byref(h), err, len(err))
        if rc:
            raise DmoeError(rc, err.value.decode())
        self._map = _Mapping(self.lib, h.value)

    @property
    def handle(self):
        m = getattr(self, "_map", None)
        if m is None:
            raise DmoeError(1, "GGUF file already closed")
        return m.handle

    def close(self):
        """Drop this object's hold on the mapping; views made earlier keep it
        mapped until they are gone."""
        self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

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
        m = self._map
        _expect("moe_gate", d.gate_w, (H, E))
        gate_w = _f32_view(m, d.gate_w, "router weight").reshape(E, H)
        bias = None
        if d.gate_bias.data:
            _expect("moe_gate_bias", d.gate_bias, (E,))
            bias = _f32_view(m, d.gate_bias, "router bias")
        _expect("moe_experts_gate", d.exp_gate, (H, FF, E))
        _expect("moe_experts_up", d.exp_up, (H, FF, E))
        _expect("moe_experts_down", d.exp_down, (FF, H, E))
        w = LayerWeights(n_embd=H, n_experts=E, top_k=hp.top_k, capacity=hp.capacity,
                         block_size=hp.block_size, moe_ff=FF, wtype=d.exp_gate.type, gate_w=gate_w,
                         exp_gate=_bytes_view(m, d.exp_gate).reshape(E, FF, -1),
                         exp_up=_bytes_view(m, d.exp_up).reshape(E, FF, -1),
                         exp_down=_bytes_view(m, d.exp_down).reshape(E, H, -1), gate_bias=bias,
                         norm_topk_prob=hp.norm_topk_prob, routed_scaling=hp.routed_scaling)
        if d.sh_gate.data and hp.n_shared > 0:
            SF = hp.shared_ff
            _expect("moe_shared_gate", d.sh_gate, (H, SF))
            _expect("moe_shared_up", d.sh_up, (H, SF))
            _expect("moe_shared_down", d.sh_down, (SF, H))
            w.n_shared, w.shared_ff, w.stype = 1, SF, d.sh_gate.type
            w.sh_gate = _bytes_view(m, d.sh_gate)
            w.sh_up = _bytes_view(m, d.sh_up)
            w.sh_down = _bytes_view(m, d.sh_down)
        return w

    def dense_weights(self, il: int) -> DenseWeights:
        g, u, dn = Tensor(), Tensor(), Tensor()
        nff = C.c_int32()
        self._check(self.lib.dmoe_gguf_dense_desc(self.handle, il, C.byref(g), C.byref(u), C.byref(dn),
                                                  C.byref(nff)), f"dense layer {il}")
        H, FF = int(g.ne[0]), nff.value
        _expect("ffn_gate", g, (H, FF))
        _expect("ffn_up", u, (H, FF))
        _expect("ffn_down", dn, (FF, H))
        m = self._map
        return DenseWeights(n_embd=H, n_ff=FF, wtype=g.type, gate=_bytes_view(m, g),
                            up=_bytes_view(m, u), down=_bytes_view(m, dn))

    def head_weights(self) -> HeadWeights:
        """The step tail's tensors as a HeadWeights of views onto the file:
        output_norm.weight, and output.weight or, when the file has none (tied
        embeddings), token_embd.weight (src/diffuse-model.cpp:129-138)."""
        m = self._map
        norm = self.tensor("output_norm.weight")
        try:
            out = self.tensor("output.weight")
        except DmoeError as e:
            if e.code != 8:
                raise
            out = self.tensor("token_embd.weight")
        H, V = int(out.ne[0]), int(out.ne[1])
        _expect("output_norm", norm, (H,))
        _expect("output", out, (H, V))
        return HeadWeights(n_embd=H, n_vocab=V, wtype=out.type, norm=_f32_view(m, norm, "output norm"),
                           output=_bytes_view(m, out))

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
        H, HD = a.n_embd, a.head_dim
        QD, QKV = a.n_head * HD, (a.n_head + 2 * a.n_head_kv) * HD
        _expect("attn_norm", d.attn_norm, (H,))
        _expect("attn_qkv", d.qkv, (H, QKV))
        _expect("attn_output", d.wo, (QD, H))
        _expect("post_attn_norm", d.post_attn_norm, (H,))
        if a.use_qk_norm:
            _expect("attn_q_norm", d.q_norm, (HD,))
            _expect("attn_k_norm", d.k_norm, (HD,))
        m = self._map
        return AttnWeights(n_embd=H, n_head=a.n_head, n_head_kv=a.n_head_kv, head_dim=HD,
                           rotary_dim=a.rotary_dim, block_length=a.block_length, rope_base=a.rope_base,
                           rms_eps=a.rms_eps, wtype=d.qkv.type, attn_norm=_f32_view(m, d.attn_norm, "norm weight"),
                           qkv=_bytes_view(m, d.qkv), wo=_bytes_view(m, d.wo),
                           post_norm=_f32_view(m, d.post_attn_norm, "norm weight"),
                           q_norm=_f32_view(m, d.q_norm, "norm weight") if a.use_qk_norm else None,
                           k_norm=_f32_view(m, d.k_norm, "norm weight") if a.use_qk_norm else None)
