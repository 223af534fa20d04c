"""A minimal GGUF (v3) writer for test fixtures, written from the container
layout as tools/quantize_streaming.py:13-88 reads it: magic "GGUF", u32
version, u64 tensor count, u64 key/value count, key/value pairs (u64-length
UTF-8 key, u32 value type, value), tensor infos (u64-length name, u32 n_dims,
n_dims x u64 ne, u32 ggml type, u64 offset from the data section), then the
data section starting at the first multiple of the alignment, each tensor's
data at an aligned offset.

Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
8 string, 9 array, 10 u64, 11 i64, 12 f64.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vtype], v)


class GGUFWriter:
    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self.kv: list[tuple[str, int, object]] = []
        self.tensors: list[tuple[str, int, list[int], bytes]] = []

    def add(self, key: str, vtype: int, value):
        self.kv.append((key, vtype, value))

    def add_tensor(self, name: str, ggml_type: int, ne, data):
        """ne in ggml order (ne[0] innermost); data: bytes or a numpy array."""
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        self.tensors.append((name, ggml_type, [int(x) for x in ne], raw))

    def header_bytes(self):
        """(header + key/values + tensor infos, data offsets)."""
        out = [b"GGUF", struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))]
        for k, t, v in self.kv:
            out.append(_str(k) + struct.pack("<I", t) + _value(t, v))
        offs, off = [], 0
        for name, gt, ne, raw in self.tensors:
            offs.append(off)
            out.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
                       + struct.pack("<IQ", gt, off))
            off += (len(raw) + self.alignment - 1) // self.alignment * self.alignment
        return b"".join(out), offs

    def write(self, path):
        head, offs = self.header_bytes()
        with open(path, "wb") as f:
            f.write(head)
            pad = (-len(head)) % self.alignment
            f.write(b"\0" * pad)
            pos = 0
            for (name, gt, ne, raw), off in zip(self.tensors, offs):
                f.write(b"\0" * (off - pos))
                f.write(raw)
                pos = off + len(raw)


def moe_keys(w, n_layer: int, first_k_dense: int = 0, prefix: str = "diffuse"):
    """The MoE hyper-parameter keys of a LayerWeights under `prefix`, as the
    reference's converter writes them (tools/convert-llada2-fast.py:125-144)."""
    return [(f"{prefix}.block_count", U32, n_layer),
            (f"{prefix}.embedding_length", U32, w.n_embd),
            (f"{prefix}.expert_count", U32, w.n_experts),
            (f"{prefix}.expert_used_count", U32, w.top_k),
            (f"{prefix}.expert_shared_count", U32, w.n_shared if w.sh_gate is not None else 0),
            (f"{prefix}.expert_feed_forward_length", U32, w.moe_ff),
            (f"{prefix}.first_k_dense_replace", U32, first_k_dense),
            (f"{prefix}.norm_topk_prob", U32, w.norm_topk_prob),
            (f"{prefix}.expert_capacity", U32, w.capacity),
            (f"{prefix}.moe_block_size", U32, w.block_size),
            (f"{prefix}.routed_scaling_factor", F32, w.routed_scaling)]


def add_moe_layer(wr: GGUFWriter, il: int, w):
    """blk.<il>.moe_* tensors of a LayerWeights (numpy)."""
    H, E, FF = w.n_embd, w.n_experts, w.moe_ff
    wr.add_tensor(f"blk.{il}.moe_gate.weight", 0, [H, E], np.ascontiguousarray(w.gate_w, np.float32))
    if w.gate_bias is not None:
        wr.add_tensor(f"blk.{il}.moe_gate_bias.weight", 0, [E], np.ascontiguousarray(w.gate_bias, np.float32))
    wr.add_tensor(f"blk.{il}.moe_experts_gate.weight", w.wtype, [H, FF, E], w.exp_gate)
    wr.add_tensor(f"blk.{il}.moe_experts_up.weight", w.wtype, [H, FF, E], w.exp_up)
    wr.add_tensor(f"blk.{il}.moe_experts_down.weight", w.wtype, [FF, H, E], w.exp_down)
    if w.sh_gate is not None:
        SF = w.shared_ff
        wr.add_tensor(f"blk.{il}.moe_shared_gate.weight", w.stype, [H, SF], w.sh_gate)
        wr.add_tensor(f"blk.{il}.moe_shared_up.weight", w.stype, [H, SF], w.sh_up)
        wr.add_tensor(f"blk.{il}.moe_shared_down.weight", w.stype, [SF, H], w.sh_down)


def add_dense_layer(wr: GGUFWriter, il: int, d):
    wr.add_tensor(f"blk.{il}.ffn_gate.weight", d.wtype, [d.n_embd, d.n_ff], d.gate)
    wr.add_tensor(f"blk.{il}.ffn_up.weight", d.wtype, [d.n_embd, d.n_ff], d.up)
    wr.add_tensor(f"blk.{il}.ffn_down.weight", d.wtype, [d.n_ff, d.n_embd], d.down)


def attn_keys(a, prefix: str = "diffuse"):
    """The attention hyper-parameter keys of an AttnWeights, as the
    reference's converter writes them (tools/convert-llada2-fast.py:125-144)."""
    return [(f"{prefix}.attention.head_count", U32, a.n_head),
            (f"{prefix}.attention.head_count_kv", U32, a.n_head_kv),
            (f"{prefix}.head_dim", U32, a.head_dim),
            (f"{prefix}.rotary_dim", U32, a.rotary_dim),
            (f"{prefix}.use_qk_norm", U32, 1 if a.q_norm is not None else 0),
            (f"{prefix}.block_length", U32, a.block_length),
            (f"{prefix}.rope.freq_base", F32, a.rope_base),
            (f"{prefix}.attention.layer_norm_rms_epsilon", F32, a.rms_eps)]


def add_attn_layer(wr: GGUFWriter, il: int, a):
    """blk.<il>.attn_* tensors of an AttnWeights (numpy)."""
    H, QD, QKV = a.n_embd, a.n_head * a.head_dim, (a.n_head + 2 * a.n_head_kv) * a.head_dim
    wr.add_tensor(f"blk.{il}.attn_norm.weight", 0, [H], np.ascontiguousarray(a.attn_norm, np.float32))
    wr.add_tensor(f"blk.{il}.post_attn_norm.weight", 0, [H], np.ascontiguousarray(a.post_norm, np.float32))
    wr.add_tensor(f"blk.{il}.attn_qkv.weight", a.wtype, [H, QKV], a.qkv)
    wr.add_tensor(f"blk.{il}.attn_output.weight", a.wtype, [QD, H], a.wo)
    if a.q_norm is not None:
        wr.add_tensor(f"blk.{il}.attn_q_norm.weight", 0, [a.head_dim], np.ascontiguousarray(a.q_norm, np.float32))
        wr.add_tensor(f"blk.{il}.attn_k_norm.weight", 0, [a.head_dim], np.ascontiguousarray(a.k_norm, np.float32))
