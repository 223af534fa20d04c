"""ctypes mirror of the structs in include/dmoe.h (field order and types
must match the header exactly)."""
import ctypes as C

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_Q8_K = 15          # activation-only type (vec_dot_type of Q4_K and Q6_K)

TYPE_NAMES = {TYPE_F32: "F32", TYPE_F16: "F16", TYPE_Q8_0: "Q8_0", TYPE_Q4_K: "Q4_K", TYPE_Q6_K: "Q6_K"}
TYPE_BY_NAME = {v: k for k, v in TYPE_NAMES.items()}

OK = 0
ERR_INVALID_ARG = 1
ERR_UNSUPPORTED_TYPE = 2
ERR_SHAPE = 3
ERR_HIP = 4
ERR_OOM = 5
ERR_NONFINITE = 6
ERR_FORMAT = 7
ERR_NOT_FOUND = 8


class Tensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("data", C.c_void_p),
                ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4)]


class HParams(C.Structure):
    _fields_ = [("n_embd", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32),
                ("capacity", C.c_int32), ("block_size", C.c_int32), ("moe_ff", C.c_int32),
                ("n_shared", C.c_int32), ("shared_ff", C.c_int32),
                ("norm_topk_prob", C.c_int32), ("routed_scaling", C.c_float)]


class LayerDesc(C.Structure):
    _fields_ = [(n, Tensor) for n in ("gate_w", "gate_bias", "exp_gate", "exp_up", "exp_down",
                                      "sh_gate", "sh_up", "sh_down")]


class AttnHParams(C.Structure):
    _fields_ = [("n_embd", C.c_int32), ("n_head", C.c_int32), ("n_head_kv", C.c_int32),
                ("head_dim", C.c_int32), ("rotary_dim", C.c_int32), ("use_qk_norm", C.c_int32),
                ("block_length", C.c_int32), ("rope_base", C.c_float), ("rms_eps", C.c_float)]


class AttnDesc(C.Structure):
    _fields_ = [(n, Tensor) for n in ("attn_norm", "qkv", "q_norm", "k_norm", "wo", "post_attn_norm")]


class Debug(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("probs", C.c_void_p), ("bmax", C.c_void_p),
                ("thr", C.c_void_p), ("allowed", C.c_void_p), ("idx", C.c_void_p),
                ("weights", C.c_void_p), ("counts", C.c_void_p), ("offsets", C.c_void_p),
                ("perm", C.c_void_p), ("use_block_routing", C.c_void_p)]


def block_elems(t: int) -> int:
    return {TYPE_F32: 1, TYPE_F16: 1, TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q6_K: 256, TYPE_Q8_K: 256}[t]


def block_bytes(t: int) -> int:
    return {TYPE_F32: 4, TYPE_F16: 2, TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q8_K: 292}[t]


def row_size(t: int, n: int) -> int:
    be = block_elems(t)
    if n % be:
        raise ValueError(f"row of {n} values is not a whole number of {TYPE_NAMES.get(t, t)} blocks")
    return n // be * block_bytes(t)
