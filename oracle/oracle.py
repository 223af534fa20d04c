"""ctypes loader for the CPU oracle (oracle/libdmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker.  tests/, the smoke entry and the
CPU-baseline leg of bench.py use it; the product never does.  The C sources
(dmoe_oracle.c) restate src/diffuse-moe-graph.cpp:188-289 of Akicou/diffuse-cpp
with ggml's CPU semantics; see the header of dmoe_oracle.h for what pins each
function.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ROOT = ORACLE_DIR.parent
LIB_PATH = ORACLE_DIR / "libdmoe_oracle.so"
sys.path.insert(0, str(ROOT / "diffuse-cpp_amd"))

from dmoe import _abi  # noqa: E402  (struct layouts of include/dmoe.h)
from dmoe._abi import AttnDesc, AttnHParams, Debug, HParams, LayerDesc, Tensor  # noqa: E402

TYPE_Q8_K = _abi.TYPE_Q8_K

_lib = None


def build(force: bool = False) -> Path:
    srcs = [ORACLE_DIR / "dmoe_oracle.c", ORACLE_DIR / "dmoe_cpu_simd.c", ORACLE_DIR / "dmoe_oracle.h",
            ROOT / "include" / "dmoe.h"]
    if force or not LIB_PATH.exists() or any(s.stat().st_mtime > LIB_PATH.stat().st_mtime for s in srcs):
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "-B" if force else "all"], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = C.CDLL(str(LIB_PATH))
    P = C.c_void_p
    lib.dmo_f16_to_f32.argtypes = [C.c_uint16]
    lib.dmo_f16_to_f32.restype = C.c_float
    lib.dmo_f32_to_f16.argtypes = [C.c_float]
    lib.dmo_f32_to_f16.restype = C.c_uint16
    lib.dmo_f16_to_f32_n.argtypes = [P, P, C.c_int64]
    lib.dmo_f32_to_f16_n.argtypes = [P, P, C.c_int64]
    lib.dmo_expf.argtypes = [C.c_float]
    lib.dmo_expf.restype = C.c_float
    lib.dmo_expf_n.argtypes = [P, P, C.c_int64]
    lib.dmo_sigmoid.argtypes = [C.c_float]
    lib.dmo_sigmoid.restype = C.c_float
    lib.dmo_row_size.argtypes = [C.c_int32, C.c_int64]
    lib.dmo_row_size.restype = C.c_size_t
    lib.dmo_q4K_scale_min.argtypes = [C.c_int, P, P, P]
    lib.dmo_q4K_scale_min.restype = None
    lib.dmo_dequant_row.argtypes = [C.c_int32, P, P, C.c_int64]
    lib.dmo_quantize_rows.argtypes = [C.c_int32, P, P, C.c_int64, C.c_int64, C.c_int]
    lib.dmo_quantize_row_act.argtypes = [C.c_int32, P, P, C.c_int64]
    lib.dmo_vec_dot.argtypes = [C.c_int32, C.c_int64, P, P]
    lib.dmo_vec_dot.restype = C.c_float
    lib.dmo_router_logits.argtypes = [P, C.c_int64, P, C.c_int, C.c_int, C.c_int, P]
    lib.dmo_router_logits.restype = None
    lib.dmo_use_block_routing.argtypes = [C.POINTER(HParams), C.c_int]
    lib.dmo_block_fold.argtypes = [P, C.c_int, C.c_int]
    lib.dmo_block_fold.restype = C.c_float
    lib.dmo_route.argtypes = [C.POINTER(HParams), P, P, C.c_int, P, P, P, P, P, P]
    lib.dmo_dispatch.argtypes = [P, C.c_int, C.c_int, C.c_int, P, P, P]
    lib.dmo_dispatch.restype = None
    lib.dmo_layer_forward.argtypes = [C.POINTER(HParams), C.POINTER(LayerDesc), P, C.c_int, P,
                                      C.POINTER(Debug), C.c_int]
    lib.dmo_dense_forward.argtypes = [C.c_int, C.c_int, C.POINTER(Tensor), C.POINTER(Tensor),
                                      C.POINTER(Tensor), P, C.c_int, P, C.c_int]
    lib.dmo_rms_norm.argtypes = [P, P, C.c_int, C.c_float, P]
    lib.dmo_rms_norm.restype = None
    lib.dmo_argmax_prob.argtypes = [P, C.c_int, P, P]
    lib.dmo_argmax_prob.restype = None
    lib.dmo_simd_available.argtypes = []
    lib.dmo_set_simd.argtypes = [C.c_int]
    lib.dmo_dot_q4K_simd.argtypes = [C.c_int64, P, P]
    lib.dmo_dot_q4K_simd.restype = C.c_float
    lib.dmo_dot_q8_0_simd.argtypes = [C.c_int64, P, P]
    lib.dmo_dot_q8_0_simd.restype = C.c_float
    lib.dmo_dot_f32_simd.argtypes = [C.c_int64, P, P]
    lib.dmo_dot_f32_simd.restype = C.c_float
    lib.dmo_dot_f16_simd.argtypes = [C.c_int64, P, P]
    lib.dmo_dot_f16_simd.restype = C.c_float
    lib.dmo_rope_neox.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_float]
    lib.dmo_rope_neox.restype = None
    lib.dmo_attn_forward.argtypes = [C.POINTER(AttnHParams), C.POINTER(AttnDesc), P, C.c_int, P, P, C.c_int]
    lib.dmo_head_forward.argtypes = [C.c_int, C.c_int, P, C.POINTER(Tensor), P, C.c_int, C.c_float,
                                     P, P, P, C.c_int]
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    load().dmo_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    load().dmo_f32_to_f16_n(_p(f), _p(out), f.size)
    return out


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    load().dmo_expf_n(_p(x), _p(out), x.size)
    return out


def sigmoid(v: float) -> float:
    return load().dmo_sigmoid(v)


def row_size(t: int, n: int) -> int:
    return load().dmo_row_size(t, n)


def q4k_scale_min(j: int, scales: bytes):
    s = np.frombuffer(bytes(scales), np.uint8).copy()
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    load().dmo_q4K_scale_min(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def dequant_rows(t: int, data: np.ndarray, nrows: int, n: int) -> np.ndarray:
    data = np.ascontiguousarray(data).view(np.uint8).reshape(nrows, -1)
    out = np.empty((nrows, n), np.float32)
    for r in range(nrows):
        if load().dmo_dequant_row(t, _p(data[r]), _p(out[r]), n):
            raise ValueError("dequant failed")
    return out


def quantize_rows(t: int, f: np.ndarray, n_threads: int = 0) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    rows, n = f.shape
    out = np.empty((rows, row_size(t, n)), np.uint8)
    if load().dmo_quantize_rows(t, _p(f), _p(out), rows, n, n_threads):
        raise ValueError("quantize failed")
    return out


def act_row_size(at: int, n: int) -> int:
    return n * 4 if at == 0 else (n * 2 if at == 1 else row_size(at, n))


def quantize_act(at: int, f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    rows, n = f.shape
    out = np.empty((rows, act_row_size(at, n)), np.uint8)
    for r in range(rows):
        if load().dmo_quantize_row_act(at, _p(f[r]), _p(out[r]), n):
            raise ValueError("act quantize failed")
    return out


def vec_dot(wt: int, n: int, wrow: np.ndarray, xrow: np.ndarray) -> float:
    wrow = np.ascontiguousarray(wrow)
    xrow = np.ascontiguousarray(xrow)
    return load().dmo_vec_dot(wt, n, _p(wrow), _p(xrow))


def router_logits(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    E, H = W.shape
    N = x.shape[0]
    out = np.empty((N, E), np.float32)
    load().dmo_router_logits(_p(W), H, _p(x), N, H, E, _p(out))
    return out


def block_fold(s: np.ndarray) -> np.float32:
    s = np.ascontiguousarray(s, dtype=np.float32)
    return np.float32(load().dmo_block_fold(_p(s), s.size, 1))


def route(hp: HParams, logits: np.ndarray, bias=None) -> dict:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    N, E = logits.shape
    K = hp.top_k
    use = bool(load().dmo_use_block_routing(C.byref(hp), N))
    B = N // hp.block_size if use else 0
    out = dict(probs=np.zeros((N, E), np.float32), bmax=np.zeros((B, E), np.float32),
               thr=np.zeros((B,), np.float32), allowed=np.zeros((B, E), np.uint8),
               idx=np.zeros((N, K), np.int32), weights=np.zeros((N, K), np.float32))
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = load().dmo_route(C.byref(hp), _p(b), _p(logits), N, _p(out["probs"]),
                          _p(out["bmax"]) if B else None, _p(out["thr"]) if B else None,
                          _p(out["allowed"]) if B else None, _p(out["idx"]), _p(out["weights"]))
    if rc:
        raise ValueError("route failed")
    out["use_block_routing"] = use
    c, o, p = dispatch(out["idx"], E)
    out.update(counts=c, offsets=o, perm=p)
    return out


def dispatch(idx: np.ndarray, n_experts: int):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    N, K = idx.shape
    counts = np.zeros(n_experts, np.int32)
    offsets = np.zeros(n_experts, np.int32)
    perm = np.zeros(N * K, np.int32)
    load().dmo_dispatch(_p(idx), N, K, n_experts, _p(counts), _p(offsets), _p(perm))
    return counts, offsets, perm


def layer_forward(w, x: np.ndarray, debug: bool = False, n_threads: int = 0):
    """w: dmoe.LayerWeights with numpy arrays."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    N = x.shape[0]
    hp, d = w.hparams(), w.desc()
    y = np.empty_like(x)
    dbg = None
    if debug:
        from dmoe import DebugOut
        dbg = DebugOut(hp, N)
        ds = dbg.struct()
    rc = load().dmo_layer_forward(C.byref(hp), C.byref(d), _p(x), N, _p(y),
                                  C.byref(ds) if debug else None, n_threads)
    if rc:
        raise ValueError("oracle layer forward failed")
    return (y, dbg.as_dict()) if debug else y


def dense_forward(w, x: np.ndarray, n_threads: int = 0) -> np.ndarray:
    """w: dmoe.DenseWeights with numpy arrays (src/diffuse-moe-graph.cpp:181-187)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    N = x.shape[0]
    g, u, d = w.views()
    y = np.empty_like(x)
    rc = load().dmo_dense_forward(w.n_embd, w.n_ff, C.byref(g), C.byref(u), C.byref(d), _p(x), N,
                                  _p(y), n_threads)
    if rc:
        raise ValueError("oracle dense forward failed")
    return y


def rms_norm(x: np.ndarray, w=None, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    wp = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    for i in range(x.shape[0]):
        load().dmo_rms_norm(_p(x[i]), _p(wp), x.shape[1], eps, _p(out[i]))
    return out


def argmax_prob(logits: np.ndarray):
    """(tokens i32 [N], probs f32 [N]) of logits [N][V]."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    N, V = logits.shape
    tok = np.zeros(N, np.int32)
    prob = np.zeros(N, np.float32)
    for i in range(N):
        load().dmo_argmax_prob(_p(logits[i]), V, _p(tok[i:i + 1]), _p(prob[i:i + 1]))
    return tok, prob


def head_forward(w, h: np.ndarray, eps: float = 1e-6, n_threads: int = 0):
    """w: dmoe.HeadWeights (numpy).  Returns (tokens, probs, logits)."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    N = h.shape[0]
    V = w.n_vocab
    tok = np.zeros(N, np.int32)
    prob = np.zeros(N, np.float32)
    logits = np.zeros((N, V), np.float32)
    norm = np.ascontiguousarray(w.norm, dtype=np.float32)
    ov = w.output_view()
    rc = load().dmo_head_forward(w.n_embd, V, _p(norm), C.byref(ov), _p(h), N, eps, _p(tok), _p(prob),
                                 _p(logits), n_threads)
    if rc:
        raise ValueError("oracle head forward failed")
    return tok, prob, logits


def simd_available() -> bool:
    return bool(load().dmo_simd_available())


def set_simd(on: bool) -> bool:
    """Route the dots through the AVX-512 versions (the CPU baseline's fast
    path: bit-identical results for the quantised types, binary32 sums for
    F32 / F16).  Returns whether they are in use."""
    return bool(load().dmo_set_simd(1 if on else 0))


def vec_dot_simd(wt: int, n: int, wrow: np.ndarray, xrow: np.ndarray) -> float:
    lib = load()
    f = {12: lib.dmo_dot_q4K_simd, 8: lib.dmo_dot_q8_0_simd, 0: lib.dmo_dot_f32_simd,
         1: lib.dmo_dot_f16_simd}[wt]
    return float(f(n, _p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(xrow))))


def rope_neox(x: np.ndarray, n_dims: int, pos: int, base: float) -> np.ndarray:
    """A rotated copy of one head vector x (NEOX pairs (i, i + n_dims/2))."""
    y = np.array(x, dtype=np.float32, copy=True)
    load().dmo_rope_neox(_p(y), y.shape[0], n_dims, pos, base)
    return y


def attn_forward(w, h: np.ndarray, n_threads: int = 0):
    """w: dmoe.AttnWeights (numpy).  Returns (h_out, moe_in)."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    N = h.shape[0]
    a, d = w.hparams(), w.desc()
    h_out = np.empty_like(h)
    moe_in = np.empty_like(h)
    if load().dmo_attn_forward(C.byref(a), C.byref(d), _p(h), N, _p(h_out), _p(moe_in), n_threads):
        raise ValueError("oracle attention forward failed")
    return h_out, moe_in


def n_threads_default() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
