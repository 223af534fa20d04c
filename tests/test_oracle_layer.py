"""CPU: pins the oracle's whole segment against an independent float64 model.

The model takes the oracle's routing (pinned in test_oracle_router.py) and
recomputes the experts in float64 from dequantised weights
(diffuse-moe-graph.cpp:264-286): the routed products use the activations
converted to the weight's vec_dot_type, as ggml_mul_mat_id does, the shared
expert uses F32 activations (its weights are cast to F32, :8-12).  Agreement
within float32 accumulation noise pins the expert wiring (gate vs up, SwiGLU,
down, slot weights, left-fold combine, shared add); a second model with
unquantised activations bounds how far ggml's activation conversion moves the
output.
"""
import numpy as np
import pytest

F32, F16, Q8_0, Q4_K, Q8_K = 0, 1, 8, 12, 15
ACT = {F32: F32, F16: F16, Q8_0: Q8_0, Q4_K: Q8_K}


def _act_values(at, b, n):
    b = np.ascontiguousarray(b)
    if at == F32:
        return b.view(np.float32).astype(np.float64)
    if at == F16:
        return b.view(np.float16).astype(np.float64)
    if at == Q8_0:
        blk = b.reshape(n // 32, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)
        return (blk[:, 2:].view(np.int8).astype(np.float64) * d).reshape(-1)
    blk = b.reshape(n // 256, 292)
    d = blk[:, :4].copy().view(np.float32).astype(np.float64)
    return (blk[:, 4:260].view(np.int8).astype(np.float64) * d).reshape(-1)


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _model(O, w, x, idx, weights, quantise_acts=True):
    H, E, FF, K = w.n_embd, w.n_experts, w.moe_ff, w.top_k
    N = x.shape[0]
    t = w.wtype
    at = ACT[t]

    def deq(arr, rows, n, typ):
        return O.dequant_rows(typ, arr.reshape(rows, -1), rows, n).astype(np.float64)

    def act(v):                      # v: float32 [n] -> float64 values seen by the dot
        if not quantise_acts:
            return v.astype(np.float64)
        return _act_values(at, O.quantize_act(at, v[None].astype(np.float32))[0], v.size)

    y = np.zeros((N, H), np.float64)
    cache = {}
    for tok in range(N):
        xa = act(x[tok])
        for s in range(K):
            e = int(idx[tok, s])
            if e not in cache:
                cache[e] = (deq(w.exp_gate[e], FF, H, t), deq(w.exp_up[e], FF, H, t),
                            deq(w.exp_down[e], H, FF, t))
            Wg, Wu, Wd = cache[e]
            h = (_silu(Wg @ xa) * (Wu @ xa)).astype(np.float32)
            y[tok] += float(weights[tok, s]) * (Wd @ act(h))
    if w.sh_gate is not None:
        SF = w.shared_ff
        Sg = deq(w.sh_gate, SF, H, w.stype)
        Su = deq(w.sh_up, SF, H, w.stype)
        Sd = deq(w.sh_down, H, SF, w.stype)
        xs = x.astype(np.float64)
        hs = (_silu(xs @ Sg.T) * (xs @ Su.T)).astype(np.float32).astype(np.float64)
        y += hs @ Sd.T
    return y


def _cfg(wtype, n_tokens=64):
    from dmoe import synth
    if wtype == F32:
        return synth.CONFIGS["tiny"]
    return synth.LayerConfig(f"small_{wtype}", 512, 16, 256, 6, 4, 32, 256, wtype, wtype,
                             n_tokens, -0.05, 0.05)


@pytest.mark.parametrize("wtype", [F32, F16, Q8_0, Q4_K], ids=["F32", "F16", "Q8_0", "Q4_K"])
def test_layer_matches_float64_model(O, wtype):
    from dmoe import synth
    cfg = _cfg(wtype)
    w = synth.host_layer(cfg, 31, O.quantize_rows)
    x = synth.make_x(cfg, 31)
    y, dbg = O.layer_forward(w, x, debug=True)
    ref = _model(O, w, x, dbg["idx"], dbg["weights"])
    err = np.abs(y - ref).max() / np.abs(ref).max()
    assert err < 2e-4, err


@pytest.mark.parametrize("wtype", [Q8_0, Q4_K])
def test_activation_conversion_effect_is_bounded(O, wtype):
    """ggml's conversion of the activations to Q8_0 / Q8_K moves the output
    by well under the 2e-2 layer tolerance relative to exact activations."""
    from dmoe import synth
    cfg = _cfg(wtype)
    w = synth.host_layer(cfg, 32, O.quantize_rows)
    x = synth.make_x(cfg, 32)
    y, dbg = O.layer_forward(w, x, debug=True)
    exact = _model(O, w, x, dbg["idx"], dbg["weights"], quantise_acts=False)
    err = np.abs(y - exact).max() / np.abs(exact).max()
    assert 1e-5 < err < 2e-2, err


def test_layer_threads_do_not_change_bits(O):
    from dmoe import synth
    cfg = _cfg(Q4_K)
    w = synth.host_layer(cfg, 33, O.quantize_rows)
    x = synth.make_x(cfg, 33)
    a = O.layer_forward(w, x, n_threads=1)
    b = O.layer_forward(w, x, n_threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
