"""CPU: pins the oracle's dense MLP (src/diffuse-moe-graph.cpp:181-187)
against an independent float64 model on the dequantised weights:
y = W_down (silu(W_gate x) * (W_up x)), the weights cast to F32 (:8-12) and
F32 activations.  Swapping gate and up, dropping the SiLU or transposing a
matrix moves the result by O(1), far outside the float32 accumulation noise
the bound allows."""
import numpy as np
import pytest

F32, F16, Q8_0, Q4_K = 0, 1, 8, 12


def _model(O, w, x):
    H, FF, t = w.n_embd, w.n_ff, w.wtype
    Wg = O.dequant_rows(t, w.gate, FF, H).astype(np.float64)
    Wu = O.dequant_rows(t, w.up, FF, H).astype(np.float64)
    Wd = O.dequant_rows(t, w.down, H, FF).astype(np.float64)
    xs = x.astype(np.float64)
    g = xs @ Wg.T
    h = (g / (1.0 + np.exp(-g))) * (xs @ Wu.T)
    return h.astype(np.float32).astype(np.float64) @ Wd.T


@pytest.mark.parametrize("wtype", [F32, F16, Q8_0, Q4_K], ids=["F32", "F16", "Q8_0", "Q4_K"])
def test_dense_matches_float64_model(O, wtype):
    from dmoe import synth
    H, FF, N = 512, 768, 24
    w = synth.host_dense(H, FF, wtype, 41, O.quantize_rows)
    x = synth.normal(41, synth.S_X, N * H).reshape(N, H)
    y = O.dense_forward(w, x)
    ref = _model(O, w, x)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    assert err < 1e-5, err
    # gate and up are not interchangeable: the swapped model is far away
    swapped = _model(O, synth.replace(w, gate=w.up, up=w.gate), x)
    assert np.abs(swapped - ref).max() / np.abs(ref).max() > 0.1


def test_dense_threads_do_not_change_bits(O):
    from dmoe import synth
    w = synth.host_dense(512, 512, Q4_K, 42, O.quantize_rows)
    x = synth.normal(42, synth.S_X, 16 * 512).reshape(16, 512)
    a = O.dense_forward(w, x, n_threads=1)
    b = O.dense_forward(w, x, n_threads=5)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
