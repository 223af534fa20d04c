"""CPU: pins the oracle's step tail (src/diffuse-moe-graph.cpp:295-300 and
the temperature-0 sampler, src/diffuse-sampler.cpp:29-49): RMSNorm against
float64 numpy and a closed form, argmax / confidence against known answers
(ties to the first index, a NaN first logit, one-hot and uniform rows) and a
float64 softmax, and the LM-head logits against float64 numpy on the
dequantised output weight."""
import numpy as np
import pytest

F32, F16, Q8_0, Q4_K = 0, 1, 8, 12


def test_rms_norm(O):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((5, 512)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 512).astype(np.float32)
    y = O.rms_norm(x, w, 1e-6)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(1, keepdims=True) + 1e-6) * w
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-6
    c = np.full((1, 256), 0.75, np.float32)                   # all equal: c / sqrt(c^2 + eps)
    assert np.allclose(O.rms_norm(c, None, 1e-6), 0.75 / np.sqrt(0.5625 + 1e-6), rtol=1e-6)


def test_argmax_prob_known_answers(O):
    V = 1000
    rows = np.zeros((5, V), np.float32)
    rows[0, [10, 20]] = 5.0                                    # tie: the first index
    rows[1, 0] = np.nan                                        # NaN first: token 0, prob NaN
    rows[1, 3] = 9.0
    rows[2, 7] = 100.0                                         # one-hot: prob 1
    rows[4, 999] = 1.0                                         # the last index
    tok, prob = O.argmax_prob(rows)
    assert tok.tolist() == [10, 0, 7, 0, 999]
    assert np.isnan(prob[1])
    assert prob[2] == np.float32(1.0)
    assert np.isclose(prob[3], 1.0 / V, rtol=1e-5)             # uniform row
    # the sum runs in float, sequentially (the reference's loop): with 998
    # equal terms added to a sum near 8.7 each addition rounds the same way,
    # a systematic error of a few 1e-5 relative against the exact value
    e = np.exp(np.float64(-5.0))
    assert np.isclose(prob[0], 1.0 / (2 + (V - 2) * e), rtol=1e-4)
    s = np.float32(0.0)
    for v in rows[0]:
        s = np.float32(s + np.float32(np.exp(np.float64(v) - 5.0)))
    assert prob[0] == np.float32(1.0) / s


def test_argmax_prob_against_float64(O):
    rng = np.random.default_rng(2)
    logits = (rng.standard_normal((8, 4096)) * 4).astype(np.float32)
    tok, prob = O.argmax_prob(logits)
    assert np.array_equal(tok, logits.argmax(1))
    ld = logits.astype(np.float64)
    ref = 1.0 / np.exp(ld - ld.max(1, keepdims=True)).sum(1)
    assert np.abs(prob - ref).max() / ref.max() < 1e-5


@pytest.mark.parametrize("wtype", [F32, Q8_0, Q4_K], ids=["F32", "Q8_0", "Q4_K"])
def test_head_logits_against_float64(O, wtype):
    from dmoe import synth
    H, V, N = 512, 1024, 6
    w = synth.host_head(H, V, wtype, 9, O.quantize_rows)
    h = (synth.normal(9, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    tok, prob, logits = O.head_forward(w, h, 1e-6)
    xn = O.rms_norm(h, w.norm, 1e-6).astype(np.float64)
    Wd = O.dequant_rows(wtype, w.output, V, H).astype(np.float64)
    ref = xn @ Wd.T
    assert np.abs(logits - ref).max() / np.abs(ref).max() < 1e-6
    t2, p2 = O.argmax_prob(logits)
    assert np.array_equal(tok, t2) and np.array_equal(prob, p2)
