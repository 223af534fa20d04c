"""CPU: the AVX-512 dots the CPU baseline uses (oracle/dmoe_cpu_simd.c).  The
VNNI quantised dots equal the scalar oracle's bit for bit: random Q4_K and
Q8_0 rows against Q8_K / Q8_0 activations, including extreme blocks (all-15
nibbles with the largest scales, -127 / 127 activations).  The F32 / F16
dots sum in binary32 (ggml's SIMD order) and stay within 1e-5 of the sum of
|w x| of the scalar binary64 sums; a layer forward with the fast dots keeps
every routing output bit for bit and its output within 1e-4 relative (an
f32 difference in gate / up can move an f16 rounding of h: one f16 step is
~5e-4 relative; the F16 layer contract is 1e-3)."""
import numpy as np
import pytest

import oracle as O

Q4_K, Q8_0, Q8_K = 12, 8, 15


@pytest.fixture(autouse=True)
def _need_simd(request):
    request.getfixturevalue("O")
    if not O.simd_available():
        pytest.skip("CPU without AVX-512 VNNI")


@pytest.mark.parametrize("seed", range(4))
def test_q4k_dot_bit_exact(seed):
    rng = np.random.default_rng(seed)
    n, rows = 4096, 64
    w = O.quantize_rows(Q4_K, (rng.standard_normal((rows, n)) * (0.02 + seed)).astype(np.float32))
    xs = rng.standard_normal((8, n)).astype(np.float32) * (1 + 10 * seed)
    xq = list(O.quantize_act(Q8_K, xs))
    for r in range(rows):
        for x in xq:
            a = np.float32(O.vec_dot(Q4_K, n, w[r], x))
            b = np.float32(O.vec_dot_simd(Q4_K, n, w[r], x))
            assert a.view(np.uint32) == b.view(np.uint32)


def test_q4k_dot_extremes():
    n = 256
    w = np.zeros(144, np.uint8)
    w[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    w[2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    w[4:16] = 0xFF                                          # every 6-bit scale and min at 63
    w[16:] = 0xFF                                           # every nibble 15
    for val in (127, -127):
        x = np.full(n, val / 127.0 * 3.0, np.float32)
        xq = O.quantize_act(Q8_K, x[None])[0]
        a = np.float32(O.vec_dot(Q4_K, n, w, xq))
        b = np.float32(O.vec_dot_simd(Q4_K, n, w, xq))
        assert a.view(np.uint32) == b.view(np.uint32)


@pytest.mark.parametrize("seed", range(3))
def test_q8_0_dot_bit_exact(seed):
    rng = np.random.default_rng(100 + seed)
    n, rows = 2048, 64
    w = O.quantize_rows(Q8_0, rng.standard_normal((rows, n)).astype(np.float32))
    xq = list(O.quantize_act(Q8_0, rng.standard_normal((8, n)).astype(np.float32)))
    for r in range(rows):
        for x in xq:
            a = np.float32(O.vec_dot(Q8_0, n, w[r], x))
            b = np.float32(O.vec_dot_simd(Q8_0, n, w[r], x))
            assert a.view(np.uint32) == b.view(np.uint32)


@pytest.mark.parametrize("wt", [0, 1], ids=["F32", "F16"])
@pytest.mark.parametrize("n", [4096, 1024, 100])
def test_float_dots_within_tolerance(wt, n):
    rng = np.random.default_rng(7 + n + wt)
    w = (rng.standard_normal((16, n)) * 0.02).astype(np.float32)
    x = rng.standard_normal((4, n)).astype(np.float32)
    if wt == 1:
        w, x = w.astype(np.float16), x.astype(np.float16)
    for r in range(16):
        for t in range(4):
            a = O.vec_dot(wt, n, w[r], x[t])
            b = O.vec_dot_simd(wt, n, w[r], x[t])
            scale = float(np.abs(w[r].astype(np.float64) * x[t].astype(np.float64)).sum())
            assert abs(a - b) <= 1e-5 * scale, (r, t, a, b)


@pytest.mark.parametrize("wt", [12, 1], ids=["Q4_K", "F16"])
def test_layer_forward_with_simd_dots(wt):
    import dmoe
    from dmoe import synth
    cfg = synth.LayerConfig("simd_small", 512, 32, 256, 8, 4, 32, 256, wt, wt, 64, -0.05, 0.05)
    w = synth.host_layer(cfg, 9, O.quantize_rows)
    x = synth.make_x(cfg, 9, 64)
    O.set_simd(False)
    y0, d0 = O.layer_forward(w, x, debug=True)
    try:
        assert O.set_simd(True)
        y1, d1 = O.layer_forward(w, x, debug=True)
    finally:
        O.set_simd(False)
    for k in ("logits", "idx", "weights", "perm"):
        assert np.array_equal(d0[k], d1[k]), k
    assert np.abs(y1 - y0).max() <= 1e-4 * np.abs(y0).max()
