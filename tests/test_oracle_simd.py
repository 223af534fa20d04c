"""CPU: the AVX-512 VNNI dots the CPU baseline uses (oracle/dmoe_cpu_simd.c)
equal the scalar oracle's bit for bit: random Q4_K and Q8_0 rows against
Q8_K / Q8_0 activations, including extreme blocks (all-15 nibbles with the
largest scales, -127 / 127 activations), and the whole flash-shaped layer
forward with the fast dots switched on equals the scalar forward."""
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


def test_layer_forward_with_simd_dots():
    import dmoe
    from dmoe import synth
    cfg = synth.LayerConfig("simd_small", 512, 32, 256, 8, 4, 32, 256, dmoe.TYPE_Q4_K, dmoe.TYPE_Q4_K, 64,
                            -0.05, 0.05)
    w = synth.host_layer(cfg, 9, O.quantize_rows)
    x = synth.make_x(cfg, 9, 64)
    O.set_simd(False)
    y0 = O.layer_forward(w, x)
    try:
        assert O.set_simd(True)
        y1 = O.layer_forward(w, x)
    finally:
        O.set_simd(False)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
