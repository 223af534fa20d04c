"""CPU: pins the oracle's number formats, quantisers, dots and exp.

Each check is chosen so that a plausible mistake (dropped term, swapped
nibble half, wrong scale index, wrong rounding mode) fails it: known-answer
blocks built by hand, numpy's IEEE conversions, float64 references and
closed-form error bounds.  No check restates the oracle's own code.
"""
import numpy as np
import pytest

F32, F16, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 8, 12, 14, 15


def test_f16_to_f32_all_halves(O):
    h = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even(O):
    rng = np.random.default_rng(0)
    f = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 3,
        (rng.standard_normal(50000) * 1e-6).astype(np.float32),       # subnormal halves
        np.array([65504, 65519.99, 65520, 1e9, -65520, 2**-24, 2**-25, 2**-25 * 1.0001,
                  3 * 2**-26, 0.0, -0.0, np.inf, -np.inf, 1 + 2**-11, 1 + 3 * 2**-11],
                 np.float32)])
    got = O.f32_to_f16(f)
    ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# --- Q4_K ------------------------------------------------------------------
# Hand-packed 12 scale bytes.  Sub-blocks 0..3 keep 6-bit (sc, m) in the low
# bits of bytes j and j+4; sub-blocks 4..7 keep their low nibbles in byte j+4
# and their top two bits in the top bits of bytes j-4 (sc) and j (m).
SCALES = bytes([0xC1, 0x42, 0x83, 0x04,     # sc0..3 = 1,2,3,4 ; top bits -> sc4..7 hi
                0x45, 0x86, 0x07, 0xC8,     # m0..3 = 5,6,7,8 ; top bits -> m4..7 hi
                0x19, 0x2A, 0x3B, 0x4C])    # sc4..7 lo / m4..7 lo nibbles
# sc4 = 0x9 | (0xC1>>6)<<4 = 9+48 = 57, m4 = 0x1 | (0x45>>6)<<4 = 1+16 = 17
# sc5 = 0xA | (0x42>>6)<<4 = 10+16 = 26, m5 = 0x2 | (0x86>>6)<<4 = 2+32 = 34
# sc6 = 0xB | (0x83>>6)<<4 = 11+32 = 43, m6 = 0x3 | (0x07>>6)<<4 = 3
# sc7 = 0xC | (0x04>>6)<<4 = 12,         m7 = 0x4 | (0xC8>>6)<<4 = 4+48 = 52
EXPECT_SCALE_MIN = [(1, 5), (2, 6), (3, 7), (4, 8), (57, 17), (26, 34), (43, 3), (12, 52)]


def test_q4k_scale_min_all_indices(O):
    for j in range(8):
        assert O.q4k_scale_min(j, SCALES) == EXPECT_SCALE_MIN[j], j


def _q4k_block(d_bits, dmin_bits, scales, qs):
    return (np.array([d_bits, dmin_bits], np.uint16).tobytes() + bytes(scales) + bytes(qs))


def test_q4k_dequant_known_block(O):
    # d = 0.5 (0x3800), dmin = 0.25 (0x3400); qs byte b of chunk c = (c*32 + b) % 256
    qs = [(i * 7 + 3) % 256 for i in range(128)]
    blk = np.frombuffer(_q4k_block(0x3800, 0x3400, SCALES, qs), np.uint8)
    assert blk.size == 144
    y = O.dequant_rows(Q4_K, blk, 1, 256)[0]
    # literal spot values, worked by hand from the layout:
    #  weight 0:   chunk 0 low nibble of qs[0]=3  -> sub 0: 0.5*1*3 - 0.25*5 = 0.25
    #  weight 32:  chunk 0 high nibble of qs[0]=3 -> 0   -> sub 1: 0.5*2*0 - 0.25*6 = -1.5
    #  weight 65:  chunk 1 low nibble of qs[33]=(33*7+3)%256=234 -> 10 -> sub 2: 0.5*3*10-0.25*7=13.25
    #  weight 255: chunk 3 high nibble of qs[127]=(127*7+3)%256=124 -> 7 -> sub 7: 0.5*12*7-0.25*52=29
    #  weight 200: chunk 3 low nibble of qs[104]=(104*7+3)%256=219 -> 11 -> sub 6: 0.5*43*11-0.25*3=235.75
    assert y[0] == np.float32(0.25)
    assert y[32] == np.float32(-1.5)
    assert y[65] == np.float32(13.25)
    assert y[255] == np.float32(29.0)
    assert y[200] == np.float32(235.75)
    # every value is d*sc*q - dmin*m for some 4-bit q of its own sub-block
    for i in range(256):
        sc, m = EXPECT_SCALE_MIN[i // 32]
        q = (y[i] + 0.25 * m) / (0.5 * sc)
        assert abs(q - round(q)) < 1e-6 and 0 <= round(q) <= 15


def test_q8_0_dequant_known_block(O):
    qs = np.arange(-16, 16, dtype=np.int8)
    blk = np.frombuffer(np.array([0x3800], np.uint16).tobytes() + qs.tobytes(), np.uint8)
    y = O.dequant_rows(Q8_0, blk, 1, 32)[0]
    assert np.array_equal(y, (qs.astype(np.float32) * 0.5))


@pytest.mark.parametrize("t", [Q8_0, Q4_K, F16])
def test_weight_quantiser_error_bound(O, t):
    rng = np.random.default_rng(1)
    f = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    q = O.quantize_rows(t, f)
    d = O.dequant_rows(t, q, 16, 1024)
    err = np.abs(d - f)
    if t == F16:
        assert np.all(err <= np.abs(f) * 2**-11 + 2**-25)
    elif t == Q8_0:
        # q = round(x / d) against the binary32 d, dequantised with fp16(d):
        # |err| <= d/2 + 127 |fp16(d) - d| <= d (1/2 + 127 * 2^-11)
        amax = np.abs(f.reshape(16, -1, 32)).max(-1, keepdims=True).astype(np.float64)
        bound = amax / 127 * (0.5 + 127 * 2**-11) * 1.001 + 1e-9
        assert np.all(err.reshape(16, -1, 32) <= bound)
    else:
        # Per 32-value sub-block j of span S_j = max - min(min, 0): the 6-bit
        # scale is nearest(S_j/15 / d) with d = max_j(S_j/15)/63, so the step
        # d*sc_j is within d/2 of S_j/15 and the 15-step grid can fall short of
        # the span by at most 7.5 d; the 6-bit min adds at most dmin/2.
        x = f.reshape(16, 4, 8, 32).astype(np.float64)
        lo = np.minimum(x.min(-1), 0)
        span = x.max(-1) - lo
        d = (span / 15).max(-1, keepdims=True) / 63 * (1 + 2**-10)
        dmin = (-lo).max(-1, keepdims=True) / 63 * (1 + 2**-10)
        bound = 0.5 * (span / 15 + 0.5 * d) + 7.5 * d + 0.5 * dmin + 1e-9
        assert np.all(err.reshape(16, 4, 8, 32).max(-1) <= bound)
        assert np.sqrt((err.astype(np.float64) ** 2).mean()) < 0.15 * 0.02


# --- Q6_K ------------------------------------------------------------------
# block_q6_K: ql[128] (low 4 bits), qh[64] (high 2 bits), scales[16] (int8,
# one per 16 weights), d (f16): 210 bytes.
def _q6k_ggml_loop(ql, qh, sc, d):
    """ggml's dequantize_row_q6_K loop structure for one super-block, written
    out here as the published format describes it: two halves of 128 weights,
    each of 32 columns l holding four weights l, l+32, l+64, l+96 from the
    low nibbles of ql[l], ql[l+32], their high nibbles, and the 2-bit fields
    0, 2, 4, 6 of qh[l]; the scale of weight l + 32 k is sc[l // 16 + 2 k]."""
    y = np.zeros(256, np.float64)
    for half in range(2):
        L, H, S = ql[64 * half:], qh[32 * half:], sc[8 * half:]
        for l in range(32):
            is_ = l // 16
            q1 = ((int(L[l]) & 15) | (((int(H[l]) >> 0) & 3) << 4)) - 32
            q2 = ((int(L[l + 32]) & 15) | (((int(H[l]) >> 2) & 3) << 4)) - 32
            q3 = ((int(L[l]) >> 4) | (((int(H[l]) >> 4) & 3) << 4)) - 32
            q4 = ((int(L[l + 32]) >> 4) | (((int(H[l]) >> 6) & 3) << 4)) - 32
            y[128 * half + l] = d * S[is_] * q1
            y[128 * half + l + 32] = d * S[is_ + 2] * q2
            y[128 * half + l + 64] = d * S[is_ + 4] * q3
            y[128 * half + l + 96] = d * S[is_ + 6] * q4
    return y


def _q6k_block(ql, qh, sc, d_bits):
    return np.frombuffer(bytes(ql) + bytes(qh) + np.asarray(sc, np.int8).tobytes() +
                         np.array([d_bits], np.uint16).tobytes(), np.uint8)


def test_q6k_dequant_known_block(O):
    # d = 0.5; ql[i] = i (so nibbles vary), qh[i] = 0b11100100 (fields 0, 1, 2, 3),
    # scales 1..8 then -1..-8
    ql = list(range(128))
    qh = [0xE4] * 64
    sc = list(range(1, 9)) + [-k for k in range(1, 9)]
    blk = _q6k_block(ql, qh, sc, 0x3800)
    assert blk.size == 210
    y = O.dequant_rows(Q6_K, blk, 1, 256)[0]
    # worked by hand:
    #  w0:   low nibble of ql[0]=0, qh field 0 = 0  -> q=0  -> 0.5*1*(0-32)  = -16
    #  w33:  low nibble of ql[33]=1, field 1 = 1    -> q=17 -> 0.5*sc[2]=3 * -15 = -22.5
    #  w70:  high nibble of ql[6]=0, field 2 = 2    -> q=32 -> 0
    #  w127: high nibble of ql[63]=3, field 3 = 3   -> q=51 -> 0.5*sc[7]=8 * 19 = 76
    #  w200: half 1, r=72: k=2, l=8: high nibble of ql[72]=4, field 2 -> q=36 -> 0.5*sc[12]=-5 * 4 = -10
    assert y[0] == np.float32(-16.0)
    assert y[33] == np.float32(-22.5)
    assert y[70] == np.float32(0.0)
    assert y[127] == np.float32(76.0)
    assert y[200] == np.float32(-10.0)
    assert np.array_equal(y.astype(np.float64), _q6k_ggml_loop(ql, qh, sc, 0.5))


def test_q6k_dequant_random_blocks(O):
    """Every quant value at every position class, negative and zero scales,
    negative d: the oracle's decoder against the published loop."""
    rng = np.random.default_rng(11)
    for trial in range(40):
        ql = rng.integers(0, 256, 128, dtype=np.uint8)
        qh = rng.integers(0, 256, 64, dtype=np.uint8)
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        dh = np.float16(rng.choice([-1, 1]) * rng.uniform(1e-4, 2.0))
        blk = _q6k_block(ql, qh, sc, dh.view(np.uint16))
        y = O.dequant_rows(Q6_K, blk, 1, 256)[0]
        ref = _q6k_ggml_loop(ql, qh, sc.astype(np.float64), float(dh))
        assert np.array_equal(y.astype(np.float64), ref), trial   # exact in binary32


def test_q6k_quantiser_nearest_step(O):
    """The synthetic Q6_K quantiser: each weight's quant is the nearest step
    of its sub-block's d*sc grid within -32..31, and the sub-block's value of
    largest magnitude lands on quant -32 unless its scale had to be clamped
    or rounded away from -v/32."""
    rng = np.random.default_rng(12)
    f = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    f[0, :16] = 0.0                                        # an all-zero sub-block
    q = O.quantize_rows(Q6_K, f)
    assert q.shape == (8, 4 * 210)
    y = O.dequant_rows(Q6_K, q, 8, 1024).astype(np.float64)
    blk = q.reshape(8, 4, 210)
    d = blk[:, :, 208:210].copy().view(np.float16).astype(np.float64)[..., 0]
    sc = blk[:, :, 192:208].view(np.int8).astype(np.float64)
    step = (d[..., None] * sc)                               # [8, 4, 16]
    x = f.reshape(8, 4, 16, 16).astype(np.float64)
    qv = np.rint(y.reshape(8, 4, 16, 16) / np.where(step == 0, 1, step)[..., None])
    assert np.all((qv >= -32) & (qv <= 31))
    t = x / np.where(step == 0, 1, step)[..., None]
    inside = (t > -32.5) & (t < 31.5) & (step[..., None] != 0)
    assert np.all(np.abs(t - qv)[inside] <= 0.5 + 1e-5)
    assert np.all(y.reshape(8, 4, 16, 16)[0, 0, 0] == 0.0)
    err = np.abs(y - f)
    assert np.sqrt((err ** 2).mean()) < 0.03 * 0.02


def test_q6k_dot_known_answer(O):
    """All quants 33 (value +1), scales 1..16, d = 1; activations all 1 with
    d = 1: the dot is sum_j 16 (j + 1) = 2176; with the quants 31 (value -1)
    and the activations' sign alternating per sub-block it is
    -sum_j (-1)^j 16 (j + 1) = 128."""
    ql = [0x11] * 128                                      # low nibbles 1
    qh = [0xAA] * 64                                       # every field 2: q = 1 | 32 = 33
    sc = list(range(1, 17))
    w = _q6k_block(ql, qh, sc, 0x3C00)
    x = np.ones((1, 256), np.float32) * 127.0
    xq = O.quantize_act(Q8_K, x)                           # q = 127 * (-127 / 127) ... d = -1
    xd, xqs, _ = _q8K_unpack(xq[0])
    assert abs(O.vec_dot(Q6_K, 256, w, xq[0]) - 2176 * 127.0) <= 1e-3
    ql2 = [0xFF] * 128                                     # low nibbles 15
    qh2 = [0x55] * 64                                      # every field 1: q = 15 | 16 = 31
    w2 = _q6k_block(ql2, qh2, sc, 0x3C00)
    xs = np.repeat(np.where(np.arange(16) % 2 == 0, 1.0, -1.0), 16).astype(np.float32)[None] * 127.0
    got = O.vec_dot(Q6_K, 256, w2, O.quantize_act(Q8_K, xs)[0])
    assert abs(got - 127.0 * -sum((-1) ** j * 16 * (j + 1) for j in range(16))) <= 1e-3


# --- activation quantisers (vec_dot_type) ------------------------------------
def _q8K_unpack(b):
    d = b[:4].view(np.float32)[0]
    qs = b[4:260].view(np.int8)
    bs = b[260:292].view(np.int16)
    return d, qs, bs


def test_act_q8K_known_block(O):
    # the value of largest magnitude is -127, so iscale = -127/-127 = 1 exactly
    # and the other values land on exact rounding ties
    x = np.zeros(256, np.float32)
    x[10] = -127.0
    x[11] = 127.0            # same magnitude later: not the reference value
    x[0], x[1], x[2], x[3] = 2.5, 3.5, -2.5, 0.5     # ties -> 2, 4, -2, 0 (to even)
    x[16] = 100.4
    b = O.quantize_act(Q8_K, x[None])[0]
    d, qs, bs = _q8K_unpack(b)
    assert d == np.float32(1.0)
    assert qs[10] == -127 and qs[11] == 127
    assert list(qs[:4]) == [2, 4, -2, 0]
    assert qs[16] == 100
    assert np.array_equal(bs, qs.astype(np.int32).reshape(16, 16).sum(1))
    # scaled case: max magnitude 2 (negative) -> iscale 63.5, q = rint(63.5 x)
    y = np.zeros(256, np.float32)
    y[3], y[4] = -2.0, 1.0
    d2, qs2, _ = _q8K_unpack(O.quantize_act(Q8_K, y[None])[0])
    assert d2 == np.float32(1.0) / np.float32(63.5)
    assert qs2[3] == -127 and qs2[4] == 64          # 63.5 -> 64 (tie to even)


def test_act_q8K_max_sign_and_zero_block(O):
    x = np.zeros((2, 256), np.float32)
    x[0, 5] = 3.0
    x[0, 9] = -3.0          # tie in magnitude: the first (positive) one is the reference
    b = O.quantize_act(Q8_K, x)
    d, qs, bs = _q8K_unpack(b[0])
    assert qs[5] == -127 and qs[9] == 127 and d < 0
    d1, qs1, bs1 = _q8K_unpack(b[1])
    assert d1 == 0 and not qs1.any() and not bs1.any()


def test_act_q8_0_half_away_from_zero(O):
    x = np.zeros(32, np.float32)
    x[0] = 127.0              # d = 1
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 3.5, -0.5
    b = O.quantize_act(Q8_0, x[None])[0]
    d = b[:2].view(np.float16)[0]
    qs = b[2:34].view(np.int8)
    assert d == 1.0
    assert list(qs[:5]) == [127, 3, -3, 4, -1]


# --- dots ------------------------------------------------------------------
def _act_values(at, b, n):
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


@pytest.mark.parametrize("t", [F32, F16, Q8_0, Q4_K, Q6_K])
def test_vec_dot_matches_float64(O, t):
    at = {F32: F32, F16: F16, Q8_0: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K}[t]
    rng = np.random.default_rng(2)
    n = 1024
    for trial in range(20):
        w = (rng.standard_normal((1, n)) * 0.02).astype(np.float32)
        x = rng.standard_normal((1, n)).astype(np.float32)
        wq = O.quantize_rows(t, w)
        xq = O.quantize_act(at, x)
        got = O.vec_dot(t, n, wq[0], xq[0])
        wd = O.dequant_rows(t, wq, 1, n)[0].astype(np.float64)
        ref = float(np.dot(wd, _act_values(at, xq[0], n)))
        scale = float(np.abs(wd).dot(np.abs(_act_values(at, xq[0], n))))
        assert abs(got - ref) <= 1e-5 * scale, (trial, got, ref)


# --- exp ---------------------------------------------------------------------
def test_expf_correctly_rounded(O):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-110, 100, 10_000_000).astype(np.float32),
                        np.linspace(-104, 89, 100001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 88.72283, 88.7229, -87.33655,
                                  -103.97208, -104.0, 100.0, 1000.0, -1000.0], np.float32)])
    got = O.expf(x)
    with np.errstate(over="ignore", under="ignore"):
        ref = np.exp(x.astype(np.float64)).astype(np.float32)
    same = got.view(np.uint32) == ref.view(np.uint32)
    # correctly rounded except (rarely) within ~1e-16 of a rounding boundary
    assert same.mean() > 1 - 1e-6
    diff = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert diff.max() <= 1
    assert np.isnan(O.expf(np.array([np.nan], np.float32))[0])
    assert O.expf(np.array([np.inf], np.float32))[0] == np.inf
    assert O.expf(np.array([-np.inf], np.float32))[0] == 0.0


def test_sigmoid_limits(O):
    assert O.sigmoid(0.0) == 0.5
    assert O.sigmoid(200.0) == 1.0
    assert O.sigmoid(-200.0) == 0.0
    v = np.float32(1.5)
    e = np.exp(np.float64(-v)).astype(np.float32)
    assert O.sigmoid(float(v)) == np.float32(1.0) / (np.float32(1.0) + e)
