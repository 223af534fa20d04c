"""CPU: pins the oracle's attention half of the layer (dmo_rope_neox,
dmo_attn_forward; src/diffuse-moe-graph.cpp:116-178) against independent
float64 restatements:

- RoPE against the rotate_half formulation (cos / sin of the angles
  repeated over both halves), with the oracle's own f32 angle chain and with
  the closed-form angles pos * base^(-2i/n); identity at position 0, the
  pass-through of dims past rotary_dim, and the pair norms.
- The whole attention half against float64 numpy: the mask built as
  tril(ones(n_blocks)) repeated block_length times along both axes (the
  construction the reference's mask comment names), GQA by repeating each
  kv head over its group, full softmax; block_length 1 also against torch's
  scaled_dot_product_attention(is_causal=True).  Each case also checks that
  the plausible mistakes (transposed mask, kv head h % n_head_kv, no
  scale) would have failed.
"""
import numpy as np
import pytest

import dmoe
from dmoe import synth

import oracle as O

F32 = dmoe.TYPE_F32


@pytest.fixture(autouse=True)
def _oracle_built(request):
    request.getfixturevalue("O")          # builds oracle/libdmoe_oracle.so once


def _rot_half64(x, n, theta):
    """rotate_half RoPE of the first n dims of x in float64 at angles theta[n/2]."""
    x = np.asarray(x, np.float64)
    emb = np.concatenate([theta, theta])
    c, s = np.cos(emb), np.sin(emb)
    xr = x[:n]
    rh = np.concatenate([-xr[n // 2:], xr[:n // 2]])
    return np.concatenate([xr * c + rh * s, x[n:]])


def _chain(pos, n, base):
    ts = np.float32(np.float64(base) ** (-2.0 / n))
    th = np.float32(pos)
    out = []
    for _ in range(n // 2):
        out.append(np.float64(th))
        th = np.float32(th * ts)
    return np.array(out)


@pytest.mark.parametrize("pos", [1, 7, 31, 255, 1000])
@pytest.mark.parametrize("hd,n,base", [(128, 64, 3e6), (64, 64, 1e4), (128, 128, 1e6)])
def test_rope_rotate_half(pos, hd, n, base):
    x = synth.normal(3, pos, hd)
    y = O.rope_neox(x, n, pos, base)
    ref = _rot_half64(x, n, _chain(pos, n, base))
    scale = np.abs(x).max()
    assert np.abs(y - ref).max() <= 4e-6 * scale * max(1.0, np.log2(pos + 1))
    # closed-form angles: the f32 chain drifts by a few ulp of each angle
    closed = _rot_half64(x, n, pos * np.float64(base) ** (-2.0 * np.arange(n // 2) / n))
    assert np.abs(y - closed).max() <= 2e-6 * scale * (pos + 1)
    # a GPT-J (interleaved) pairing or a -1/n exponent is far off
    gptj = np.array(x, np.float64)
    th = pos * np.float64(base) ** (-2.0 * np.arange(n // 2) / n)
    gptj[0:n:2] = x[0:n:2] * np.cos(th) - x[1:n:2] * np.sin(th)
    gptj[1:n:2] = x[0:n:2] * np.sin(th) + x[1:n:2] * np.cos(th)
    assert np.abs(y - gptj).max() > 1e-2 * scale
    wrong = _rot_half64(x, n, pos * np.float64(base) ** (-1.0 * np.arange(n // 2) / n))
    assert np.abs(y - wrong).max() > 1e-2 * scale


def test_rope_invariants():
    x = synth.normal(4, 1, 128)
    assert np.array_equal(O.rope_neox(x, 64, 0, 3e6), x)           # angle 0
    y = O.rope_neox(x, 64, 123, 3e6)
    assert np.array_equal(y[64:], x[64:])                           # past rotary_dim
    n0 = np.hypot(x[:32].astype(np.float64), x[32:64])
    n1 = np.hypot(y[:32].astype(np.float64), y[32:64])
    np.testing.assert_allclose(n1, n0, rtol=1e-6)


# ---------------------------------------------------------------------------
def _rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    r = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return r if w is None else r * np.asarray(w, np.float64)


def attn_ref64(w: dmoe.AttnWeights, h, mask_fn=None, kv_map=None, scale=None):
    """The attention half in float64; mask_fn / kv_map / scale override the
    model's to check what a mistake would give."""
    N, H = h.shape
    NH, NKV, HD, RD = w.n_head, w.n_head_kv, w.head_dim, w.rotary_dim
    QD, KD = NH * HD, NKV * HD
    Wqkv = O.dequant_rows(w.wtype, w.qkv, w.qkv_dim, H).astype(np.float64)
    Wo = O.dequant_rows(w.wtype, w.wo, H, QD).astype(np.float64)
    xn = _rms64(h, w.attn_norm, w.rms_eps)
    qkv = xn @ Wqkv.T
    Q = qkv[:, :QD].reshape(N, NH, HD)
    K = qkv[:, QD:QD + KD].reshape(N, NKV, HD)
    V = qkv[:, QD + KD:].reshape(N, NKV, HD)
    if w.q_norm is not None:
        Q = _rms64(Q, w.q_norm, w.rms_eps)
        K = _rms64(K, w.k_norm, w.rms_eps)
    ang = np.arange(N)[:, None] * np.float64(w.rope_base) ** (-2.0 * np.arange(RD // 2) / RD)

    def rope(X):
        X = X.copy()
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a, b = X[..., :RD // 2].copy(), X[..., RD // 2:RD].copy()
        X[..., :RD // 2] = a * c - b * s
        X[..., RD // 2:RD] = a * s + b * c
        return X
    Q, K = rope(Q), rope(K)
    B = w.block_length
    if mask_fn is not None:
        allow = mask_fn(N, B)
    elif B <= 0:
        allow = np.ones((N, N), bool)
    else:
        nb = (N + B - 1) // B
        allow = np.kron(np.tril(np.ones((nb, nb))), np.ones((B, B)))[:N, :N] > 0
    g = NH // NKV
    kv = np.arange(NH) // g if kv_map is None else kv_map
    sc = 1.0 / np.sqrt(HD) if scale is None else scale
    att = np.empty((N, NH, HD))
    for hh in range(NH):
        S = (Q[:, hh] @ K[:, kv[hh]].T) * sc
        S = np.where(allow, S, -np.inf)
        P = np.exp(S - S.max(-1, keepdims=True))
        P /= P.sum(-1, keepdims=True)
        att[:, hh] = P @ V[:, kv[hh]]
    h_out = h.astype(np.float64) + att.reshape(N, QD) @ Wo.T
    return h_out, _rms64(h_out, w.post_norm, w.rms_eps)


CASES = [
    # n_embd, n_head, n_head_kv, head_dim, rotary_dim, block, qk_norm, N
    (256, 4, 2, 64, 32, 8, True, 40),
    (256, 4, 1, 64, 64, 16, False, 33),
    (512, 4, 4, 128, 64, 32, True, 70),
    (256, 8, 2, 64, 32, 0, True, 24),
    (256, 4, 2, 64, 32, 1, True, 20),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"H{c[0]}_h{c[1]}kv{c[2]}_d{c[3]}r{c[4]}_B{c[5]}_N{c[7]}")
def test_attention_vs_float64(case):
    H, NH, NKV, HD, RD, B, qk, N = case
    w = synth.host_attn(F32, 11, O.quantize_rows, H, NH, NKV, HD, RD, block_length=B, qk_norm=qk, w_std=0.05)
    h = synth.normal(12, 1, N * H).reshape(N, H)
    h_out, moe_in = O.attn_forward(w, h)
    r_out, r_in = attn_ref64(w, h)
    tol = 1e-4
    assert np.abs(h_out - r_out).max() <= tol * np.abs(r_out).max()
    assert np.abs(moe_in - r_in).max() <= tol * np.abs(r_in).max()
    err = lambda r: np.abs(h_out - r[0]).max()
    if 0 < B < N:
        assert err(attn_ref64(w, h, mask_fn=lambda n, b: (np.arange(n)[None] // b >= np.arange(n)[:, None] // b))) > 10 * tol
    if NKV > 1 and NH // NKV > 1:
        assert err(attn_ref64(w, h, kv_map=np.arange(NH) % NKV)) > 10 * tol
    assert err(attn_ref64(w, h, scale=1.0)) > 10 * tol


def test_attention_causal_matches_torch_sdpa():
    """block_length 1 is the causal mask: the oracle's attention output
    against torch's scaled_dot_product_attention(is_causal=True) on the same
    roped Q / K / V (float64)."""
    torch = pytest.importorskip("torch")
    H, NH, NKV, HD, RD, N = 256, 4, 2, 64, 32, 24
    w = synth.host_attn(F32, 21, O.quantize_rows, H, NH, NKV, HD, RD, block_length=1, qk_norm=True,
                        w_std=0.05)
    h = synth.normal(22, 1, N * H).reshape(N, H)
    h_out, _ = O.attn_forward(w, h)
    # the same computation with the attention core replaced by torch's
    Wqkv = O.dequant_rows(F32, w.qkv, w.qkv_dim, H).astype(np.float64)
    Wo = O.dequant_rows(F32, w.wo, H, NH * HD).astype(np.float64)
    qkv = _rms64(h, w.attn_norm, w.rms_eps) @ Wqkv.T
    QD, KD = NH * HD, NKV * HD
    Q = _rms64(qkv[:, :QD].reshape(N, NH, HD), w.q_norm, w.rms_eps)
    K = _rms64(qkv[:, QD:QD + KD].reshape(N, NKV, HD), w.k_norm, w.rms_eps)
    V = qkv[:, QD + KD:].reshape(N, NKV, HD)
    ang = np.arange(N)[:, None] * np.float64(w.rope_base) ** (-2.0 * np.arange(RD // 2) / RD)
    for X in (Q, K):
        a, b = X[..., :RD // 2].copy(), X[..., RD // 2:RD].copy()
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        X[..., :RD // 2] = a * c - b * s
        X[..., RD // 2:RD] = a * s + b * c
    tq = torch.from_numpy(Q).permute(1, 0, 2)
    tk = torch.from_numpy(np.repeat(K, NH // NKV, axis=1)).permute(1, 0, 2)
    tv = torch.from_numpy(np.repeat(V, NH // NKV, axis=1)).permute(1, 0, 2)
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    ref = h + o.permute(1, 0, 2).reshape(N, QD).numpy() @ Wo.T
    assert np.abs(h_out - ref).max() <= 1e-4 * np.abs(ref).max()


def test_full_block_equals_bidirectional():
    """block_length >= N puts every token in block 0: the same as no mask."""
    H, NH, NKV, HD, RD, N = 256, 4, 2, 64, 32, 16
    a = synth.host_attn(F32, 31, O.quantize_rows, H, NH, NKV, HD, RD, block_length=32)
    b = synth.host_attn(F32, 31, O.quantize_rows, H, NH, NKV, HD, RD, block_length=0)
    h = synth.normal(32, 1, N * H).reshape(N, H)
    assert np.array_equal(O.attn_forward(a, h)[0], O.attn_forward(b, h)[0])


def test_attention_quantized_weights():
    """Q4_K projections: the oracle against float64 on the dequantised rows."""
    H, NH, NKV, HD, RD, N = 256, 4, 2, 64, 32, 24
    w = synth.host_attn(dmoe.TYPE_Q4_K, 41, O.quantize_rows, H, NH, NKV, HD, RD, block_length=8)
    h = synth.normal(42, 1, N * H).reshape(N, H)
    h_out, moe_in = O.attn_forward(w, h)
    r_out, r_in = attn_ref64(w, h)
    assert np.abs(h_out - r_out).max() <= 1e-4 * np.abs(r_out).max()
    assert np.abs(moe_in - r_in).max() <= 1e-4 * np.abs(r_in).max()
