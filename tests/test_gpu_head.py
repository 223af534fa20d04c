"""GPU parity of the step tail (dmoe_head_*: final RMSNorm, LM head,
temperature-0 argmax and confidence; src/diffuse-moe-graph.cpp:295-300,
src/diffuse-sampler.cpp:29-49) through the C ABI against the oracle.

Bars: logits max|l - l_oracle| / max|l_oracle| <= 5e-4 for the int8-digit and
f16-pair paths (F32 weight semantics with about 16-bit activations; the
dense MLP's measured error is 1.2e-4) and 1e-5 for plain F32; confidence
within 1e-3 relative (the oracle adds the exponentials in float,
sequentially, as the reference does, the GPU hardware-exp2 terms in
binary64 in a fixed tree); the
token equals the oracle's wherever the oracle's top two logits are further
apart than twice the logit tolerance (closer ones may swap within it, and
then the GPU's token must be one of the two)."""
import numpy as np
import pytest

from conftest import max_rel_err

pytestmark = pytest.mark.gpu

TOL = {12: 5e-4, 14: 5e-4, 8: 5e-4, 1: 5e-4, 0: 1e-5}
PATH = {12: "q4k_mfma", 14: "q6k_mfma", 8: "q80_mfma", 1: "f16_gemm", 0: "gemv"}


def _say(msg):
    print(msg, flush=True)


def _check(tok, prob, lg, tr, pr, lr, tol):
    err = max_rel_err(lg, lr)
    assert err <= tol, err
    assert np.all(np.abs(prob - pr) <= 1e-3 * np.abs(pr)), np.abs(prob / pr - 1).max()
    srt = np.sort(lr, axis=1)
    gap = srt[:, -1] - srt[:, -2]
    clear = gap > 2 * tol * np.abs(lr).max()
    assert np.array_equal(tok[clear], tr[clear])
    for t in np.nonzero(~clear)[0]:
        top2 = np.argsort(lr[t])[-2:]
        assert tok[t] in top2
    return err


@pytest.mark.parametrize("wtype", [12, 14, 8, 1, 0], ids=["Q4_K", "Q6_K", "Q8_0", "F16", "F32"])
@pytest.mark.parametrize("N", [32, 40])
def test_head_small(ctx, O, wtype, N):
    from dmoe import synth
    H, V = 512, 4096
    _say(f"case: step tail H={H} V={V} type={wtype} N={N}")
    w = synth.host_head(H, V, wtype, 70 + wtype, O.quantize_rows)
    h = (synth.normal(70 + N, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    head = ctx.head_upload(w)
    assert head.kernel_path() == PATH[wtype]
    tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
    tr, pr, lr = O.head_forward(w, h, 1e-6)
    err = _check(tok, prob, lg, tr, pr, lr, TOL[wtype])
    _say(f"  logits max rel err {err:.3e}")
    t2, p2 = ctx.head_forward(head, h, 1e-6)                  # without the logits copy
    assert np.array_equal(t2, tok) and np.array_equal(p2, prob)
    head.free()


@pytest.mark.parametrize("wtype", [12, 14], ids=["Q4_K", "Q6_K"])
@pytest.mark.parametrize("N", [1, 9, 17, 25, 72])
def test_head_q4k_column_blocks(ctx, O, N, wtype):
    """The few-token projection at each column-block count (1 to 4 blocks of
    8 tokens, the last one partly filled), Q4_K and Q6_K, against the
    oracle; 72 tokens: Q6_K in chunks of 32, 32 and 8 tokens."""
    from dmoe import synth
    H, V = 512, 4096
    _say(f"case: step tail type={wtype} H={H} V={V} N={N}")
    w = synth.host_head(H, V, wtype, 90 + N, O.quantize_rows)
    h = (synth.normal(91 + N, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    head = ctx.head_upload(w)
    assert head.kernel_path() == PATH[wtype]
    tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
    tr, pr, lr = O.head_forward(w, h, 1e-6)
    err = _check(tok, prob, lg, tr, pr, lr, TOL[wtype])
    _say(f"  logits max rel err {err:.3e}")
    head.free()


def test_head_gemv_vocab(ctx, O):
    """A vocabulary that is not a whole number of row groups: GEMV kernels."""
    from dmoe import synth
    w = synth.host_head(512, 1000, 8, 77, O.quantize_rows)
    h = synth.normal(77, synth.S_X, 16 * 512).reshape(16, 512)
    head = ctx.head_upload(w)
    assert head.kernel_path() == "gemv"
    tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
    tr, pr, lr = O.head_forward(w, h, 1e-6)
    _check(tok, prob, lg, tr, pr, lr, 1e-5)


@pytest.mark.parametrize("wtype", [8, 12, 14], ids=["Q8_0", "Q4_K", "Q6_K"])
def test_head_flash(ctx, O, wtype):
    """LLaDA2-flash's step tail: hidden 4096, 157184 tokens of vocabulary,
    32 positions, device weights (Q6_K: the output.weight type of the
    reference's Q4_K schemes); the device forward writes tokens and probs
    only, equal to the host forward's."""
    import torch
    from dmoe import synth
    H, V = synth.HEAD_FLASH
    N = 32
    _say(f"case: flash step tail type={wtype} V={V} N={N}")
    wd = synth.device_head(H, V, wtype, 5, ctx)
    head = ctx.head_wrap_device(wd)
    h = (synth.normal(5, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
    tr, pr, lr = O.head_forward(synth.head_to_host(wd), h, 1e-6)
    err = _check(tok, prob, lg, tr, pr, lr, TOL[wtype])
    _say(f"  logits max rel err {err:.3e}")
    hd = torch.from_numpy(h).cuda()
    td = torch.zeros(N, dtype=torch.int32, device="cuda")
    pd = torch.zeros(N, dtype=torch.float32, device="cuda")
    ctx.head_forward_device(head, hd, N, 1e-6, td, pd, None, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(td.cpu().numpy(), tok) and np.array_equal(pd.cpu().numpy(), prob)
    head.free()
    del wd
    torch.cuda.empty_cache()


def test_head_errors(ctx, O):
    import dmoe
    from dmoe import synth
    _say("case: step tail argument errors")
    w = synth.host_head(512, 1024, 12, 3, O.quantize_rows)
    head = ctx.head_upload(w)
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.forward(head, np.zeros((32, 512), np.float32))    # not a MoE layer
    assert ei.value.code == dmoe._abi.ERR_INVALID_ARG
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.head_forward(head, np.zeros((4, 512), np.float32), -1.0)
    assert ei.value.code == dmoe._abi.ERR_INVALID_ARG
    head.free()
    import ctypes as C
    nv, ov = w.norm_view(), w.output_view()
    nv.ne[0] = 256                                            # norm shorter than n_embd
    out = C.c_void_p()
    rc = dmoe.load().dmoe_head_upload(ctx.handle, 512, 1024, C.byref(nv), C.byref(ov), C.byref(out))
    assert rc == dmoe._abi.ERR_SHAPE and not out.value


def _tie_head(H, V, wtype, quantize_rows, h, g, plan, nan_rows=()):
    """An output matrix whose rows listed in plan[t] are all equal and point
    along position t's normalised hidden state (so they hold that position's
    largest logit, bit-equal across the copies: equal weight rows give equal
    logits on every kernel path); the other rows N(0, 0.02).  nan_rows are
    set to NaN (F32 only)."""
    from dmoe import HeadWeights, row_size, synth
    f = synth.normal(404, synth.S_OUT, V * H, 0.02).reshape(V, H).astype(np.float32)
    hn = h / np.sqrt((h.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    u = hn * g
    for t, rows in enumerate(plan):
        d = (0.5 * u[t] / np.linalg.norm(u[t])).astype(np.float32)
        for r in rows:
            f[r] = d
    for r in nan_rows:
        f[r] = np.nan
    out = np.ascontiguousarray(quantize_rows(wtype, f)).view(np.uint8).reshape(V, row_size(wtype, H))
    return HeadWeights(n_embd=H, n_vocab=V, wtype=wtype, norm=g, output=out)


@pytest.mark.parametrize("wtype", [12, 0], ids=["Q4_K", "F32"])
def test_head_argmax_ties(ctx, O, wtype):
    """The sampler's argmax rule on the GPU (src/diffuse-sampler.cpp:33-40:
    the first index of the largest logit): equal largest logits inside one
    4096-logit chunk (one thread's two values, two threads), in chunks far
    apart, across a chunk boundary, three copies over three chunks, and a
    largest logit at the very last index; the token is the lower index every
    time, as the oracle's."""
    from dmoe import synth
    H, V = 512, 16384
    plan = [(100, 200), (4000, 9000), (V - 1,), (4095, 4096), (5, V - 2), (8191, 8192, 12000),
            (12295, 12588), (259, 3)]
    expect = np.array([min(r) for r in plan], np.int32)
    N = len(plan)
    _say(f"case: argmax ties, type={wtype}, V={V}, N={N}")
    h = (synth.normal(405, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    g = synth.uniform(405, synth.S_ONORM, H, 0.5, 1.5)
    w = _tie_head(H, V, wtype, O.quantize_rows, h, g, plan)
    head = ctx.head_upload(w)
    tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
    tr, pr, lr = O.head_forward(w, h, 1e-6)
    for t, rows in enumerate(plan):
        vals = lg[t, list(rows)].view(np.uint32)
        assert np.all(vals == vals[0]), (t, rows)            # the copies' logits are bit-equal
        assert lg[t, rows[0]] == lg[t].max()
    assert np.array_equal(tr, expect)
    assert np.array_equal(tok, expect), (tok, expect)
    assert np.all(np.abs(prob - pr) <= 1e-3 * np.abs(pr))
    head.free()


def test_head_argmax_nan(ctx, O):
    """NaN logits on the GPU as the sampler's loop treats them
    (src/diffuse-sampler.cpp:34-40): a NaN never becomes the maximum, so a
    NaN at index 0 keeps index 0 for the row, and one later in the row leaves
    the argmax where it was; the confidence is NaN either way (its sum has a
    NaN term).  F32 weights with a NaN row give a NaN logit at that index in
    every row."""
    from dmoe import synth
    H, V = 512, 16384
    plan = [(100, 200), (4000, 9000), (V - 1,), (4095, 4096)]
    N = len(plan)
    h = (synth.normal(406, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    g = synth.uniform(406, synth.S_ONORM, H, 0.5, 1.5)
    for nan_row, expect in ((0, np.zeros(N, np.int32)), (4097, np.array([100, 4000, V - 1, 4095], np.int32))):
        _say(f"case: argmax with NaN logits at index {nan_row}")
        w = _tie_head(H, V, 0, O.quantize_rows, h, g, plan, nan_rows=(nan_row,))
        head = ctx.head_upload(w)
        tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
        tr, pr, _ = O.head_forward(w, h, 1e-6)
        assert np.isnan(lg[:, nan_row]).all()
        assert np.array_equal(tr, expect)
        assert np.array_equal(tok, expect), (tok, expect)
        assert np.isnan(pr).all() and np.isnan(prob).all()
        head.free()
