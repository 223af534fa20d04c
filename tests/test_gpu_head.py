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

TOL = {12: 5e-4, 8: 5e-4, 1: 5e-4, 0: 1e-5}
PATH = {12: "q4k_mfma", 8: "q80_mfma", 1: "f16_gemm", 0: "gemv"}


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


@pytest.mark.parametrize("wtype", [12, 8, 1, 0], ids=["Q4_K", "Q8_0", "F16", "F32"])
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


@pytest.mark.parametrize("N", [1, 9, 17, 25])
def test_head_q4k_column_blocks(ctx, O, N):
    """The few-token projection at each column-block count (1 to 4 blocks of
    8 tokens, the last one partly filled), Q4_K, against the oracle."""
    from dmoe import synth
    H, V = 512, 4096
    _say(f"case: step tail Q4_K H={H} V={V} N={N}")
    w = synth.host_head(H, V, 12, 90 + N, O.quantize_rows)
    h = (synth.normal(91 + N, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
    head = ctx.head_upload(w)
    assert head.kernel_path() == PATH[12]
    tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
    tr, pr, lr = O.head_forward(w, h, 1e-6)
    err = _check(tok, prob, lg, tr, pr, lr, TOL[12])
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


@pytest.mark.parametrize("wtype", [8, 12], ids=["Q8_0", "Q4_K"])
def test_head_flash(ctx, O, wtype):
    """LLaDA2-flash's step tail: hidden 4096, 157184 tokens of vocabulary,
    32 positions, device weights; the device forward writes tokens and
    probs only, equal to the host forward's."""
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
