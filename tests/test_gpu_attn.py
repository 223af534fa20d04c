"""GPU parity of the attention half of the layer (dmoe_attn_*: input RMSNorm,
fused QKV, QK RMSNorm, partial NEOX RoPE, block-causal flash attention with
GQA, output projection, residual and post-attention RMSNorm;
src/diffuse-moe-graph.cpp:116-178) through the C ABI against the oracle.

Bar: max|y - y_oracle| / max|y_oracle| <= 1e-4 for h_out and for the MoE
input with Q4_K / Q8_0 projections (int8 digits of the activations: measured
2.0e-5 at the flash shape), 1e-5 with F16 / F32 projections (measured
1.5e-7); the attention itself runs in fp32 on MFMA with another summation
order and expf per 64-key tile.  Edge cases: ragged last block
and ragged 64-query tile, block_length 0 (bidirectional) and 1 (causal),
n_head == n_head_kv, no QK norm, rotary_dim == head_dim, head_dim 64 and 128,
the flash shape (n_embd 4096, 32 / 4 heads of 128, RoPE over 64 dims)."""
import numpy as np
import pytest

from conftest import max_rel_err

pytestmark = pytest.mark.gpu

TOL = {12: 1e-4, 14: 1e-4, 8: 1e-4, 1: 1e-5, 0: 1e-5}
PATH = {12: "q4k_mfma", 14: "q6k_mfma", 8: "q80_mfma", 1: "f16_gemm", 0: "gemv"}


def _say(msg):
    print(msg, flush=True)


def _run(ctx, O, w, N, seed, tol):
    from dmoe import synth
    h = (synth.normal(seed, synth.S_X, N * w.n_embd).reshape(N, w.n_embd) * 2).astype(np.float32)
    layer = ctx.attn_upload(w)
    h_out, moe_in = ctx.attn_forward(layer, h)
    r_out, r_in = O.attn_forward(w, h)
    e1, e2 = max_rel_err(h_out, r_out), max_rel_err(moe_in, r_in)
    _say(f"  h_out err {e1:.3e}  moe_in err {e2:.3e}")
    assert e1 <= tol and e2 <= tol, (e1, e2)
    return layer, h, h_out, moe_in


@pytest.mark.parametrize("wtype", [12, 14, 8, 1, 0], ids=["Q4_K", "Q6_K", "Q8_0", "F16", "F32"])
def test_attn_small(ctx, O, wtype):
    from dmoe import synth
    _say(f"case: attn H=256 4/2 heads d64 r32 B8 N40 type={wtype}")
    w = synth.host_attn(wtype, 80 + wtype, O.quantize_rows, 256, 4, 2, 64, 32, block_length=8)
    layer, *_ = _run(ctx, O, w, 40, 81, TOL[wtype])
    assert layer.kernel_path() == PATH[wtype]
    layer.free()


SHAPES = [
    # n_embd, n_head, n_head_kv, head_dim, rotary_dim, block, qk_norm, N
    (512, 4, 4, 128, 128, 0, False, 70),
    (256, 8, 2, 64, 32, 1, True, 65),
    (512, 8, 2, 64, 64, 16, True, 130),
    (256, 4, 1, 64, 32, 64, True, 64),
    (512, 4, 2, 128, 64, 32, True, 1),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda c: f"H{c[0]}_h{c[1]}kv{c[2]}_d{c[3]}r{c[4]}_B{c[5]}_N{c[7]}")
def test_attn_shapes(ctx, O, shape):
    from dmoe import synth
    H, NH, NKV, HD, RD, B, qk, N = shape
    _say(f"case: attn {shape} Q4_K")
    w = synth.host_attn(12, 90 + N, O.quantize_rows, H, NH, NKV, HD, RD, block_length=B, qk_norm=qk)
    layer, *_ = _run(ctx, O, w, N, 91 + N, TOL[12])
    layer.free()


@pytest.fixture(scope="module")
def flash_attn(O):
    from dmoe import synth
    return synth.host_attn(12, 5, O.quantize_rows, **synth.ATTN_FLASH)


@pytest.mark.parametrize("N", [32, 256, 1024])
def test_attn_flash(ctx, O, flash_attn, N):
    _say(f"case: attn flash shape Q4_K N={N}")
    layer, *_ = _run(ctx, O, flash_attn, N, 100 + N, TOL[12])
    layer.free()


@pytest.mark.parametrize("waves", ["4", "8"])
def test_attn_waves(ctx, O, flash_attn, monkeypatch, waves):
    """The attention kernel with four or eight wavefronts per workgroup (64 or
    128 queries; the grid size picks one, the switch pins it): the flash shape
    at 256 tokens and a ragged small shape against the oracle."""
    import dmoe
    from dmoe import synth
    monkeypatch.setenv("DMOE_ATTN_WAVES", waves)
    c = dmoe.Context(0)
    monkeypatch.delenv("DMOE_ATTN_WAVES")
    try:
        _say(f"case: attn flash shape Q4_K N=256, {waves} wavefronts")
        layer, *_ = _run(c, O, flash_attn, 256, 200, TOL[12])
        layer.free()
        _say(f"case: attn H512 8/2 heads d64 B16 N=200 F32, {waves} wavefronts")
        w = synth.host_attn(0, 201, O.quantize_rows, 512, 8, 2, 64, 64, block_length=16)
        layer, *_ = _run(c, O, w, 200, 202, TOL[0])
        layer.free()
    finally:
        c.close()


def test_attn_device_entry(ctx, O, flash_attn):
    """dmoe_attn_wrap_device + dmoe_attn_forward_device on torch buffers: the
    same bits as the host-io entry; without moe_in only h_out is written."""
    import torch
    from dmoe import synth
    N = 32
    _say(f"case: attn flash device entry N={N}")
    dev = torch.device("cuda:0")
    host = ctx.attn_upload(flash_attn)
    h = (synth.normal(7, synth.S_X, N * 4096).reshape(N, 4096) * 2).astype(np.float32)
    ref_out, ref_in = ctx.attn_forward(host, h)
    wd = synth.attn_to_device(flash_attn, dev)
    layer = ctx.attn_wrap_device(wd)
    hd = torch.from_numpy(h).to(dev)
    out = torch.empty_like(hd)
    mi = torch.empty_like(hd)
    s = torch.cuda.current_stream(dev)
    ctx.attn_forward_device(layer, hd, N, out, mi, stream=s.cuda_stream)
    torch.cuda.synchronize(dev)
    assert np.array_equal(out.cpu().numpy(), ref_out)
    assert np.array_equal(mi.cpu().numpy(), ref_in)
    mi.fill_(7.0)
    ctx.attn_forward_device(layer, hd, N, out, None, stream=s.cuda_stream)
    torch.cuda.synchronize(dev)
    assert np.array_equal(out.cpu().numpy(), ref_out)
    assert bool((mi == 7.0).all())
    assert np.array_equal(hd.cpu().numpy(), h)                # the input is not written
    layer.free()
    host.free()


def test_attn_rejects(ctx, O):
    import dmoe
    from dmoe import synth
    w = synth.host_attn(12, 3, O.quantize_rows, 256, 4, 2, 64, 32)
    bad = [dict(head_dim=96, rotary_dim=32), dict(n_head_kv=3), dict(rotary_dim=66), dict(rotary_dim=31)]
    from dataclasses import replace
    for b in bad:
        with pytest.raises(dmoe.DmoeError):
            ctx.attn_upload(replace(w, **b))
    layer = ctx.attn_upload(w)
    with pytest.raises(dmoe.DmoeError):
        ctx.forward(layer, np.zeros((8, 256), np.float32))      # not a MoE layer
    dense = synth.host_dense(256, 512, 12, 4, O.quantize_rows)
    dl = ctx.dense_upload(dense)
    with pytest.raises(dmoe.DmoeError):
        ctx.attn_forward(dl, np.zeros((8, 256), np.float32))    # not an attention layer
    dl.free()
    layer.free()


@pytest.mark.parametrize("N", [32, 96])
def test_attn_flash_q6k(ctx, O, N):
    """The flash-shaped attention half with Q6_K projections (the q6_k
    scheme's attn tensors): 32 tokens through the fused norm and few-token
    kernel, 96 in chunks of 32."""
    from dmoe import synth
    _say(f"case: attn flash shape Q6_K N={N}")
    w = synth.host_attn(14, 6, O.quantize_rows, **synth.ATTN_FLASH)
    layer, *_ = _run(ctx, O, w, N, 110 + N, TOL[14])
    assert layer.kernel_path() == PATH[14]
    layer.free()
