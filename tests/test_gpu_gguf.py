"""GPU: a layer loaded from a GGUF file through the C ABI (dmoe_gguf_* then
dmoe_layer_upload / dmoe_dense_upload straight from the mapping) against the
oracle on the same mapped bytes.  The file holds a dense layer 0 (hidden 4096,
n_ff 9216) and one LLaDA2-flash-shaped MoE layer 1 (256 Q4_K experts, moe_ff
1024, shared expert, F32 router and bias), written by tests/gguf_writer.py
from weights generated and quantised on the GPU.  Bars as in
test_gpu_parity.py / test_gpu_dense.py: routing bit-exact, output 3e-3 (MoE,
Q4_K) and 5e-4 (dense, F32 weight semantics)."""
import numpy as np
import pytest

from conftest import max_rel_err
from gguf_writer import GGUFWriter, STR, add_dense_layer, add_moe_layer, moe_keys

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def test_flash_layer_from_gguf(ctx, O, tmp_path):
    import torch
    from dmoe import synth
    from dmoe.gguf import GGUF
    cfg = synth.CONFIGS["flash_q4k"]
    _say("case: flash Q4_K MoE layer + dense layer 0 through a GGUF file")
    w = synth.to_host(synth.device_layer(cfg, 13, ctx))
    H, FF = synth.DENSE_FLASH
    d = synth.dense_to_host(synth.device_dense(H, FF, 12, 13, ctx))
    torch.cuda.empty_cache()
    wr = GGUFWriter()
    for k, t, v in moe_keys(w, n_layer=2, first_k_dense=1):
        wr.add(k, t, v)
    wr.add("diffuse.model_type", STR, "llada2_moe")
    add_dense_layer(wr, 0, d)
    add_moe_layer(wr, 1, w)
    path = tmp_path / "flash2.gguf"
    wr.write(path)
    del w, d
    _say(f"  wrote {path.stat().st_size / 2**30:.2f} GiB")
    with GGUF(path) as g:
        hp, n_layer, fk = g.moe_hparams()
        assert (n_layer, fk, hp.n_experts, hp.moe_ff, hp.shared_ff) == (2, 1, 256, 1024, 1024)
        lw = g.layer_weights(1)
        layer = ctx.upload(lw)
        assert layer.kernel_path() == "q4k_mfma"
        x = synth.make_x(cfg, 13)
        y, dg = ctx.forward(layer, x, debug=True)
        yr, dr = O.layer_forward(lw, x, debug=True)
        for k in ("logits", "probs", "bmax", "thr", "allowed", "idx", "weights", "counts", "offsets", "perm"):
            assert np.array_equal(np.asarray(dg[k]).view(np.uint8), np.asarray(dr[k]).view(np.uint8)), k
        err = max_rel_err(y, yr)
        _say(f"  MoE layer 1: max rel err {err:.3e}")
        assert err <= 3e-3
        layer.free()
        dw = g.dense_weights(0)
        dl = ctx.dense_upload(dw)
        yd = ctx.forward(dl, x)
        err = max_rel_err(yd, O.dense_forward(dw, x))
        _say(f"  dense layer 0: max rel err {err:.3e}")
        assert err <= 5e-4
        dl.free()
    torch.cuda.empty_cache()


def test_attention_from_gguf(ctx, O, tmp_path):
    """The flash-shaped attention half (32 / 4 heads of 128, RoPE over 64
    dims, QK norm, Q4_K projections) loaded through dmoe_gguf_attn_hparams /
    dmoe_gguf_attn_desc and dmoe_attn_upload from the mapping, against the
    oracle on the same mapped bytes (bar 1e-4, as tests/test_gpu_attn.py)."""
    from dmoe import synth
    from dmoe.gguf import GGUF
    from gguf_writer import U32, add_attn_layer, attn_keys
    _say("case: flash attention half through a GGUF file")
    a = synth.host_attn(12, 17, O.quantize_rows, **synth.ATTN_FLASH)
    wr = GGUFWriter()
    wr.add("diffuse.block_count", U32, 1)
    wr.add("diffuse.embedding_length", U32, a.n_embd)
    for k, t, v in attn_keys(a):
        wr.add(k, t, v)
    add_attn_layer(wr, 0, a)
    path = tmp_path / "attn.gguf"
    wr.write(path)
    with GGUF(path) as g:
        aw = g.attn_weights(0)
        layer = ctx.attn_upload(aw)
        h = (synth.normal(18, synth.S_X, 32 * a.n_embd).reshape(32, a.n_embd) * 2).astype(np.float32)
        h_out, moe_in = ctx.attn_forward(layer, h)
        r_out, r_in = O.attn_forward(aw, h)
        e1, e2 = max_rel_err(h_out, r_out), max_rel_err(moe_in, r_in)
        _say(f"  h_out err {e1:.3e}  moe_in err {e2:.3e}")
        assert e1 <= 1e-4 and e2 <= 1e-4
        layer.free()


def test_head_q6k_from_gguf(ctx, O, tmp_path):
    """The step tail of a file quantised as the reference's Q4_K schemes do
    it: output.weight Q6_K (hidden 4096, 32768 tokens of vocabulary) and an
    F32 output_norm, read by GGUF.head_weights from the mapping, uploaded and
    run on 32 positions against the oracle on the same mapped bytes (bars of
    tests/test_gpu_head.py)."""
    import torch
    from dmoe import synth
    from dmoe.gguf import GGUF
    from test_gpu_head import TOL, _check
    H, V, N = 4096, 32768, 32
    _say(f"case: Q6_K output.weight through a GGUF file, V={V}")
    w = synth.head_to_host(synth.device_head(H, V, 14, 31, ctx))
    torch.cuda.empty_cache()
    wr = GGUFWriter()
    wr.add("diffuse.embedding_length", 4, H)
    wr.add_tensor("output_norm.weight", 0, [H], np.ascontiguousarray(w.norm, np.float32))
    wr.add_tensor("output.weight", 14, [H, V], w.output)
    path = tmp_path / "head.gguf"
    wr.write(path)
    with GGUF(path) as g:
        hw = g.head_weights()
        assert (hw.n_embd, hw.n_vocab, hw.wtype) == (H, V, 14)
        head = ctx.head_upload(hw)
        assert head.kernel_path() == "q6k_mfma"
        h = (synth.normal(32, synth.S_X, N * H).reshape(N, H) * 2).astype(np.float32)
        tok, prob, lg = ctx.head_forward(head, h, 1e-6, logits=True)
        tr, pr, lr = O.head_forward(hw, h, 1e-6)
        err = _check(tok, prob, lg, tr, pr, lr, TOL[14])
        _say(f"  logits max rel err {err:.3e}")
        head.free()
