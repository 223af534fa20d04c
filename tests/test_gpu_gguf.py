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
