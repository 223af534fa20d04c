"""GPU: the allocation-free forward (dmoe_layer_forward_device_noalloc)
against the allocating device forward (dmoe_layer_forward_device), through
the C ABI.  Both run the same kernels on the same inputs, so the outputs are
compared bit for bit (stricter than the layer tolerance); two calls in a row,
the second with fewer tokens, so the second runs on what the first left in
the GPU's scratch array.  A forward whose workspace exceeds the scratch is
rejected before anything is queued."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _run_pair(ctx, layer, x_host, n_tokens, stream):
    import torch
    dev = torch.device("cuda:0")
    x = torch.from_numpy(np.ascontiguousarray(x_host[:n_tokens])).to(dev)
    y_ref = torch.full_like(x, float("nan"))
    y_new = torch.full_like(x, float("nan"))
    ctx.forward_device(layer, x, n_tokens, y_ref, stream)
    ctx.forward_device_noalloc(layer, x, n_tokens, y_new, stream)
    torch.cuda.synchronize(dev)
    return y_ref.cpu().numpy(), y_new.cpu().numpy()


@pytest.mark.parametrize("case", ["flash_q4k", "small_f16", "small_q8_0"])
def test_noalloc_matches_forward_device(ctx, O, case):
    import torch
    from dmoe import synth
    if case == "flash_q4k":
        cfg = synth.CONFIGS["flash_q4k"]
        w = synth.device_layer(cfg, 3, ctx)
        layer = ctx.wrap_device(w)
        sizes = (256, 32)
    else:
        wt = 1 if case == "small_f16" else 8
        cfg = synth.LayerConfig(case, 512, 32, 256, 8, 4, 32, 256, wt, wt, 96, -0.05, 0.05)
        w = synth.host_layer(cfg, 3, O.quantize_rows)
        layer = ctx.upload(w)
        sizes = (96, 40)            # the second without block routing
    x_host = synth.make_x(cfg, 3, max(sizes))
    stream = torch.cuda.current_stream().cuda_stream
    for n in sizes:
        _say(f"case: allocation-free forward, {case}, N={n}")
        y_ref, y_new = _run_pair(ctx, layer, x_host, n, stream)
        assert np.isfinite(y_ref).all()
        assert np.array_equal(y_new.view(np.uint32), y_ref.view(np.uint32)), (case, n)
    layer.free()
    del w
    torch.cuda.empty_cache()


def test_noalloc_dense(ctx, O):
    """The dense MLP through the allocation-free forward: bit for bit with
    the allocating one, 32 then 24 tokens."""
    import torch
    from dmoe import synth
    w = synth.host_dense(512, 768, 12, 5, O.quantize_rows)
    layer = ctx.dense_upload(w)
    x_host = synth.normal(5, synth.S_X, 32 * 512).reshape(32, 512)
    stream = torch.cuda.current_stream().cuda_stream
    for n in (32, 24):
        _say(f"case: allocation-free forward, dense MLP, N={n}")
        y_ref, y_new = _run_pair(ctx, layer, x_host, n, stream)
        assert np.isfinite(y_ref).all()
        assert np.array_equal(y_new.view(np.uint32), y_ref.view(np.uint32))
    layer.free()


def test_noalloc_rejects_oversize(ctx, O):
    """The flash Q4_K layer at 4096 tokens needs far more than the scratch:
    rejected with DMOE_ERR_INVALID_ARG and a message naming the limit; the
    output buffer is left untouched."""
    import torch
    import dmoe
    from dmoe import synth
    _say("case: allocation-free forward above the scratch size")
    cfg = synth.CONFIGS["flash_q4k"]
    w = synth.device_layer(cfg, 4, ctx)
    layer = ctx.wrap_device(w)
    n = 4096
    dev = torch.device("cuda:0")
    x = torch.zeros((n, cfg.n_embd), dtype=torch.float32, device=dev)
    y = torch.full_like(x, 7.0)
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.forward_device_noalloc(layer, x, n, y, torch.cuda.current_stream().cuda_stream)
    assert ei.value.code == dmoe._abi.ERR_INVALID_ARG
    assert "scratch" in str(ei.value)
    torch.cuda.synchronize(dev)
    assert bool((y == 7.0).all())
    layer.free()
    del w
    torch.cuda.empty_cache()


def test_noalloc_forward_replayed_from_a_hip_graph(ctx):
    """The allocation-free forward captured into a HIP graph (torch's graph
    capture on a side stream of default priority) and replayed on three new
    inputs copied into the captured input buffer: every replay equals the
    allocating forward's eager result on the same input bit for bit, with an
    eager forward and a synchronisation between the replays.  (The forward
    clears its flags and counters with fill kernels, not memset nodes.)"""
    import torch
    from dmoe import synth
    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS["flash_q4k"]
    w = synth.device_layer(cfg, 7, ctx)
    layer = ctx.wrap_device(w)
    xs = [torch.from_numpy(synth.make_x(cfg, 70 + i, 32)).to(dev) for i in range(3)]
    main = torch.cuda.current_stream(dev)
    refs = []
    for x in xs:
        y = torch.empty_like(x)
        ctx.forward_device(layer, x, 32, y, main.cuda_stream)
        refs.append(y)
    torch.cuda.synchronize(dev)
    x_in = torch.zeros_like(xs[0])
    y_out = torch.full_like(xs[0], float("nan"))
    side = torch.cuda.Stream(dev)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        # one eager call on the capture stream first
        ctx.forward_device_noalloc(layer, x_in, 32, y_out, side.cuda_stream)
    side.synchronize()
    g = torch.cuda.CUDAGraph()
    _say("case: allocation-free forward captured in a HIP graph, flash Q4_K, N=32")
    with torch.cuda.graph(g, stream=side):
        ctx.forward_device_noalloc(layer, x_in, 32, y_out, side.cuda_stream)
    torch.cuda.synchronize(dev)
    for i, x in enumerate(xs):
        x_in.copy_(x)
        y_out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(y_out.view(torch.int32), refs[i].view(torch.int32)), f"replay {i}"
        # eager work between the replays
        y = torch.empty_like(x)
        ctx.forward_device(layer, xs[(i + 1) % 3], 32, y, main.cuda_stream)
        torch.cuda.synchronize(dev)
        assert torch.equal(y.view(torch.int32), refs[(i + 1) % 3].view(torch.int32))
    del g
    layer.free()
    del w
    torch.cuda.empty_cache()
