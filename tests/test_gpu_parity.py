"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bar (tolerances written here, per the layer contract):
  * routing — logits, probs, block max, threshold, allowed set, top-k indices,
    gate weights, per-expert counts/offsets and the dispatch permutation — is
    bit-exact on identical fp32 inputs;
  * layer output: max|y - y_oracle| / max|y_oracle| <= 3e-3 for one layer
    with quantised expert weights (Q8_0, Q4_K; the layer contract allows
    2e-2, the worst measured is 8.7e-4, so the bar sits at about 3x that to
    catch a lost term), <= 1e-3 for F16, <= 1e-4 for F32; the 32-layer chain's
    accumulated error is held to the contract's 2e-2.
"""
import numpy as np
import pytest

from conftest import max_rel_err

pytestmark = pytest.mark.gpu

TOL = {0: 1e-4, 1: 1e-3, 8: 3e-3, 12: 3e-3, 14: 3e-3}
TOL_CHAIN = 2e-2
ROUTE_KEYS = ("logits", "probs", "bmax", "thr", "allowed", "idx", "weights", "counts",
              "offsets", "perm", "use_block_routing")


def _say(msg):
    print(msg, flush=True)


def _check_routing(dg, dr, keys=ROUTE_KEYS):
    for k in keys:
        a, b = dg[k], dr[k]
        if isinstance(a, np.ndarray):
            assert a.shape == b.shape, k
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{k} differs"
        else:
            assert a == b, k


def _ctx_with(monkeypatch, env):
    """A context created with the kernel-selection variables in env set (a
    context reads them once, at creation); they are cleared again after."""
    import dmoe
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    c = dmoe.Context(0)
    for k in env:
        monkeypatch.delenv(k)
    return c


def _small(dmoe, synth, wtype, n_tokens=64, seed=3):
    return synth.LayerConfig(f"small_{wtype}", 512, 32, 256, 8, 4, 32, 256, wtype, wtype,
                             n_tokens, -0.05, 0.05)


def test_tiny_layer(ctx, O):
    import dmoe
    from dmoe import synth
    _say("case: tiny F32 layer, N=32")
    cfg = synth.CONFIGS["tiny"]
    w = synth.host_layer(cfg, 11, O.quantize_rows)
    x = synth.make_x(cfg, 11)
    layer = ctx.upload(w)
    y, dg = ctx.forward(layer, x, debug=True)
    yr, dr = O.layer_forward(w, x, debug=True)
    _check_routing(dg, dr)
    assert max_rel_err(y, yr) <= TOL[0]


@pytest.mark.parametrize("wtype", [12, 8, 1], ids=["Q4_K", "Q8_0", "F16"])
@pytest.mark.parametrize("n_tokens", [32, 96, 40, 128], ids=["N32", "N96", "N40_noblock", "N128"])
def test_small_layer(ctx, O, wtype, n_tokens):
    import dmoe
    from dmoe import synth
    _say(f"case: small layer type={wtype} N={n_tokens}")
    cfg = _small(dmoe, synth, wtype, n_tokens)
    w = synth.host_layer(cfg, 5 + wtype, O.quantize_rows)
    x = synth.make_x(cfg, 5 + wtype, n_tokens)
    layer = ctx.upload(w)
    y, dg = ctx.forward(layer, x, debug=True)
    yr, dr = O.layer_forward(w, x, debug=True)
    _check_routing(dg, dr)
    assert dg["use_block_routing"] == (n_tokens % 32 == 0)
    err = max_rel_err(y, yr)
    _say(f"  max rel err {err:.3e}")
    assert err <= TOL[wtype]


@pytest.mark.parametrize("wtype", [12, 8, 1], ids=["Q4_K", "Q8_0", "F16"])
def test_small_layer_many_items(ctx, O, wtype):
    """Layers of moe_ff 256 over 2048 tokens.  Q4_K: down items of two steps
    (the fewest the LDS rings can run on across) and several items per
    workgroup, so each item's first steps are issued by the previous item's.
    Q8_0: more items than the persistent grid.  F16: the grouped GEMM with
    8 and 16 k steps per item, so its ring's first and last steps overlap."""
    import dmoe
    from dmoe import synth
    n_tokens = 2048
    _say(f"case: small layer type={wtype} N={n_tokens}, many items per workgroup")
    cfg = _small(dmoe, synth, wtype, n_tokens)
    w = synth.host_layer(cfg, 31, O.quantize_rows)
    x = synth.make_x(cfg, 31, n_tokens)
    layer = ctx.upload(w)
    y, dg = ctx.forward(layer, x, debug=True)
    yr, dr = O.layer_forward(w, x, debug=True)
    _check_routing(dg, dr)
    err = max_rel_err(y, yr)
    _say(f"  max rel err {err:.3e}")
    assert err <= TOL[wtype]


@pytest.mark.parametrize("name", ["flash_q4k", "flash_q8_0", "flash_q4k_n256", "flash_q4k_n512",
                                  "flash_q4k_n768", "flash_q4k_n1024", "flash_q4k_n2048", "flash_q8_0_n256",
                                  "flash_q8_0_n2048", "flash_f16", "prefill_f16"])
def test_flash_layer(ctx, O, name):
    """Flash-shaped layers: one 32-token block (Q4_K, Q8_0), eight blocks
    (Q4_K, 256 tokens, each block its own allowed set), the sampler's 512-
    and 768-token windows (one column block with more pairs than the
    register-ring kernel's LDS routing tables hold), its 1024- and 2048-token
    windows, Q8_0 over 256 and 2048 tokens, F16 over one block and the
    2048-token F16 prefill.  From 256 tokens the Q4_K and Q8_0 layers run on
    the tile kernels (many tokens per expert); the one-block F16 layer runs
    on them too (few tokens per expert), the prefill on the grouped GEMM."""
    import torch
    import dmoe
    from dmoe import synth
    _say(f"case: {name}, {synth.CONFIGS[name].n_tokens} tokens")
    cfg = synth.CONFIGS[name]
    wd = synth.device_layer(cfg, 21, ctx)
    layer = ctx.wrap_device(wd)
    x = synth.make_x(cfg, 21)
    y, dg = ctx.forward(layer, x, debug=True)
    wh = synth.to_host(wd)
    yr, dr = O.layer_forward(wh, x, debug=True)
    _check_routing(dg, dr)
    touched = int((dr["counts"] > 0).sum())
    allowed = int(dr["allowed"].sum())
    err = max_rel_err(y, yr)
    _say(f"  touched experts {touched}, allowed {allowed}, max rel err {err:.3e}")
    assert allowed >= cfg.capacity
    assert err <= TOL[cfg.wtype]
    del layer, wd
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["flash_q4k_n1024", "small_q4k_n2048"])
def test_q4k_column_blocks_bit_exact(ctx, name, monkeypatch):
    """Q4_K work items of 1, 2 and 4 column blocks (16, 32, 64 pairs of an
    expert per weight-tile read) compute every product in the same order:
    the layer outputs are identical bit for bit."""
    import dmoe
    from dmoe import synth
    if name.startswith("small"):
        cfg = _small(dmoe, synth, 12, 2048)
    else:
        cfg = synth.CONFIGS[name]
    _say(f"case: Q4_K column blocks 1 / 2 / 4, {name}")
    wd = synth.device_layer(cfg, 23, ctx)
    layer = ctx.wrap_device(wd)
    x = synth.make_x(cfg, 23, cfg.n_tokens)
    ys = []
    for nc in ("1", "2", "4"):
        c = _ctx_with(monkeypatch, {"DMOE_Q4K_COLUMN_BLOCKS": nc})
        ys.append(c.forward(layer, x))
        c.close()
    ys.append(ctx.forward(layer, x))                      # the automatic choice
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))


@pytest.mark.parametrize("name", ["flash_q4k", "small_q4k_n40", "small_q4k_n96", "small_q4k_n128"])
def test_down_span_bit_exact(ctx, name, monkeypatch):
    """Few-token Q4_K down products by spans of (unit, 16-row tile) work,
    then the combine launch, against the fused kernel that folds in LDS: the
    same products in the same order, so the layer outputs are identical bit
    for bit.  Each span call follows one on other inputs of the same size, so
    products left in HBM by that call would show if the combine read them."""
    import dmoe
    from dmoe import synth
    if name.startswith("small"):
        cfg = _small(dmoe, synth, 12, int(name.rsplit("_n", 1)[1]))
    else:
        cfg = synth.CONFIGS[name]
    _say(f"case: down spans vs down rows, {name}")
    wd = synth.device_layer(cfg, 27, ctx)
    layer = ctx.wrap_device(wd)
    x = synth.make_x(cfg, 27, cfg.n_tokens)
    xo = synth.make_x(cfg, 28, cfg.n_tokens)
    n2 = cfg.n_tokens // 2 + 3
    # (the few-token kernels at every size: 96 and 128 tokens of the small
    # layer would otherwise take the tile kernels)
    c = _ctx_with(monkeypatch, {"DMOE_DOWN_FUSED": "1", "DMOE_EXPERT_TILE": "0"})
    ref = [c.forward(layer, a) for a in (x, xo, x[:n2], xo[:n2])]
    c.close()
    c = _ctx_with(monkeypatch, {"DMOE_EXPERT_TILE": "0"})
    got = [c.forward(layer, a) for a in (xo, x, xo[:n2], x[:n2])]
    c.close()
    for r, g in zip(ref, (got[1], got[0], got[3], got[2])):
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32))


@pytest.mark.parametrize("name", ["flash_q4k", "flash_q4k_n256", "flash_q4k_n512", "flash_q4k_n768",
                                  "small_q4k_n40", "small_q4k_n128"])
def test_gateup_register_ring_bit_exact(ctx, name, monkeypatch):
    """Q4_K gate/up items of one column block with the weights streamed to
    registers and the item's activations in LDS, against the kernel with LDS
    rings for both: the same products in the same order, so the layer
    outputs are identical bit for bit.  At 512 and 768 tokens the
    register-ring kernel looks its routing up in HBM (more pairs than its
    LDS tables hold)."""
    import dmoe
    from dmoe import synth
    if name.startswith("small"):
        cfg = _small(dmoe, synth, 12, int(name.rsplit("_n", 1)[1]))
    else:
        cfg = synth.CONFIGS[name]
    _say(f"case: gate/up register ring vs LDS rings, {name}")
    wd = synth.device_layer(cfg, 29, ctx)
    layer = ctx.wrap_device(wd)
    x = synth.make_x(cfg, 29, cfg.n_tokens)
    xo = synth.make_x(cfg, 30, cfg.n_tokens)
    # (the one-column-block kernels at every size: from 256 tokens the flash
    # layer would otherwise take the tile kernels)
    c = _ctx_with(monkeypatch, {"DMOE_GATEUP_LDS": "1", "DMOE_EXPERT_TILE": "0"})
    ref = [c.forward(layer, a) for a in (x, xo)]
    c.close()
    c = _ctx_with(monkeypatch, {"DMOE_EXPERT_TILE": "0"})
    got = [c.forward(layer, a) for a in (xo, x)]
    c.close()
    assert np.array_equal(got[1].view(np.uint32), ref[0].view(np.uint32))
    assert np.array_equal(got[0].view(np.uint32), ref[1].view(np.uint32))


@pytest.mark.parametrize("name", ["flash_q4k_n256", "flash_q4k_n2048", "small_q4k_n40", "small_q4k_n96",
                                  "small_q4k_n2048", "small_q4k_n1000", "flash_q8_0_n256", "small_q80_n96",
                                  "small_q80_n1000"])
def test_tile_path_bit_exact(ctx, name, monkeypatch):
    """Products of many tokens per expert on the tile kernels (units of up to
    32 pairs of an expert with their activations held in LDS, h through HBM
    and one conversion) against the item kernels (Q4_K: four column blocks;
    Q8_0: k_expert_q80): the same products in the same order, so the layer
    outputs are identical bit for bit.  Each tile call follows one on other
    inputs of the same size (h and pair lists left by that call must not leak
    into this one); 40 and 1000 tokens run without block routing, and the
    small layer's shared expert spans partial units."""
    import dmoe
    from dmoe import synth
    if name.startswith("small"):
        wt = 8 if "q80" in name else 12
        cfg = _small(dmoe, synth, wt, int(name.rsplit("_n", 1)[1]))
    else:
        cfg = synth.CONFIGS[name]
    _say(f"case: tile kernels vs item kernels, {name}")
    wd = synth.device_layer(cfg, 33, ctx)
    layer = ctx.wrap_device(wd)
    x = synth.make_x(cfg, 33, cfg.n_tokens)
    xo = synth.make_x(cfg, 34, cfg.n_tokens)
    ref_env = {"DMOE_EXPERT_TILE": "0"}
    if cfg.wtype == 12:
        ref_env["DMOE_Q4K_COLUMN_BLOCKS"] = "4"
    c = _ctx_with(monkeypatch, ref_env)
    ref = [c.forward(layer, a) for a in (x, xo)]
    c.close()
    c = _ctx_with(monkeypatch, {"DMOE_EXPERT_TILE": "1"})
    got = [c.forward(layer, a) for a in (xo, x)]
    c.close()
    assert np.isfinite(ref[0]).all()
    assert np.array_equal(got[1].view(np.uint32), ref[0].view(np.uint32))
    assert np.array_equal(got[0].view(np.uint32), ref[1].view(np.uint32))


@pytest.mark.parametrize("name", ["flash_q4k_n2048", "flash_q4k_n1024", "flash_q4k_n256", "mid_q4k_n1000",
                                  "mid_q4k_n200", "mid_noshared_q4k_n1000"])
def test_q4k_gemm_bit_exact(ctx, name, monkeypatch):
    """Q4_K products on the grouped GEMM (units of up to 128 pairs of an
    expert, eight column blocks per weight-tile step, weights and activations
    streamed through LDS together) against the tile kernels: the same integer
    sums per super-block and the same epilogue in the same order, so the layer
    outputs are identical bit for bit.  Each GEMM call follows one on other
    inputs of the same size; 256 and 200 tokens force the GEMM onto units of
    one or two blocks, and the mid-sized layers (1000 and 200 tokens, no block
    routing) end their shared expert on a partial unit; one has no shared
    expert at all."""
    import dmoe
    from dmoe import synth
    if name.startswith("mid"):
        n = int(name.rsplit("_n", 1)[1])
        sf = 0 if "noshared" in name else 512
        cfg = synth.LayerConfig(name, 512, 32, 512, 8, 4, 32, sf, 12, 12, n, -0.05, 0.05)
    else:
        cfg = synth.CONFIGS[name]
    _say(f"case: grouped Q4_K GEMM vs tile kernels, {name}")
    wd = synth.device_layer(cfg, 35, ctx)
    layer = ctx.wrap_device(wd)
    x = synth.make_x(cfg, 35, cfg.n_tokens)
    xo = synth.make_x(cfg, 36, cfg.n_tokens)
    c = _ctx_with(monkeypatch, {"DMOE_EXPERT_TILE": "1", "DMOE_EXPERT_GEMM": "0"})
    ref = [c.forward(layer, a) for a in (x, xo)]
    c.close()
    c = _ctx_with(monkeypatch, {"DMOE_EXPERT_GEMM": "1"})
    got = [c.forward(layer, a) for a in (xo, x)]
    c.close()
    assert np.isfinite(ref[0]).all()
    assert np.array_equal(got[1].view(np.uint32), ref[0].view(np.uint32))
    assert np.array_equal(got[0].view(np.uint32), ref[1].view(np.uint32))


@pytest.mark.parametrize("n_tokens,tile", [(32, 0), (40, 0), (128, 1), (2048, 1), (1000, 1)],
                         ids=["N32_gemm", "N40_gemm", "N128_tile", "N2048_tile", "N1000_tile"])
def test_f16_paths(ctx, O, n_tokens, tile, monkeypatch):
    """F16 experts through the path the automatic choice does not take at
    that size: the grouped GEMM at few tokens per expert, the tile kernels
    (16-pair units, f16 x and h held in LDS per item) at many, each against
    the oracle within the F16 bar (1000 tokens: no block routing)."""
    import dmoe
    from dmoe import synth
    _say(f"case: small F16 layer N={n_tokens}, DMOE_EXPERT_TILE={tile}")
    cfg = _small(dmoe, synth, 1, n_tokens)
    w = synth.host_layer(cfg, 41, O.quantize_rows)
    x = synth.make_x(cfg, 41, n_tokens)
    c = _ctx_with(monkeypatch, {"DMOE_EXPERT_TILE": str(tile)})
    layer = c.upload(w)
    y, dg = c.forward(layer, x, debug=True)
    yr, dr = O.layer_forward(w, x, debug=True)
    _check_routing(dg, dr)
    err = max_rel_err(y, yr)
    _say(f"  max rel err {err:.3e}")
    assert err <= TOL[1]
    layer.free()
    c.close()


def test_route_logits_flash_shape(ctx, O):
    import dmoe
    _say("case: routing from injected logits, flash shape, 8 blocks")
    rng = np.random.default_rng(0)
    hp = dmoe.hparams_of(4096, 256, 8, 48, 32)
    N = 256
    logits = (rng.standard_normal((N, 256)) * 1.28).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, 256).astype(np.float32)
    dg = ctx.route_logits(hp, logits, bias)
    dr = O.route(hp, logits, bias)
    _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])


@pytest.mark.parametrize("N", [2304, 4128, 2312], ids=["72groups", "129groups", "73groups_noblock"])
def test_route_logits_many_groups(ctx, O, N):
    """More routing groups than one LDS chunk of the dispatch holds (64
    groups of 256 experts): the histograms are scanned chunk by chunk, the
    last chunk partial (one group; a partial group without block routing)."""
    import dmoe
    _say(f"case: routing from injected logits, 256 experts, N={N}")
    rng = np.random.default_rng(N)
    hp = dmoe.hparams_of(4096, 256, 8, 48, 32)
    logits = (rng.standard_normal((N, 256)) * 1.28).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, 256).astype(np.float32)
    dg = ctx.route_logits(hp, logits, bias)
    dr = O.route(hp, logits, bias)
    assert dg["use_block_routing"] == (N % 32 == 0)
    _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])


def test_route_logits_ties_and_slack(ctx, O):
    import dmoe
    _say("case: routing ties / slack")
    hp = dmoe.hparams_of(256, 64, 4, 8, 32)
    N = 64
    # many exact ties: logits from a tiny set of values
    rng = np.random.default_rng(1)
    logits = rng.choice(np.array([-1.0, 0.0, 0.5, 0.5, 2.0], np.float32), size=(N, 64))
    for bias in (None, np.zeros(64, np.float32)):
        dg = ctx.route_logits(hp, logits, bias)
        dr = O.route(hp, logits, bias)
        _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])
        assert dg["allowed"].sum(1).min() >= 8


def _slack_bias(E, cap):
    """Selection-score bias that puts, with all logits 0 (probs 0.5), cap
    experts at block max 0.6, one expert just inside the 1e-6 slack below
    the threshold (admitted), one exactly at fl(thr - 1e-6) (rejected: the
    test is strict, src/diffuse-moe-graph.cpp:241-242) and one just outside
    the slack; the rest far below.  Same construction as the oracle's
    slack test."""
    bias = np.full(E, -0.2, np.float32)
    bias[:cap] = 0.1
    tp = np.float32(np.float32(0.6) + np.float32(-1e-6))
    bias[cap] = np.float32(np.float32(0.6) - np.float32(4e-7)) - np.float32(0.5)
    bias[cap + 1] = tp - np.float32(0.5)
    bias[cap + 2] = np.float32(0.6 - 3e-6) - np.float32(0.5)
    return bias


@pytest.mark.parametrize("E,K,cap,N", [(16, 2, 4, 32), (256, 8, 48, 64), (256, 8, 48, 32)],
                         ids=["E16_one_block", "flash_two_blocks", "flash_one_block"])
def test_route_logits_slack_boundary(ctx, O, E, K, cap, N):
    """The capacity test admits a block max inside fl(thr - 1e-6) and rejects
    one exactly at it: the allowed set holds cap + 1 experts, bit for bit
    with the oracle (one-group and many-group routing kernels)."""
    import dmoe
    _say(f"case: routing slack boundary E={E} K={K} cap={cap} N={N}")
    hp = dmoe.hparams_of(4096 if E == 256 else 256, E, K, cap, 32)
    logits = np.zeros((N, E), np.float32)
    bias = _slack_bias(E, cap)
    dg = ctx.route_logits(hp, logits, bias)
    dr = O.route(hp, logits, bias)
    assert np.all(dr["thr"] == np.float32(0.6))
    al = dg["allowed"].astype(bool)
    assert al[:, :cap].all() and al[:, cap].all()
    assert not al[:, cap + 1].any() and not al[:, cap + 2].any()
    assert (al.sum(1) == cap + 1).all()
    _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])


@pytest.mark.parametrize("cap", [256, 300], ids=["cap_eq_E", "cap_gt_E"])
def test_route_logits_capacity_at_least_experts(ctx, O, cap):
    """capacity >= n_experts switches block routing off (plain top-k over all
    experts, src/diffuse-moe-graph.cpp:215-216)."""
    import dmoe
    _say(f"case: routing with capacity {cap} >= 256 experts")
    rng = np.random.default_rng(cap)
    hp = dmoe.hparams_of(4096, 256, 8, cap, 32)
    N = 64
    logits = (rng.standard_normal((N, 256)) * 1.28).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, 256).astype(np.float32)
    dg = ctx.route_logits(hp, logits, bias)
    dr = O.route(hp, logits, bias)
    assert not dg["use_block_routing"] and not dr["use_block_routing"]
    _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])


@pytest.mark.parametrize("E,blk,K,cap,N", [(256, 64, 8, 48, 128), (512, 32, 8, 48, 64),
                                           (64, 64, 20, 40, 128)],
                         ids=["blk64_E256", "E512", "blk64_K20"])
def test_route_logits_general_kernel(ctx, O, E, blk, K, cap, N):
    """Routing groups too large for the LDS kernels (block_size x E above 8192
    scores, or top_k x block above 1024 pairs) take k_route_general and
    k_dispatch_general: bit-exact with the oracle, including the slack
    boundary on the first group."""
    import dmoe
    _say(f"case: general routing kernel E={E} blk={blk} K={K} cap={cap} N={N}")
    rng = np.random.default_rng(E + blk + K)
    hp = dmoe.hparams_of(4096, E, K, cap, blk)
    logits = (rng.standard_normal((N, E)) * 1.28).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    dg = ctx.route_logits(hp, logits, bias)
    dr = O.route(hp, logits, bias)
    assert dg["use_block_routing"]
    _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])
    logits[:blk] = 0.0
    bias = _slack_bias(E, cap)
    dg = ctx.route_logits(hp, logits, bias)
    dr = O.route(hp, logits, bias)
    assert dg["allowed"][0].sum() == cap + 1
    _check_routing(dg, dr, [k for k in ROUTE_KEYS if k != "logits"])


# Layers whose types or widths the MFMA kernels do not take run the GEMV
# kernels (k_gemv.hip); each case reaches one of its quantised instantiations.
_GEMV_CASES = {
    # n_embd 768: not a whole number of 512-row down items
    "q4k_h768": (768, 256, 256, 12, 12),
    # shared expert twice as wide as the routed ones
    "q4k_wide_shared": (512, 256, 512, 12, 12),
    # Q4_K routed experts with a Q8_0 shared expert
    "q4k_q80_shared": (512, 256, 256, 12, 8),
    # moe_ff 96: not a whole number of 256-value steps
    "q80_ff96": (512, 96, 96, 8, 8),
    # F16 routed experts with an F32 shared expert
    "f16_f32_shared": (512, 256, 256, 1, 0),
    # Q6_K routed and shared experts (the reference's q6_k scheme)
    "q6k_experts": (512, 256, 256, 14, 14),
    # Q4_K routed experts with a Q6_K shared expert
    "q4k_q6k_shared": (512, 256, 256, 12, 14),
}


@pytest.mark.parametrize("case", list(_GEMV_CASES))
def test_gemv_path_layer(ctx, O, case):
    from dmoe import synth
    H, FF, SF, wt, st = _GEMV_CASES[case]
    N = 64
    _say(f"case: GEMV path {case}: H={H} moe_ff={FF} shared_ff={SF} types {wt}/{st}, N={N}")
    cfg = synth.LayerConfig(case, H, 32, FF, 8, 4, 32, SF, wt, st, N, -0.05, 0.05)
    w = synth.host_layer(cfg, 41, O.quantize_rows)
    x = synth.make_x(cfg, 41, N)
    layer = ctx.upload(w)
    assert layer.kernel_path() == "gemv"
    y, dg = ctx.forward(layer, x, debug=True)
    yr, dr = O.layer_forward(w, x, debug=True)
    _check_routing(dg, dr)
    err = max_rel_err(y, yr)
    _say(f"  max rel err {err:.3e}")
    assert err <= max(TOL[wt], TOL[st])


def test_mfma_paths_selected(ctx, O):
    """The shapes of the flash layer take the MFMA kernels for each type."""
    from dmoe import synth
    _say("case: kernel path of the small layers")
    for wt, name in ((12, "q4k_mfma"), (8, "q80_mfma"), (1, "f16_gemm"), (0, "gemv")):
        cfg = _small(None, synth, wt, 32)
        layer = ctx.upload(synth.host_layer(cfg, 2, O.quantize_rows))
        assert layer.kernel_path() == name, (wt, layer.kernel_path())
        layer.free()


def test_sigmoid_sweep(ctx, O):
    """GPU sigmoid (binary64 exp) equals the oracle's on a sweep of fp32
    logits: every 509th bit pattern of [-110, 100] plus 2^20 random values."""
    import dmoe
    _say("case: sigmoid sweep")
    lo = np.float32(-110.0).view(np.uint32)
    hi = np.float32(100.0).view(np.uint32)
    neg = np.arange(np.uint32(0x80000000), lo, 509, dtype=np.uint64).astype(np.uint32)
    pos = np.arange(0, hi, 509, dtype=np.uint64).astype(np.uint32)
    rng = np.random.default_rng(2)
    vals = np.concatenate([neg.view(np.float32), pos.view(np.float32),
                           rng.uniform(-110, 100, 1 << 20).astype(np.float32)])
    E = 256
    vals = vals[: (len(vals) // E) * E].reshape(-1, E)
    hp = dmoe.hparams_of(256, E, 1, 0, 32)   # capacity 0: no block routing
    probs = np.empty_like(vals)
    for c0 in range(0, vals.shape[0], 16384):
        dg = ctx.route_logits(hp, vals[c0:c0 + 16384], None)
        probs[c0:c0 + 16384] = dg["probs"]
    ref = np.empty_like(vals)
    flat = vals.reshape(-1)
    e = O.expf(-flat)
    ref = (np.float32(1.0) / (np.float32(1.0) + e)).reshape(vals.shape)
    assert np.array_equal(probs.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("wtype", [12, 14, 8, 1])
def test_device_quantizer_matches_oracle(ctx, O, wtype):
    import torch
    _say(f"case: device quantizer type {wtype}")
    rng = np.random.default_rng(4)
    f = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    f[3, :256] = 0.0                         # all-zero super-block
    f[5, :] = np.abs(f[5, :])                # positive-only rows (min clamps to 0)
    ref = O.quantize_rows(wtype, f)
    src = torch.from_numpy(f).cuda()
    dst = torch.zeros(ref.shape, dtype=torch.uint8, device="cuda")
    ctx.quantize_device(wtype, src, dst, 64, 1024)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), ref)


def test_forward_device_matches_host(ctx, O):
    import torch
    from dmoe import synth
    _say("case: device-pointer forward == host forward")
    cfg = _small(None, synth, 12, 64)
    w = synth.host_layer(cfg, 9, O.quantize_rows)
    x = synth.make_x(cfg, 9, 64)
    layer = ctx.upload(w)
    y = ctx.forward(layer, x)
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty_like(xd)
    s = torch.cuda.current_stream()
    ctx.forward_device(layer, xd, 64, yd, s.cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(yd.cpu().numpy(), y)
    # deterministic: repeat is bit-identical
    assert np.array_equal(ctx.forward(layer, x), y)


def test_error_paths(ctx, O):
    import dmoe
    from dmoe import synth
    _say("case: error paths")
    cfg = synth.CONFIGS["tiny"]
    w = synth.host_layer(cfg, 1, O.quantize_rows)
    bad = synth.replace(w, wtype=2)                      # Q4_0: unsupported
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.upload(bad)
    assert ei.value.code == dmoe._abi.ERR_UNSUPPORTED_TYPE
    hp = w.hparams()
    hp.moe_ff = 64                                       # hparams disagree with ne
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.upload(w, hp=hp)
    assert ei.value.code == dmoe._abi.ERR_SHAPE
    d = w.desc()
    d.exp_down.nb[1] = 8                                 # stride below the row size
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.upload(w, desc=d)
    assert ei.value.code == dmoe._abi.ERR_SHAPE
    layer = ctx.upload(w)
    x = synth.make_x(cfg, 1)
    x[3, 7] = np.nan
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.forward(layer, x)
    assert ei.value.code == dmoe._abi.ERR_NONFINITE


@pytest.mark.parametrize("rows,H,with_y,with_gain", [(32, 4096, True, False), (96, 512, True, True),
                                                     (7, 4096, False, True)])
def test_residual_rmsnorm(ctx, rows, H, with_y, with_gain):
    """h += y, x = rms_norm(h) [* gain] (src/diffuse-moe-graph.cpp:292,
    :175-178) against ggml_rms_norm's definition evaluated in numpy: the f32
    squares summed in float64, the mean rounded to f32, scale = 1 / sqrt(mean +
    eps) in f32.  h is bit-exact (one f32 add per element); x within 2 ulp
    (the double sum runs in another order than ggml's sequential one, which
    can move the f32 mean by one ulp)."""
    import torch
    import dmoe
    _say(f"case: residual rmsnorm rows={rows} H={H} y={with_y} gain={with_gain}")
    rng = np.random.default_rng(rows + H)
    h0 = (rng.standard_normal((rows, H)) * 3).astype(np.float32)
    y = rng.standard_normal((rows, H)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, H).astype(np.float32)
    dev = torch.device("cuda:0")
    hd = torch.from_numpy(h0).to(dev)
    yd = torch.from_numpy(y).to(dev) if with_y else None
    gd = torch.from_numpy(g).to(dev) if with_gain else None
    xd = torch.empty_like(hd)
    ctx.residual_rmsnorm(hd, yd, xd, rows, H, 1e-6, gain_dev=gd)
    torch.cuda.synchronize()
    h_ref = (h0 + y).astype(np.float32) if with_y else h0
    x_ref = _rmsnorm_np(h_ref)
    if with_gain:
        x_ref = (x_ref * g).astype(np.float32)
    assert np.array_equal(hd.cpu().numpy().view(np.uint32), h_ref.view(np.uint32))
    x = xd.cpu().numpy()
    ulp = np.spacing(np.abs(x_ref).astype(np.float32))
    assert np.all(np.abs(x - x_ref) <= 2 * ulp)
    # argument checks (before any launch)
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.residual_rmsnorm(hd, yd, hd, rows, H, 1e-6)            # h and x overlap
    assert ei.value.code == dmoe._abi.ERR_INVALID_ARG
    with pytest.raises(dmoe.DmoeError) as ei:
        ctx.residual_rmsnorm(hd, yd, xd, rows, H - 2, 1e-6)        # n_embd % 4
    assert ei.value.code == dmoe._abi.ERR_SHAPE


def test_injected_alloc_failure(O, monkeypatch):
    import dmoe
    from dmoe import synth
    _say("case: injected workspace allocation failure")
    cfg = synth.CONFIGS["tiny"]
    w = synth.host_layer(cfg, 1, O.quantize_rows)
    c = dmoe.Context(0)
    layer = c.upload(w)
    monkeypatch.setenv("DMOE_FAIL_ALLOC", "1")
    with pytest.raises(dmoe.DmoeError) as ei:
        c.forward(layer, synth.make_x(cfg, 1))
    assert ei.value.code == dmoe._abi.ERR_OOM
    monkeypatch.delenv("DMOE_FAIL_ALLOC")
    y = c.forward(layer, synth.make_x(cfg, 1))
    assert np.isfinite(y).all()
    layer.free()
    c.close()


def _rmsnorm_np(h, eps=1e-6):
    """RMSNorm without weight (float64 mean of the float32 squares, ggml_rms_norm)."""
    sq = (h * h).astype(np.float64).sum(axis=1, keepdims=True)
    mean = (sq / h.shape[1]).astype(np.float32)
    return (h * (np.float32(1.0) / np.sqrt(mean + np.float32(eps)))).astype(np.float32)


def test_stack32_chain(ctx, O):
    """32 stacked flash-shaped Q4_K layers with Zipf-skewed routing over one
    32-token block, chained through a synthetic residual RMSNorm (eps 1e-6).
    Every layer is checked on the chain's own input: routing bit-exact, output
    within 2e-2.  The final hidden state is checked against h0 plus the
    oracle's outputs on the same per-layer inputs (the chain's accumulated
    error).  An independent CPU chain is run for information only: layer
    outputs agree to tolerance, not bit for bit, so a near-tie selection score
    deep in the stack can route differently and the two chains then part."""
    import torch
    from dmoe import synth
    cfg = synth.CONFIGS["stack32_q4k"]
    _say(f"case: {cfg.n_layers} stacked layers, {cfg.n_tokens} tokens")
    dev = torch.device("cuda:0")
    h0 = synth.make_x(cfg, 5)
    h = torch.from_numpy(h0).to(dev)
    h_ref = h0.copy()                           # h0 + oracle outputs on the chain's inputs
    h_cpu = h0.copy()                           # independent CPU chain
    keep = []                                   # router / bias referenced by the wrapped layers
    worst, split_at = 0.0, None
    for li in range(cfg.n_layers):
        wd = synth.device_layer(cfg, 5, ctx, layer=li)
        layer = ctx.wrap_device(wd)
        wh = synth.to_host(wd)
        keep.append((layer, wd.gate_w, wd.gate_bias))
        wd.exp_gate = wd.exp_up = wd.exp_down = wd.sh_gate = wd.sh_up = wd.sh_down = None
        x = _rmsnorm_np(h.cpu().numpy())
        y, dg = ctx.forward(layer, x, debug=True)
        yr, dr = O.layer_forward(wh, x, debug=True)
        _check_routing(dg, dr)
        err = max_rel_err(y, yr)
        worst = max(worst, err)
        assert err <= TOL[cfg.wtype], f"layer {li}: max rel err {err}"
        h = h + torch.from_numpy(y).to(dev)
        h_ref = h_ref + yr
        yc, dc = O.layer_forward(wh, _rmsnorm_np(h_cpu), debug=True)
        if split_at is None and not np.array_equal(dc["idx"], dg["idx"]):
            split_at = li
        h_cpu = h_cpu + yc
        del wh
        torch.cuda.empty_cache()
    hf = h.cpu().numpy()
    final = float(np.abs(hf - h_ref).max() / np.abs(h_ref).max())
    indep = float(np.abs(hf - h_cpu).max() / np.abs(h_cpu).max())
    _say(f"  per-layer max rel err {worst:.3e}; final hidden state {final:.3e}; "
         f"independent CPU chain: first routing difference at layer {split_at}, "
         f"final difference {indep:.3e}")
    assert final <= TOL_CHAIN
