"""CPU: pins the oracle's router (src/diffuse-moe-graph.cpp:203-262) and the
dispatch grouping.

* logits: exact rational emulation of the canonical fp32 order on small
  shapes (bit-exact), and a float64 error bound at the flash shape;
* the block max fold: the 1-ulp known answer (0x3f61fdaf, 0x3ea25e9b);
* threshold / allowed / top-k / weights: recomputed with numpy's sort and
  lexsort (a different mechanism from the oracle's rank counting) on many
  random blocks, plus constructed ties, the 1e-6 slack boundary, cap >= E and
  N % block != 0;
* dispatch: permutation, histogram, scan and stable-order invariants.
"""
from fractions import Fraction

import numpy as np
import pytest


def _hp(E, K, cap, blk=32, H=256, norm=1, scale=2.5):
    import dmoe
    return dmoe.hparams_of(H, E, K, cap, blk, norm_topk_prob=norm, routed_scaling=scale)


def _round_f32(q: Fraction) -> np.float32:
    """Nearest binary32 to an exact rational, ties to even."""
    c = np.float32(float(q))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - q)
        key = (d, int(np.array(cand, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return np.float32(best[1])


def _fma32(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_router_logits_canonical_order_exact(O):
    rng = np.random.default_rng(0)
    E, N, H = 3, 2, 512
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((N, H)).astype(np.float32)
    L = O.router_logits(W, x)
    for t in range(N):
        for e in range(E):
            a = []
            for l in range(64):
                acc = np.float32(0.0)
                for i in range(H // 256):
                    for j in range(4):
                        k = 256 * i + 4 * l + j
                        acc = _fma32(W[e, k], x[t, k], acc)
                a.append(acc)
            for m in (32, 16, 8, 4, 2, 1):
                a = [np.float32(a[l] + a[l ^ m]) for l in range(64)]
            assert L[t, e].view(np.uint32) == np.float32(a[0]).view(np.uint32), (t, e)


def test_router_logits_float64_bound(O):
    rng = np.random.default_rng(1)
    E, N, H = 16, 4, 4096
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((N, H)).astype(np.float32)
    L = O.router_logits(W, x).astype(np.float64)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    absref = np.abs(x.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
    # 64 sequential fma chains of 64 terms + 6 pairwise rounds: <= ~70 u sum|w x|
    assert np.all(np.abs(L - ref) <= 70 * 2**-24 * absref)


def test_block_fold_known_answer(O):
    a = np.array([0x3f61fdaf], np.uint32).view(np.float32)[0]
    b = np.array([0x3ea25e9b], np.uint32).view(np.float32)[0]
    m = O.block_fold(np.array([a, b], np.float32))
    assert np.array([m], np.float32).view(np.uint32)[0] == 0x3f61fdb0     # a + 1 ulp, not max
    # equal scores fold to themselves; a larger later score is taken exactly
    assert O.block_fold(np.full(32, 0.375, np.float32)) == np.float32(0.375)
    assert O.block_fold(np.array([0.1, 0.2, 0.7], np.float32)) == np.float32(0.7)


def _check_route(hp, logits, bias, r):
    N, E = logits.shape
    K, cap, blk = hp.top_k, hp.capacity, hp.block_size
    p = r["probs"]
    with np.errstate(over="ignore"):
        e = np.exp(-logits.astype(np.float64)).astype(np.float32)
    # probs: 1/(1+exp(-L)) with a correctly rounded exp (at most 1 ulp off in exp)
    pref = np.float32(1) / (np.float32(1) + e)
    assert np.abs(p.view(np.int32).astype(np.int64) - pref.view(np.int32)).max() <= 1
    s = p + (bias if bias is not None else np.float32(0))
    sel = s.copy()
    use = blk > 1 and 0 < cap < E and N % blk == 0
    assert r["use_block_routing"] == use
    if use:
        for b in range(N // blk):
            blk_s = s[b * blk:(b + 1) * blk]
            bm = r["bmax"][b]
            for ee in range(E):
                assert bm[ee] == O_fold(blk_s[:, ee])
            thr = np.sort(bm)[::-1][cap - 1]
            assert r["thr"][b] == thr
            allowed = bm > np.float32(thr + np.float32(-1e-6))
            assert np.array_equal(r["allowed"][b].astype(bool), allowed)
            assert allowed.sum() >= cap
            sel[b * blk:(b + 1) * blk] += np.where(allowed, np.float32(0), np.float32(-1e30))
    for t in range(N):
        order = np.lexsort((np.arange(E), -sel[t].astype(np.float64)))
        assert np.array_equal(r["idx"][t], order[:K]), t
        w = p[t, order[:K]]
        if hp.norm_topk_prob:
            w = w / np.float32(w.astype(np.float64).sum())
        if hp.routed_scaling != 1.0:
            w = w * np.float32(hp.routed_scaling)
        assert np.array_equal(r["weights"][t], w.astype(np.float32)), t


O_fold = None


@pytest.fixture(autouse=True)
def _fold(O):
    global O_fold
    O_fold = O.block_fold


@pytest.mark.parametrize("seed", range(6))
def test_route_random_blocks(O, seed):
    rng = np.random.default_rng(100 + seed)
    E, K, cap, N = [(16, 4, 8, 64), (64, 6, 12, 96), (256, 8, 48, 64)][seed % 3]
    hp = _hp(E, K, cap)
    logits = (rng.standard_normal((N, E)) * 1.28).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, E).astype(np.float32) if seed % 2 == 0 else None
    _check_route(hp, logits, bias, O.route(hp, logits, bias))


def test_route_slack_admits_more_than_capacity(O):
    E, K, cap = 16, 2, 4
    hp = _hp(E, K, cap)
    logits = np.zeros((32, E), np.float32)        # probs 0.5 everywhere
    bias = np.full(E, -0.2, np.float32)
    bias[:cap] = 0.1                               # cap experts at bmax 0.6
    tp = np.float32(np.float32(0.6) + np.float32(-1e-6))
    bias[cap] = np.float32(np.float32(0.6) - np.float32(4e-7)) - np.float32(0.5)  # inside slack
    bias[cap + 1] = tp - np.float32(0.5)           # exactly thr - 1e-6: not allowed (strict >)
    bias[cap + 2] = np.float32(0.6 - 3e-6) - np.float32(0.5)                      # outside slack
    r = O.route(hp, logits, bias)
    assert r["thr"][0] == np.float32(0.6)
    al = r["allowed"][0].astype(bool)
    assert al[:cap].all() and al[cap] and not al[cap + 1] and not al[cap + 2]
    assert al.sum() == cap + 1
    _check_route(hp, logits, bias, r)


def test_route_ties_pick_lower_ids(O):
    hp = _hp(16, 4, 8)
    logits = np.zeros((32, 16), np.float32)
    r = O.route(hp, logits, None)
    assert r["allowed"].all()                       # all bmax equal thr
    assert np.array_equal(r["idx"], np.tile(np.arange(4), (32, 1)))
    assert np.allclose(r["weights"], 2.5 / 4)


@pytest.mark.parametrize("case", ["cap_ge_E", "N_not_multiple", "cap_zero", "blk_one"])
def test_route_plain_topk_cases(O, case):
    rng = np.random.default_rng(5)
    E, K, N = 16, 4, 32
    hp = {"cap_ge_E": _hp(E, K, 16), "N_not_multiple": _hp(E, K, 8),
          "cap_zero": _hp(E, K, 0), "blk_one": _hp(E, K, 8, blk=1)}[case]
    if case == "N_not_multiple":
        N = 40
    logits = (rng.standard_normal((N, E)) * 1.28).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    r = O.route(hp, logits, bias)
    assert not r["use_block_routing"]
    _check_route(hp, logits, bias, r)


@pytest.mark.parametrize("norm,scale", [(0, 1.0), (1, 1.0), (0, 2.5)])
def test_route_weight_options(O, norm, scale):
    rng = np.random.default_rng(6)
    hp = _hp(16, 4, 8, norm=norm, scale=scale)
    logits = (rng.standard_normal((64, 16)) * 1.28).astype(np.float32)
    r = O.route(hp, logits, None)
    _check_route(hp, logits, None, r)
    if norm:
        assert np.allclose(r["weights"].sum(1), scale, rtol=1e-6)


def test_dispatch_invariants(O):
    rng = np.random.default_rng(7)
    E, N, K = 32, 96, 6
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(N)]).astype(np.int32)
    counts, offsets, perm = O.dispatch(idx, E)
    assert np.array_equal(counts, np.bincount(idx.ravel(), minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)[:-1]]))
    assert np.array_equal(np.sort(perm), np.arange(N * K))
    flat = idx.ravel()
    for e in range(E):
        seg = perm[offsets[e]:offsets[e] + counts[e]]
        assert np.all(flat[seg] == e)
        assert np.all(np.diff(seg) > 0)      # ascending pair id: t-major, slot-minor
