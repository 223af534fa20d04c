"""Synthetic LLaDA2 MoE layers and activations.

There is no network (no checkpoint): weights are random-init with the layer
shapes of LLaDA2-flash (hidden 4096, 256 experts, moe_ff 1024, capacity 48,
top-8, routed scaling 2.5, one shared expert) or the tiny CPU case, quantised
into GGUF block bytes.

Host-side values come from a counter-based generator,
splitmix64(seed, stream, index) -> uniform -> Box-Muller, so any index of any
tensor can be regenerated independently.  Large expert tensors are generated
on the GPU (torch's seeded generator) and quantised there by
dmoe_quantize_device; the parity tests copy those bytes back for the oracle.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import (AttnWeights, DenseWeights, HeadWeights, LayerWeights, TYPE_F16, TYPE_F32, TYPE_Q4_K, TYPE_Q8_0, row_size)

_M1 = np.uint64(0x9E3779B97F4A7C15)
_M2 = np.uint64(0xBF58476D1CE4E5B9)
_M3 = np.uint64(0x94D049BB133111EB)


def splitmix64(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64) + _M1
    z = (z ^ (z >> np.uint64(30))) * _M2
    z = (z ^ (z >> np.uint64(27))) * _M3
    return z ^ (z >> np.uint64(31))


def _keys(seed: int, stream: int, n: int, salt: int = 0) -> np.ndarray:
    base = splitmix64(np.array([(seed * 0x10001 + stream * 0x1F1F1F1F + salt) & (2**64 - 1)],
                               dtype=np.uint64))[0]
    with np.errstate(over="ignore"):
        return splitmix64(np.arange(n, dtype=np.uint64) ^ base)


def uniform(seed: int, stream: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    with np.errstate(over="ignore"):
        u = (_keys(seed, stream, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 2**53)
    return (lo + (hi - lo) * u).astype(np.float32)


def normal(seed: int, stream: int, n: int, std: float = 1.0) -> np.ndarray:
    with np.errstate(over="ignore"):
        a = (_keys(seed, stream, n, 1) >> np.uint64(11)).astype(np.float64) * (1.0 / 2**53)
        b = (_keys(seed, stream, n, 2) >> np.uint64(11)).astype(np.float64) * (1.0 / 2**53)
    z = np.sqrt(-2.0 * np.log1p(-a)) * np.cos(2.0 * np.pi * b)
    return (std * z).astype(np.float32)


# tensor stream ids
S_X, S_GATE_W, S_BIAS, S_EG, S_EU, S_ED, S_SG, S_SU, S_SD = range(1, 10)
S_FG, S_FU, S_FD = range(20, 23)        # dense MLP (ffn_gate, ffn_up, ffn_down)
S_ONORM, S_OUT = 30, 31                 # step tail (output_norm, output)
S_ANORM, S_QKV, S_QN, S_KN, S_WO, S_PNORM = range(40, 46)   # attention half


@dataclass(frozen=True)
class LayerConfig:
    name: str
    n_embd: int
    n_experts: int
    moe_ff: int
    capacity: int
    top_k: int
    block_size: int
    shared_ff: int          # 0: no shared expert
    wtype: int              # routed expert type
    stype: int              # shared expert type
    n_tokens: int
    bias_lo: float
    bias_hi: float
    bias_mode: str = "uniform"     # uniform | hot | zipf
    hot_delta: float = 0.5         # the hot set's bias offset (bias_mode "hot")
    routed_scaling: float = 2.5
    n_layers: int = 1
    w_std: float = 0.02


CONFIGS = {
    # tiny CPU-runnable layer: F32 weights, 16 experts, capacity 8, top-4
    "tiny": LayerConfig("tiny", 256, 16, 128, 8, 4, 32, 128, TYPE_F32, TYPE_F32, 32, -0.05, 0.05),
    # LLaDA2-flash shape, Q8_0 experts, one 32-token block
    "flash_q8_0": LayerConfig("flash_q8_0", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q8_0,
                              TYPE_Q8_0, 32, -0.1, 0.1),
    # Q8_0 experts over 8 blocks and over the sampler's 2048-token window
    "flash_q8_0_n256": LayerConfig("flash_q8_0_n256", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q8_0,
                                   TYPE_Q8_0, 256, -0.1, 0.1),
    "flash_q8_0_n2048": LayerConfig("flash_q8_0_n2048", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q8_0,
                                    TYPE_Q8_0, 2048, -0.1, 0.1),
    # the headline workload: Q4_K experts, one 32-token block
    "flash_q4k": LayerConfig("flash_q4k", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K, TYPE_Q4_K,
                             32, -0.1, 0.1),
    # 8 independent 32-token blocks
    "flash_q4k_n256": LayerConfig("flash_q4k_n256", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K,
                                  TYPE_Q4_K, 256, -0.1, 0.1),
    # the sampler's growing window (N = 32 (blk + 1)): 16, 24, 32 and 64 blocks
    "flash_q4k_n512": LayerConfig("flash_q4k_n512", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K,
                                  TYPE_Q4_K, 512, -0.1, 0.1),
    "flash_q4k_n768": LayerConfig("flash_q4k_n768", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K,
                                  TYPE_Q4_K, 768, -0.1, 0.1),
    "flash_q4k_n1024": LayerConfig("flash_q4k_n1024", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K,
                                   TYPE_Q4_K, 1024, -0.1, 0.1),
    "flash_q4k_n2048": LayerConfig("flash_q4k_n2048", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K,
                                   TYPE_Q4_K, 2048, -0.1, 0.1),
    # F16 experts on one 32-token block (few tokens per expert on the GEMM path)
    "flash_f16": LayerConfig("flash_f16", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_F16, TYPE_F16, 32,
                             -0.1, 0.1),
    "flash_f16_n256": LayerConfig("flash_f16_n256", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_F16, TYPE_F16,
                                  256, -0.1, 0.1),
    # prompt prefill: F16 experts, 64 blocks; bias ~U(-0.05, 0.05) plus 0.05 on
    # a hot quarter of the experts, so that about 60% of each block's routed
    # pairs go to the layer's 48 most-used experts (routing_stats'
    # "share_top48"; 0.66 on the default seed, 167 experts touched, ~100
    # tokens per touched expert)
    "prefill_f16": LayerConfig("prefill_f16", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_F16,
                               TYPE_F16, 2048, -0.05, 0.05, bias_mode="hot", hot_delta=0.05),
    # 32 stacked Q4_K layers, Zipf-skewed bias, one 32-token block
    "stack32_q4k": LayerConfig("stack32_q4k", 4096, 256, 1024, 48, 8, 32, 1024, TYPE_Q4_K,
                               TYPE_Q4_K, 32, 0.0, 0.0, bias_mode="zipf", n_layers=32),
}


def make_bias(cfg: LayerConfig, seed: int, layer: int = 0) -> np.ndarray:
    E = cfg.n_experts
    s = seed + 1000 * layer
    if cfg.bias_mode == "uniform":
        return uniform(s, S_BIAS, E, cfg.bias_lo, cfg.bias_hi)
    if cfg.bias_mode == "hot":
        # a hot set of experts (a quarter) gets +hot_delta so that blocks tend
        # to agree on their most-used experts; the rest ~U(lo, hi)
        b = uniform(s, S_BIAS, E, cfg.bias_lo, cfg.bias_hi)
        order = np.argsort(uniform(s, S_BIAS + 100, E))
        b[order[: E // 4]] += np.float32(cfg.hot_delta)
        return b.astype(np.float32)
    if cfg.bias_mode == "zipf":
        # bias proportional to rank^-1.1 over a per-layer random expert order
        order = np.argsort(uniform(s, S_BIAS + 100, E))
        b = np.zeros(E, np.float32)
        b[order] = (0.5 * (np.arange(1, E + 1, dtype=np.float64) ** -1.1)).astype(np.float32)
        return b
    raise ValueError(cfg.bias_mode)


def routing_stats(idx: np.ndarray, n_experts: int, block: int) -> dict:
    """Realised routing of a layer forward: idx [N][top_k] expert ids.
    touched experts, tokens per touched expert (max, mean, histogram) and
    share_top48: the mean over blocks of the fraction of a block's routed
    pairs that go to the layer's 48 most-used experts."""
    idx = np.asarray(idx).reshape(-1, np.asarray(idx).shape[-1])
    N = idx.shape[0]
    counts = np.bincount(idx.ravel(), minlength=n_experts)
    top = np.argsort(-counts, kind="stable")[:48]
    in_top = np.isin(idx, top)
    nb = max(1, N // block)
    share = float(np.mean([in_top[b * block:(b + 1) * block].mean() for b in range(nb)]))
    edges = [1, 16, 32, 64, 128, 256, 512, 1 << 30]
    hist = {f"{lo}-{hi - 1}" if hi < (1 << 30) else f"{lo}+": int(((counts >= lo) & (counts < hi)).sum())
            for lo, hi in zip(edges[:-1], edges[1:])}
    t = counts[counts > 0]
    return {"touched_experts": int(t.size), "max_tokens_per_expert": int(counts.max()),
            "mean_tokens_per_touched_expert": round(float(t.mean()), 1) if t.size else 0.0,
            "tokens_per_expert_hist": hist, "share_top48": round(share, 3)}


def make_x(cfg: LayerConfig, seed: int, n_tokens: int | None = None) -> np.ndarray:
    N = cfg.n_tokens if n_tokens is None else n_tokens
    return normal(seed, S_X, N * cfg.n_embd).reshape(N, cfg.n_embd)


def make_router(cfg: LayerConfig, seed: int, layer: int = 0) -> np.ndarray:
    return normal(seed + 1000 * layer, S_GATE_W, cfg.n_experts * cfg.n_embd,
                  cfg.w_std).reshape(cfg.n_experts, cfg.n_embd)


def host_layer(cfg: LayerConfig, seed: int, quantize_rows, layer: int = 0) -> LayerWeights:
    """A LayerWeights in host memory.  quantize_rows(type, f32[rows, n]) -> u8 bytes
    (the caller chooses the quantiser: the oracle on a CPU-only host)."""
    H, E, FF, SF = cfg.n_embd, cfg.n_experts, cfg.moe_ff, cfg.shared_ff
    s = seed + 1000 * layer

    def q(t, stream, rows, n):
        f = normal(s, stream, rows * n, cfg.w_std).reshape(rows, n)
        return np.ascontiguousarray(quantize_rows(t, f)).view(np.uint8).reshape(rows, row_size(t, n))

    eg = q(cfg.wtype, S_EG, E * FF, H).reshape(E, FF, -1)
    eu = q(cfg.wtype, S_EU, E * FF, H).reshape(E, FF, -1)
    ed = q(cfg.wtype, S_ED, E * H, FF).reshape(E, H, -1)
    w = LayerWeights(n_embd=H, n_experts=E, top_k=cfg.top_k, capacity=cfg.capacity,
                     block_size=cfg.block_size, moe_ff=FF, wtype=cfg.wtype,
                     gate_w=make_router(cfg, seed, layer), exp_gate=eg, exp_up=eu, exp_down=ed,
                     gate_bias=make_bias(cfg, seed, layer), routed_scaling=cfg.routed_scaling)
    if SF:
        w.n_shared, w.shared_ff, w.stype = 1, SF, cfg.stype
        w.sh_gate = q(cfg.stype, S_SG, SF, H)
        w.sh_up = q(cfg.stype, S_SU, SF, H)
        w.sh_down = q(cfg.stype, S_SD, H, SF)
    return w


def device_layer(cfg: LayerConfig, seed: int, ctx, layer: int = 0, chunk_rows: int = 65536,
                 weight_seed: int | None = None):
    """A LayerWeights whose expert tensors are torch uint8 tensors on the GPU,
    generated N(0, w_std) by torch's seeded CUDA generator and quantised by
    dmoe_quantize_device.  Router and bias come from the host generator (seed);
    weight_seed (default: seed) seeds the expert tensors only, so copies with
    different weight seeds route identically."""
    import torch

    dev = torch.device(f"cuda:{ctx.device}")
    H, E, FF, SF = cfg.n_embd, cfg.n_experts, cfg.moe_ff, cfg.shared_ff
    g = torch.Generator(device=dev)
    ws = seed if weight_seed is None else weight_seed
    g.manual_seed(ws * 7919 + layer * 104729 + 17)

    def q(t, rows, n):
        rs = row_size(t, n)
        out = torch.empty((rows, rs), dtype=torch.uint8, device=dev)
        for r0 in range(0, rows, chunk_rows):
            r1 = min(rows, r0 + chunk_rows)
            f = torch.randn((r1 - r0, n), generator=g, device=dev, dtype=torch.float32)
            f.mul_(cfg.w_std)
            ctx.quantize_device(t, f, out[r0:r1], r1 - r0, n)
            torch.cuda.synchronize(dev)
            del f
        return out

    eg = q(cfg.wtype, E * FF, H).view(E, FF, -1)
    eu = q(cfg.wtype, E * FF, H).view(E, FF, -1)
    ed = q(cfg.wtype, E * H, FF).view(E, H, -1)
    gate_w = torch.from_numpy(make_router(cfg, seed, layer)).to(dev)
    bias = torch.from_numpy(make_bias(cfg, seed, layer)).to(dev)
    w = LayerWeights(n_embd=H, n_experts=E, top_k=cfg.top_k, capacity=cfg.capacity,
                     block_size=cfg.block_size, moe_ff=FF, wtype=cfg.wtype, gate_w=gate_w,
                     exp_gate=eg, exp_up=eu, exp_down=ed, gate_bias=bias,
                     routed_scaling=cfg.routed_scaling)
    if SF:
        w.n_shared, w.shared_ff, w.stype = 1, SF, cfg.stype
        w.sh_gate = q(cfg.stype, SF, H)
        w.sh_up = q(cfg.stype, SF, H)
        w.sh_down = q(cfg.stype, H, SF)
    return w


def to_host(w: LayerWeights) -> LayerWeights:
    """Copy a device LayerWeights (torch) to numpy."""
    def h(a):
        if a is None:
            return None
        return a.detach().cpu().numpy() if hasattr(a, "detach") else a
    return replace(w, gate_w=h(w.gate_w), gate_bias=h(w.gate_bias), exp_gate=h(w.exp_gate),
                   exp_up=h(w.exp_up), exp_down=h(w.exp_down), sh_gate=h(w.sh_gate),
                   sh_up=h(w.sh_up), sh_down=h(w.sh_down))


# The dense MLP of layer 0 at the LLaDA2-flash shape: hidden 4096, n_ff 9216
# (first_k_dense = 1; the intermediate size the published Q4_K_S file size
# implies for that layer).
DENSE_FLASH = (4096, 9216)


def host_dense(n_embd: int, n_ff: int, wtype: int, seed: int, quantize_rows,
               w_std: float = 0.02) -> DenseWeights:
    """A DenseWeights in host memory, N(0, w_std) weights quantised by quantize_rows."""
    def q(stream, rows, n):
        f = normal(seed, stream, rows * n, w_std).reshape(rows, n)
        return np.ascontiguousarray(quantize_rows(wtype, f)).view(np.uint8).reshape(rows, row_size(wtype, n))
    return DenseWeights(n_embd=n_embd, n_ff=n_ff, wtype=wtype, gate=q(S_FG, n_ff, n_embd),
                        up=q(S_FU, n_ff, n_embd), down=q(S_FD, n_embd, n_ff))


def device_dense(n_embd: int, n_ff: int, wtype: int, seed: int, ctx, w_std: float = 0.02) -> DenseWeights:
    """A DenseWeights on the GPU: torch's seeded generator, dmoe_quantize_device."""
    import torch
    dev = torch.device(f"cuda:{ctx.device}")
    g = torch.Generator(device=dev)
    g.manual_seed(seed * 7919 + 31)

    def q(rows, n):
        out = torch.empty((rows, row_size(wtype, n)), dtype=torch.uint8, device=dev)
        f = torch.randn((rows, n), generator=g, device=dev, dtype=torch.float32).mul_(w_std)
        ctx.quantize_device(wtype, f, out, rows, n)
        torch.cuda.synchronize(dev)
        return out
    return DenseWeights(n_embd=n_embd, n_ff=n_ff, wtype=wtype, gate=q(n_ff, n_embd),
                        up=q(n_ff, n_embd), down=q(n_embd, n_ff))


def dense_to_host(w: DenseWeights) -> DenseWeights:
    def h(a):
        return a.detach().cpu().numpy() if hasattr(a, "detach") else a
    return replace(w, gate=h(w.gate), up=h(w.up), down=h(w.down))


# The step tail of LLaDA2-flash: hidden 4096, vocabulary 157184.
HEAD_FLASH = (4096, 157184)


def host_head(n_embd: int, n_vocab: int, wtype: int, seed: int, quantize_rows,
              w_std: float = 0.02) -> HeadWeights:
    """output_norm ~ U(0.5, 1.5), output N(0, w_std) quantised by quantize_rows."""
    f = normal(seed, S_OUT, n_vocab * n_embd, w_std).reshape(n_vocab, n_embd)
    out = np.ascontiguousarray(quantize_rows(wtype, f)).view(np.uint8).reshape(n_vocab, row_size(wtype, n_embd))
    return HeadWeights(n_embd=n_embd, n_vocab=n_vocab, wtype=wtype,
                       norm=uniform(seed, S_ONORM, n_embd, 0.5, 1.5), output=out)


def device_head(n_embd: int, n_vocab: int, wtype: int, seed: int, ctx, w_std: float = 0.02,
                chunk_rows: int = 32768) -> HeadWeights:
    import torch
    dev = torch.device(f"cuda:{ctx.device}")
    g = torch.Generator(device=dev)
    g.manual_seed(seed * 7919 + 131)
    out = torch.empty((n_vocab, row_size(wtype, n_embd)), dtype=torch.uint8, device=dev)
    for r0 in range(0, n_vocab, chunk_rows):
        r1 = min(n_vocab, r0 + chunk_rows)
        f = torch.randn((r1 - r0, n_embd), generator=g, device=dev, dtype=torch.float32).mul_(w_std)
        ctx.quantize_device(wtype, f, out[r0:r1], r1 - r0, n_embd)
        torch.cuda.synchronize(dev)
        del f
    norm = torch.from_numpy(uniform(seed, S_ONORM, n_embd, 0.5, 1.5)).to(dev)
    return HeadWeights(n_embd=n_embd, n_vocab=n_vocab, wtype=wtype, norm=norm, output=out)


def head_to_host(w: HeadWeights) -> HeadWeights:
    def h(a):
        return a.detach().cpu().numpy() if hasattr(a, "detach") else a
    return replace(w, norm=h(w.norm), output=h(w.output))


# LLaDA2.0-flash attention: GQA 32 / 4, head_dim 128, NEOX RoPE over the first
# 64 dims with base 3e6, QK RMSNorm, 32-token blocks.
ATTN_FLASH = dict(n_embd=4096, n_head=32, n_head_kv=4, head_dim=128, rotary_dim=64, block_length=32,
                  rope_base=3e6, rms_eps=1e-6)


def host_attn(wtype: int, seed: int, quantize_rows, n_embd: int, n_head: int, n_head_kv: int, head_dim: int,
              rotary_dim: int, block_length: int = 32, rope_base: float = 3e6, rms_eps: float = 1e-6,
              qk_norm: bool = True, w_std: float = 0.02) -> AttnWeights:
    """Norm gains ~ U(0.5, 1.5); wqkv and wo N(0, w_std) quantised by quantize_rows."""
    QD, QKV = n_head * head_dim, (n_head + 2 * n_head_kv) * head_dim

    def q(stream, rows, n):
        f = normal(seed, stream, rows * n, w_std).reshape(rows, n)
        return np.ascontiguousarray(quantize_rows(wtype, f)).view(np.uint8).reshape(rows, row_size(wtype, n))

    return AttnWeights(n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim,
                       rotary_dim=rotary_dim, block_length=block_length, rope_base=rope_base, rms_eps=rms_eps,
                       wtype=wtype, attn_norm=uniform(seed, S_ANORM, n_embd, 0.5, 1.5),
                       qkv=q(S_QKV, QKV, n_embd), wo=q(S_WO, n_embd, QD),
                       post_norm=uniform(seed, S_PNORM, n_embd, 0.5, 1.5),
                       q_norm=uniform(seed, S_QN, head_dim, 0.5, 1.5) if qk_norm else None,
                       k_norm=uniform(seed, S_KN, head_dim, 0.5, 1.5) if qk_norm else None)


def attn_to_device(w: AttnWeights, device) -> AttnWeights:
    import torch

    def d(a):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return replace(w, attn_norm=d(w.attn_norm), qkv=d(w.qkv), wo=d(w.wo), post_norm=d(w.post_norm),
                   q_norm=d(w.q_norm), k_norm=d(w.k_norm))


def device_attn(wtype: int, seed: int, ctx, n_embd: int, n_head: int, n_head_kv: int, head_dim: int,
                rotary_dim: int, block_length: int = 32, rope_base: float = 3e6, rms_eps: float = 1e-6,
                qk_norm: bool = True, w_std: float = 0.02) -> AttnWeights:
    """An AttnWeights on the GPU: projections from torch's seeded generator
    quantised by dmoe_quantize_device, norm gains ~ U(0.5, 1.5)."""
    import torch
    dev = torch.device(f"cuda:{ctx.device}")
    g = torch.Generator(device=dev)
    g.manual_seed(seed * 7919 + 57)
    QD, QKV = n_head * head_dim, (n_head + 2 * n_head_kv) * head_dim

    def q(rows, n):
        out = torch.empty((rows, row_size(wtype, n)), dtype=torch.uint8, device=dev)
        f = torch.randn((rows, n), generator=g, device=dev, dtype=torch.float32).mul_(w_std)
        ctx.quantize_device(wtype, f, out, rows, n)
        torch.cuda.synchronize(dev)
        return out

    def u(stream, n):
        return torch.from_numpy(uniform(seed, stream, n, 0.5, 1.5)).to(dev)
    return AttnWeights(n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim,
                       rotary_dim=rotary_dim, block_length=block_length, rope_base=rope_base, rms_eps=rms_eps,
                       wtype=wtype, attn_norm=u(S_ANORM, n_embd), qkv=q(QKV, n_embd), wo=q(n_embd, QD),
                       post_norm=u(S_PNORM, n_embd),
                       q_norm=u(S_QN, head_dim) if qk_norm else None,
                       k_norm=u(S_KN, head_dim) if qk_norm else None)
