#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X.

A step is one forward of the LLaDA2 block-routed MoE layer (the segment of
src/diffuse-moe-graph.cpp:188-289) over one batch of synthetic tokens, with
weights and activations already resident in HBM.  Default workload: the
LLaDA2-flash-shaped layer with Q4_K experts over one 32-token block.

Prints one JSON line with tokens/s, the roofline of the dominant kernel
(timed live with HIP events on the launch stream), the realised routing
(touched experts, tokens per expert), the CPU baseline (the oracle, timed on
this host over a bounded sample) and, under "prefill", the same record for
the 2048-token F16 prefill layer (its dominant kernel MFMA-bound).

    python bench.py [--steps K] [--warmup W] [--config flash_q4k]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "diffuse-cpp_amd"))

METRIC = "MoE-layer tokens/s + % HBM-BW roofline (32-tok block, Q4_K); prefill % MFMA"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32
MFMA_INT8_PEAK_TOPS = 5000.0   # MI355X dense int8


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="flash_q4k")
    ap.add_argument("--copies", type=int, default=3,
                    help="weight copies rotated per step so the 256 MB MALL cannot serve repeats")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--rows-steps", type=int, default=20,
                    help="calls of each row next to the segment (attention, dense MLP, step tail) "
                         "timed after the layer records (0: skip)")
    ap.add_argument("--prefill-steps", type=int, default=10,
                    help="steps of the 2048-token F16 prefill layer measured after the headline "
                         "(0: skip)")
    ap.add_argument("--config-steps", type=int, default=20,
                    help="steps of each further workload recorded under \"configs\" by the default "
                         "run (Q8_0 at 32 tokens, Q4_K at 256 and 2048 tokens; the 32-layer chain "
                         "takes a quarter as many); 0: skip")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the bench, run 5 plain device copies of this many MiB "
                         "(the calibration kernel of the HBM-traffic counters)")
    return ap.parse_args()


def traffic_from_profile(kernel, workload):
    """{"traffic": HBM bytes per launch, "traffic_source": where it comes from}
    for `kernel`: the counters are not read in this run (rocprofv3 --pmc runs
    apart from the timed ones), so the value is the one the committed summary
    under profiles/ holds (FETCH_SIZE + WRITE_SIZE of that launch, scaled by
    the counters' reading of a device copy of known size); None without one."""
    f = ROOT / "profiles" / f"{kernel}_{workload}_traffic.md"
    if f.exists():
        for line in f.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return {"traffic": int(line.split(":", 1)[1].strip()),
                        "traffic_source": f"profiles/{f.name} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                                          "copied from the committed summary, not measured in this run)"}
    return {"traffic": None, "traffic_source": None}


def cpu_info():
    """CPU model and physical core count of this host (/proc/cpuinfo)."""
    model, cores = None, set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    flags = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                flags = line
                break
    except OSError:
        pass
    isa = [f for f in ("avx2", "avx512f", "avx512_vnni", "avx_vnni", "amx_int8") if f" {f}" in flags]
    return {"model": model, "physical_cores": len(cores) or None, "logical_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "isa": isa}


def uses_tile_kernels(cfg):
    """Whether the library runs cfg's expert products on its tile kernels
    (k_expert_tile.hip): the rule of use_tile_path in dmoe_api.cpp for the
    flash shapes (Q8_0 always; Q4_K from 8 pairs per expert averaged over
    all experts, N k / E; F16 below 8), DMOE_EXPERT_TILE overriding it."""
    import dmoe
    env = os.environ.get("DMOE_EXPERT_TILE")
    if env in ("0", "1"):
        return env == "1"
    avg = cfg.n_tokens * cfg.top_k // cfg.n_experts
    if cfg.wtype == dmoe.TYPE_Q8_0:
        return True
    if cfg.wtype == dmoe.TYPE_Q4_K:
        return avg >= 8
    if cfg.wtype == dmoe.TYPE_F16:
        return avg < 8
    return False


def uses_q4k_gemm(cfg):
    """Whether the library runs cfg's Q4_K expert products on its grouped
    GEMM (k_expert_gemm.hip): the rule of use_q4k_gemm in dmoe_api.cpp for
    the flash shapes (64 or more pairs per expert averaged over all experts,
    N k / E), DMOE_EXPERT_GEMM overriding it and DMOE_EXPERT_TILE turning it
    off."""
    import dmoe
    if cfg.wtype != dmoe.TYPE_Q4_K:
        return False
    env = os.environ.get("DMOE_EXPERT_GEMM")
    if env in ("0", "1"):
        return env == "1"
    if os.environ.get("DMOE_EXPERT_TILE") in ("0", "1") or os.environ.get("DMOE_Q4K_COLUMN_BLOCKS"):
        return False
    return cfg.n_tokens * cfg.top_k // cfg.n_experts >= 64


def bench_layer(a, cfg, steps, warmup, copies, cpu_seconds, cpu_tokens=None):
    """One MoE layer of config cfg: tokens/s, per-stage times, the dominant
    kernel's roofline, realised routing and (cpu_seconds > 0) the oracle's
    rate on this host, over the first cpu_tokens tokens of the input (all of
    them by default)."""
    import numpy as np
    import torch
    import dmoe
    from dmoe import synth

    N, H, FF, E, K = cfg.n_tokens, cfg.n_embd, cfg.moe_ff, cfg.n_experts, cfg.top_k
    ctx = dmoe.Context(0)
    dev = torch.device("cuda:0")

    t0 = time.time()
    weights = [synth.device_layer(cfg, a.seed, ctx, weight_seed=a.seed + 17 * i)
               for i in range(copies)]
    layers = [ctx.wrap_device(w) for w in weights]
    print(f"# {cfg.name}: built {copies} weight copies in {time.time() - t0:.1f}s", file=sys.stderr,
          flush=True)
    x_host = synth.make_x(cfg, a.seed)
    x = torch.from_numpy(x_host).to(dev)
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    # routing of this input (identical for every copy: same router and bias)
    _, dbg = ctx.forward(layers[0], x_host, debug=True)
    counts = dbg["counts"]
    touched = int((counts > 0).sum())
    routing = synth.routing_stats(dbg["idx"].reshape(N, K), E, cfg.block_size)
    eb = weights[0].expert_bytes()
    sb = weights[0].shared_bytes()

    def step(i):
        ctx.forward_device(layers[i % copies], x, N, y, sp)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    ms_step = ev0.elapsed_time(ev1) / steps

    # per-stage durations, HIP events around each launch on the same stream
    ctx.profile(True)
    for i in range(steps):
        step(i)
    torch.cuda.synchronize(dev)
    prof = ctx.profile_read()
    ctx.profile(False)
    stages = {k: round(v[0] / v[1] * 1e3, 2) for k, v in prof.items()}   # us per launch

    # The dominant kernel is the gate/up launch (routed experts and the shared
    # expert in one launch).  Streaming launches (Q4_K, Q8_0, and F16 at few
    # tokens per expert: HBM-bound): its algorithmic bytes are the touched
    # experts' and the shared expert's gate and up matrices, the activations
    # in their operand layout (int8 values with, for Q4_K, f16 sums of 16 and
    # an f32 scale per 256, for Q8_0 an f32 scale per 32; the shared expert's
    # as two int8 digit rows; F16: f16 hi / lo rows) and h written (the
    # few-token Q4_K kernel: in the down products' operand layout; the tile
    # kernels: f32).  The F16 grouped GEMM (the prefill, MFMA-bound): its
    # algorithmic FLOPs, 2 per multiply-add of the routed pairs' and the
    # tokens' shared gate and up products (the shared expert's two f16 passes
    # count once).
    rs_h = dmoe.row_size(cfg.wtype, H)
    SF = cfg.shared_ff
    P = N * K
    dom_stage = "gateup_routed"
    dom_us = stages.get(dom_stage)
    flops = 2.0 * N * (K * 3 * H * FF + 3 * H * SF + H * E)
    tile = uses_tile_kernels(cfg)
    if cfg.wtype == dmoe.TYPE_F16 and not tile:
        dom_kernel = "dmoe::k_gemm_f16<0>"
        dom_flops = 2.0 * (P * 2 * H * FF + N * 2 * H * SF)
        achieved = dom_flops / (dom_us * 1e-6) / 1e12 if dom_us else None
        # the launch must also stream the touched experts' gate and up
        # weights: the MFMA fraction it can reach is its MFMA time over the
        # longer of that and the weights' HBM time
        w_bytes = touched * 2 * FF * rs_h + 2 * SF * rs_h
        t_mfma = dom_flops / (MFMA_F16_PEAK_TFLOPS * 1e12)
        t_hbm = w_bytes / (HBM_PEAK_GBS * 1e9)
        roofline = {"bound": "mfma", "kernel": dom_stage,
                    "achieved": round(achieved, 1) if achieved else None,
                    "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4) if achieved else None,
                    "attainable_frac": round(t_mfma / max(t_mfma, t_hbm), 4),
                    "weight_bytes": w_bytes,
                    "weight_hbm_frac": (round(w_bytes / (dom_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                                        if dom_us else None),
                    **traffic_from_profile(dom_stage, cfg.name),
                    "algorithmic_flops": dom_flops, "hip_kernel": dom_kernel, "us_per_launch": dom_us}
    else:
        fmt = {dmoe.TYPE_Q4_K: "FmtQ4K", dmoe.TYPE_Q8_0: "FmtQ80", dmoe.TYPE_F16: "FmtF16"}.get(cfg.wtype)
        if cfg.wtype == dmoe.TYPE_Q4_K:
            def act_row(n):
                return n + (n // 16) * 2 + (n // 256) * 4
        elif cfg.wtype == dmoe.TYPE_Q8_0:
            def act_row(n):
                return n + (n // 32) * 4
        else:
            def act_row(n):
                return 2 * n
        if uses_q4k_gemm(cfg):
            dom_kernel = "dmoe::k_gemm_q4k<false>"
            h_bytes = P * FF * 4 + N * SF * 4
        elif fmt and tile:
            dom_kernel = f"dmoe::k_gu_rr<dmoe::{fmt}>"
            h_bytes = P * FF * 4 + N * SF * 4
        elif cfg.wtype == dmoe.TYPE_Q4_K:
            # items of one column block on the register-ring kernel
            dom_kernel = "dmoe::k_gateup_rr<true>"
            h_bytes = P * act_row(FF) + 2 * N * act_row(SF)
        else:
            dom_kernel = "dmoe::k_gateup_routed"
            h_bytes = P * FF * 4
        # x rows in (routed, shared digit rows), h out
        dom_bytes = touched * 2 * FF * rs_h + 2 * SF * rs_h + 3 * N * act_row(H) + h_bytes
        achieved = dom_bytes / (dom_us * 1e-6) / 1e9 if dom_us else None
        roofline = {"bound": "hbm", "kernel": dom_stage,
                    "achieved": round(achieved, 1) if achieved else None,
                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
                    **traffic_from_profile(dom_stage, cfg.name),
                    "algorithmic_bytes": dom_bytes, "hip_kernel": dom_kernel, "us_per_launch": dom_us}
        if cfg.wtype in (dmoe.TYPE_Q4_K, dmoe.TYPE_Q8_0) and dom_us:
            # the same launch against dense int8 MFMA: its integer dot
            # products, 2 per multiply-add of the routed pairs' and the
            # tokens' shared gate and up rows (the shared expert's two
            # digit rows count once)
            ops = 2.0 * (P * 2 * H * FF + N * 2 * H * SF)
            roofline["int8_ops"] = ops
            roofline["int8_frac"] = round(ops / (dom_us * 1e-6) / (MFMA_INT8_PEAK_TOPS * 1e12), 4)

    # layer-level: every weight byte the layer must read
    layer_bytes = touched * eb + sb + E * H * 4 + E * 4 + 2 * N * H * 4
    sec = ms_step * 1e-3
    rec = {
        "value": round(N / sec, 1),
        "ms_per_step": round(ms_step, 5),
        "steps": steps,
        "warmup": warmup,
        "dtype": {dmoe.TYPE_Q4_K: "i8", dmoe.TYPE_Q8_0: "i8", dmoe.TYPE_F16: "f16",
                  dmoe.TYPE_F32: "f32"}[cfg.wtype],
        "config": {
            "workload": (f"{cfg.name}: LLaDA2 MoE layer, hidden {H}, {E} experts, moe_ff {FF}, "
                         f"top-{K} within capacity {cfg.capacity} per {cfg.block_size}-token block, "
                         f"shared ff {cfg.shared_ff}, {dmoe.TYPE_NAMES[cfg.wtype]} experts, "
                         f"{N} tokens"),
            "n_tokens": N,
            "expert_type": dmoe.TYPE_NAMES[cfg.wtype],
            "router_bias": (f"{cfg.bias_mode} U({cfg.bias_lo}, {cfg.bias_hi})"
                            + (f" + {cfg.hot_delta} on a hot quarter" if cfg.bias_mode == "hot" else "")),
            "weight_copies_rotated": copies,
            **routing,
        },
        "roofline": roofline,
        "layer": {
            "bytes": layer_bytes,
            "touched_expert_bytes": touched * eb,
            "GB_s": round(layer_bytes / sec / 1e9, 1),
            "hbm_frac": round(layer_bytes / sec / 1e9 / HBM_PEAK_GBS, 4),
            "touched_expert_frac": round(touched * eb / sec / 1e9 / HBM_PEAK_GBS, 4),
            "tflops": round(flops / sec / 1e12, 2),
            "mfma_frac": round(flops / sec / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "stage_us": stages,
        },
    }

    if cpu_seconds > 0:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O
        wh = synth.to_host(weights[0])
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        ns = min(N, cpu_tokens or N)
        xs = np.ascontiguousarray(x_host[:ns])
        # the dots through AVX-512 where the host has it (quantised: VNNI,
        # the same results bit for bit as the scalar dots; F32 / F16: binary32
        # sums in ggml's SIMD order)
        simd = O.set_simd(True)
        yr = O.layer_forward(wh, xs, n_threads=threads)     # warm-up
        reps, t_start = 0, time.time()
        while True:
            O.layer_forward(wh, xs, n_threads=threads)
            reps += 1
            el = time.time() - t_start
            if el >= cpu_seconds or reps >= 1000:
                break
        info = cpu_info()
        part = (f"the same {N}-token layer" if ns == N else
                f"the first {ns} of the {N} tokens ({ns // cfg.block_size} blocks, each routed alone as in the "
                f"full input)")
        rec["cpu_baseline"] = {
            "value": round(ns * reps / el, 2),
            "unit": "tokens/s",
            "cores": threads,
            "kind": "port",
            "sample": f"{reps} forwards of {part} ({el:.1f} s), oracle (C, gcc -O2, OpenMP over rows; "
                      f"dots {'AVX-512 (VNNI for the quantised types; binary32 F32 / F16 sums)' if simd else 'scalar'}) "
                      f"with {threads} threads",
            "cpu_model": info["model"],
            "physical_cores": info["physical_cores"],
            "logical_cpus": info["logical_cpus"],
            "affinity_cpus": info["affinity_cpus"],
            "isa": info["isa"],
        }
        O.set_simd(False)
        # the GPU forward of the same sample, checked against the oracle
        xd = torch.from_numpy(xs).to(dev)
        yd = torch.empty_like(xd)
        ctx.forward_device(layers[0], xd, ns, yd, sp)
        torch.cuda.synchronize(dev)
        err = float(np.abs(yd.cpu().numpy() - yr).max() / np.abs(yr).max())
        rec["check_max_rel_err_vs_oracle"] = err
        del wh, xd, yd

    del layers, weights, x, y
    ctx.close()
    torch.cuda.empty_cache()
    return rec


def bench_rows(a):
    """The rows next to the MoE segment at their flash shapes, each timed over
    a.rows_steps calls with HIP events on the launch stream, weights resident
    in HBM (copies rotated past the 256 MB memory-side cache): the attention
    half of a layer (32, 256 and 2048 tokens), the dense layer-0 MLP (32
    tokens) and the step tail (final norm, 157,184-row LM head, argmax and
    confidence; 32 tokens).  All three stream weights: the roofline is HBM, the
    algorithmic bytes are stated per record."""
    import torch
    import dmoe
    from dmoe import synth

    ctx = dmoe.Context(0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    H = 4096
    rs = dmoe.row_size(dmoe.TYPE_Q4_K, H)
    out = {}

    def timed(fn, copies):
        for i in range(3):
            fn(i % copies)
        torch.cuda.synchronize(dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(a.rows_steps):
            fn(i % copies)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / a.rows_steps * 1e3          # us per call

    def stage_times(fn, copies, names):
        """us per launch of each stage over 10 profiled calls (HIP events
        around every stage on the launch stream), under the row's names"""
        ctx.profile(True)
        for i in range(10):
            fn(i % copies)
        torch.cuda.synchronize(dev)
        prof = ctx.profile_read()
        ctx.profile(False)
        return {names.get(k, k): round(v[0] / v[1] * 1e3, 2) for k, v in prof.items()}

    def rec(workload, us, nbytes, what):
        gbs = nbytes / (us * 1e-6) / 1e9
        return {"workload": workload, "us_per_call": round(us, 2), "algorithmic_bytes": int(nbytes),
                "bytes_are": what, "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}

    # attention half: 16 copies of the 20.2 MB of projections
    A = synth.ATTN_FLASH
    copies = 16
    layers, keep = [], []
    for i in range(copies):
        w = synth.device_attn(dmoe.TYPE_Q4_K, a.seed + i, ctx, **A)
        layers.append(ctx.attn_wrap_device(w))
        keep.append(w)
    QKV = (A["n_head"] + 2 * A["n_head_kv"]) * A["head_dim"]
    QD = A["n_head"] * A["head_dim"]
    wbytes = (QKV + H) * rs                                       # wqkv and wo, Q4_K
    recs = {}
    for N in (32, 256, 2048):
        h = torch.randn((N, H), device=dev)
        ho = torch.empty_like(h)
        mi = torch.empty_like(h)
        us = timed(lambda i: ctx.attn_forward_device(layers[i], h, N, ho, mi, stream=sp), copies)
        # weights, h read, h_out and moe_in written, the f32 qkv / attention
        # rows written and read once
        act = N * H * 4 * 3 + N * (QKV + QD) * 4 * 2
        recs[f"n{N}"] = rec(f"attention half, flash shape (32 / 4 heads of 128, RoPE 64, Q4_K projections), "
                            f"{N} tokens", us, wbytes + act, "wqkv + wo weights, h in, h_out and moe_in out, "
                            "qkv and attention rows written and read")
        recs[f"n{N}"]["stage_us"] = stage_times(
            lambda i: ctx.attn_forward_device(layers[i], h, N, ho, mi, stream=sp), copies,
            {"front": "input_norm", "gateup_shared": "qkv_proj", "act_quant_x": "qkv_x_quant",
             "route": "qk_norm_rope", "scores": "attention", "act_quant_h": "attn_out_quant",
             "down_shared": "out_proj", "combine": "residual_post_norm"})
        # the attention kernel against the compute roofline: Q K^T and P V
        # over each query's visible keys (block-causal, block_length B), two
        # flops per multiply-add; fp32 semantics, run as three f16 MFMA
        # products per multiply-add (hi / lo halves)
        B = A.get("block_length", 32)
        vis = sum(min(N, (q // B + 1) * B) if B > 0 else N for q in range(N))
        flops = 4.0 * A["head_dim"] * A["n_head"] * vis
        at_us = recs[f"n{N}"]["stage_us"].get("attention")
        if at_us:
            tf = flops / (at_us * 1e-6) / 1e12
            recs[f"n{N}"]["attention_kernel"] = {
                "us": at_us, "gflop": round(flops / 1e9, 3), "tflops": round(tf, 1),
                "of_fp32_mfma_peak": round(tf / MFMA_F32_PEAK_TFLOPS, 3),
                "split_f16_mfma_frac": round(3 * tf / MFMA_F16_PEAK_TFLOPS, 3)}
    out["attention"] = recs
    del layers, keep
    torch.cuda.empty_cache()

    # dense layer-0 MLP: 5 copies of 63.7 MB
    Hd, FF = synth.DENSE_FLASH
    copies = 5
    dl, keep = [], []
    for i in range(copies):
        w = synth.device_dense(Hd, FF, dmoe.TYPE_Q4_K, a.seed + i, ctx)
        dl.append(ctx.dense_wrap_device(w))
        keep.append(w)
    N = 32
    x = torch.randn((N, Hd), device=dev)
    y = torch.empty_like(x)
    us = timed(lambda i: ctx.forward_device(dl[i], x, N, y, sp), copies)
    wb = 2 * FF * dmoe.row_size(dmoe.TYPE_Q4_K, Hd) + Hd * dmoe.row_size(dmoe.TYPE_Q4_K, FF)
    out["dense_mlp"] = rec(f"dense layer-0 MLP {Hd} x {FF}, Q4_K (F32 weight semantics), {N} tokens", us,
                           wb + 2 * N * Hd * 4, "gate, up and down weights, x in, y out")
    out["dense_mlp"]["stage_us"] = stage_times(
        lambda i: ctx.forward_device(dl[i], x, N, y, sp), copies,
        {"act_quant_x": "x_quant", "gateup_shared": "gate_up_proj", "act_quant_h": "swiglu_h_quant",
         "down_shared": "down_proj", "combine": "slice_reduce"})
    del dl, keep
    torch.cuda.empty_cache()

    # step tail: 2 copies of the 362 MB LM head
    Hh, V = synth.HEAD_FLASH
    copies = 2
    hl, keep = [], []
    for i in range(copies):
        w = synth.device_head(Hh, V, dmoe.TYPE_Q4_K, a.seed + i, ctx)
        hl.append(ctx.head_wrap_device(w))
        keep.append(w)
    h = torch.randn((N, Hh), device=dev)
    tok = torch.empty(N, dtype=torch.int32, device=dev)
    prob = torch.empty(N, dtype=torch.float32, device=dev)
    us = timed(lambda i: ctx.head_forward_device(hl[i], h, N, 1e-6, tok, prob, None, sp), copies)
    wb = V * dmoe.row_size(dmoe.TYPE_Q4_K, Hh)
    out["step_tail"] = rec(f"step tail: RMSNorm, LM head {Hh} x {V} Q4_K, argmax + confidence, {N} tokens", us,
                           wb + 2 * N * V * 4 + N * Hh * 4, "output weights, logits written and read once, h in")
    out["step_tail"]["stage_us"] = stage_times(
        lambda i: ctx.head_forward_device(hl[i], h, N, 1e-6, tok, prob, None, sp), copies,
        {"front": "output_norm", "act_quant_h": "h_quant", "down_shared": "lm_head", "combine": "argmax_confidence"})
    del hl, keep
    ctx.close()
    torch.cuda.empty_cache()
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported",
                          "n_gpus": a.gpus}))
        sys.exit(2)

    import torch
    from dmoe import synth

    cfg = synth.CONFIGS[a.config]
    if cfg.n_layers != 1:
        print(json.dumps(stack_record(a, cfg, a.steps, a.warmup, line=True)))
        return
    rec = bench_layer(a, cfg, a.steps, a.warmup, a.copies, 0 if a.no_cpu else a.cpu_seconds)
    out = {
        "metric": METRIC,
        "value": rec.pop("value"),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": rec.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": rec.pop("dtype"),
        "data": "synthetic: random-init weights N(0,0.02) quantised on the GPU, x ~ N(0,1)",
    }
    rec.pop("steps")
    rec.pop("warmup")
    out.update(rec)

    # the metric's second half: the 2048-token prefill layer (F16 experts,
    # MFMA-bound), measured in the same run
    if a.prefill_steps > 0 and cfg.n_tokens <= 256:
        pcfg = synth.CONFIGS["prefill_f16"]
        # its CPU baseline over the first 256 tokens (a bounded sample: the
        # oracle's F16 dots over all 2048 would take minutes)
        pre = bench_layer(a, pcfg, a.prefill_steps, max(1, a.prefill_steps // 4), 1,
                          0 if a.no_cpu else a.cpu_seconds, cpu_tokens=256)
        pre["unit"] = "tokens/s"
        out["prefill"] = pre

    if a.rows_steps > 0 and cfg.n_tokens <= 256:
        out["rows"] = bench_rows(a)

    # the other single-GPU workloads of the layer, each its own record in the
    # same run: Q8_0 experts over one 32-token block, 8 independent blocks
    # (256 tokens) and the sampler's 2048-token window of Q4_K experts, and a
    # denoising step through 32 stacked Q4_K layers
    if a.config_steps > 0 and a.config == "flash_q4k":
        recs = {}
        for name in ("flash_q8_0", "flash_q4k_n256", "flash_q4k_n2048"):
            r = bench_layer(a, synth.CONFIGS[name], a.config_steps, max(2, a.config_steps // 4),
                            a.copies, 0)
            r["unit"] = "tokens/s"
            recs[name] = r
        recs["stack32_q4k"] = stack_record(a, synth.CONFIGS["stack32_q4k"], max(2, a.config_steps // 4),
                                           max(1, a.config_steps // 10))
        out["configs"] = recs

    if a.copy_probe_mib:
        dev = torch.device("cuda:0")
        n = a.copy_probe_mib * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        out["copy_probe_bytes"] = n * 4

    print(json.dumps(out))


def stack_record(a, cfg, steps, warmup, line=False):
    """A denoising step through cfg.n_layers stacked MoE layers (all resident in
    HBM), chained h <- h + MoE_l(RMSNorm(h)) over one token block; the
    residual add and the next layer's RMSNorm run as one library kernel
    (dmoe_residual_rmsnorm) between the layers.  Returns the step's record:
    tokens/s, per-layer time, the touched experts of every layer on the
    chain's own inputs and the step's HBM roofline (the touched experts'
    bytes of all layers over the step time).  line: the fields of a
    stand-alone bench line as well."""
    import numpy as np
    import torch
    import dmoe
    from dmoe import synth

    N, H, FF, E, K = cfg.n_tokens, cfg.n_embd, cfg.moe_ff, cfg.n_experts, cfg.top_k
    ctx = dmoe.Context(0)
    dev = torch.device("cuda:0")
    t0 = time.time()
    layers, keep = [], []
    eb = sb = None
    for li in range(cfg.n_layers):
        wd = synth.device_layer(cfg, a.seed, ctx, layer=li)
        if eb is None:
            eb, sb = wd.expert_bytes(), wd.shared_bytes()
        layers.append(ctx.wrap_device(wd))
        keep.append((wd.gate_w, wd.gate_bias))
        # the library keeps its own tiled copy of the Q4_K experts
        wd.exp_gate = wd.exp_up = wd.exp_down = wd.sh_gate = wd.sh_up = wd.sh_down = None
        torch.cuda.empty_cache()
    print(f"# {cfg.name}: built {cfg.n_layers} layers in {time.time() - t0:.1f}s", file=sys.stderr,
          flush=True)
    h0 = torch.from_numpy(synth.make_x(cfg, a.seed)).to(dev)
    y = torch.empty_like(h0)
    x = torch.empty_like(h0)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    eps = 1e-6

    def step():
        h = h0.clone()
        ctx.residual_rmsnorm(h, None, x, N, H, eps, stream=sp)          # x = RMSNorm(h0)
        for L in layers:
            ctx.forward_device(L, x, N, y, sp)
            ctx.residual_rmsnorm(h, y, x, N, H, eps, stream=sp)         # h += y; x = RMSNorm(h)
        return h

    # touched experts of each layer on the chain's own inputs
    touched = []
    h = h0.clone()
    ctx.residual_rmsnorm(h, None, x, N, H, eps, stream=sp)
    for L in layers:
        torch.cuda.synchronize(dev)
        _, dbg = ctx.forward(L, x.cpu().numpy(), debug=True)
        touched.append(int((dbg["counts"] > 0).sum()))
        ctx.forward_device(L, x, N, y, sp)
        ctx.residual_rmsnorm(h, y, x, N, H, eps, stream=sp)
    torch.cuda.synchronize(dev)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    ms_step = ev0.elapsed_time(ev1) / steps
    ctx.profile(True)
    step()
    torch.cuda.synchronize(dev)
    prof = ctx.profile_read()
    ctx.profile(False)
    stages = {k: round(v[0] / v[1] * 1e3, 2) for k, v in prof.items()}
    sec = ms_step * 1e-3
    t_bytes = sum(touched) * eb
    all_bytes = t_bytes + cfg.n_layers * (sb + E * H * 4 + E * 4 + 2 * N * H * 4 + 4 * N * H * 4)
    rec = {
        "value": round(N / sec, 1),
        "unit": "tokens/s",
        "ms_per_step": round(ms_step, 5),
        "steps": steps,
        "warmup": warmup,
        "dtype": "i8",
        "config": {
            "workload": (f"{cfg.name}: {cfg.n_layers} stacked LLaDA2 MoE layers (hidden {H}, {E} "
                         f"experts, moe_ff {FF}, top-{K} within capacity {cfg.capacity}, Q4_K, "
                         f"Zipf-skewed bias), one {N}-token denoising step, residual RMSNorm chain"),
            "n_tokens": N,
            "n_layers": cfg.n_layers,
            "expert_type": dmoe.TYPE_NAMES[cfg.wtype],
            "touched_experts_per_layer": touched,
        },
        # every layer streams its touched experts once per step: the step is
        # HBM bound
        "roofline": {"bound": "hbm", "kernel": "whole step (all layers)",
                     "achieved": round(t_bytes / sec / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(t_bytes / sec / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "traffic_source": None, "algorithmic_bytes": t_bytes,
                     "bytes_are": "touched experts' weights of all layers"},
        "layer_us": round(ms_step * 1e3 / cfg.n_layers, 2),
        "step": {"bytes": all_bytes, "hbm_frac": round(all_bytes / sec / 1e9 / HBM_PEAK_GBS, 4),
                 "touched_expert_frac": round(t_bytes / sec / 1e9 / HBM_PEAK_GBS, 4)},
        "stage_us": stages,
    }
    del layers, keep, x, y, h0, h
    ctx.close()
    torch.cuda.empty_cache()
    if line:
        rec = {"metric": METRIC, **rec, "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None,
               "data": "synthetic: random-init weights N(0,0.02) quantised on the GPU, x ~ N(0,1)"}
    return rec


if __name__ == "__main__":
    main()
