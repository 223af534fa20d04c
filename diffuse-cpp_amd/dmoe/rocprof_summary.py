"""Short text summaries of rocprofv3 CSV output (``--output-format csv``).

Two reports:

* ``kernels``: the per-kernel table of a ``--kernel-trace --stats`` run
  (calls, average and total duration, share of GPU time).
* ``counters``: per-dispatch means of the SQ / GRBM counters of one
  ``--pmc`` run for chosen kernels, with the utilisations they imply:
  MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (G x SIMDs), VALU busy =
  4 SQ_ACTIVE_INST_VALU / (G x SIMDs) (a wave64 VALU instruction occupies a
  SIMD four cycles), G = GRBM_GUI_ACTIVE / XCDs (the counter sums the busy
  cycles of every XCD: G matches the kernel's duration at the shader clock),
  LDS bank-conflict share = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.
* ``traffic``: HBM bytes per launch of one kernel from two ``--pmc`` runs,
  ``FETCH_SIZE`` then ``WRITE_SIZE`` (both in KiB per dispatch).  Each counter
  is scaled by what it reads for a plain device copy of known size run in the
  same process (``bench.py --copy-probe-mib``): the copy reads and writes
  exactly its size, so ``size / counter`` converts the counter to bytes.  Only
  the copy kernel's large dispatches (at least half its largest) count as the
  probe.  The report carries a ``traffic_bytes_per_launch:`` line that
  bench.py reads.

    python -m dmoe.rocprof_summary kernels --dir D --cmd "..." --out F
    python -m dmoe.rocprof_summary counters --dir D --kernel "k_gemm_f16<0>" \\
        --cmd "..." --out F
    python -m dmoe.rocprof_summary traffic --fetch D1 --write D2 \\
        --kernel "k_expert_q4k<0>" --copy-bytes B --cmd-fetch "..." \\
        --cmd-write "..." --algorithmic-bytes A --out F
"""
from __future__ import annotations

import argparse
import csv
import statistics
from pathlib import Path


def _rows(directory: str, suffix: str):
    files = sorted(Path(directory).rglob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {directory}")
    out = []
    for f in files:
        with open(f, newline="") as fh:
            out.extend(csv.DictReader(fh))
    return out


def kernel_stats(directory: str):
    rows = _rows(directory, "kernel_stats.csv")
    res = []
    for r in rows:
        res.append({
            "name": r["Name"],
            "calls": int(r["Calls"]),
            "avg_us": float(r["AverageNs"]) / 1e3,
            "total_us": float(r["TotalDurationNs"]) / 1e3,
            "pct": float(r["Percentage"]),
            "min_us": float(r["MinNs"]) / 1e3,
            "max_us": float(r["MaxNs"]) / 1e3,
        })
    res.sort(key=lambda d: -d["total_us"])
    return res


def counter_values(directory: str, counter: str):
    """{kernel name: [value per dispatch]} for one counter."""
    rows = _rows(directory, "counter_collection.csv")
    per = {}
    for r in rows:
        if r.get("Counter_Name") != counter:
            continue
        per.setdefault(r["Kernel_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
        per[r["Kernel_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
    return {k: list(v.values()) for k, v in per.items()}


def _short(name: str, width: int = 70) -> str:
    name = name.replace("void ", "").split("(")[0]
    return name if len(name) <= width else name[: width - 3] + "..."


def _pick(per: dict, pattern: str, largest: bool = False):
    hits = {k: v for k, v in per.items() if pattern in k}
    if not hits:
        raise SystemExit(f"no kernel matching {pattern!r}; have {list(per)[:20]}")
    if largest:
        return max(hits.items(), key=lambda kv: statistics.mean(kv[1]))
    if len(hits) > 1:
        raise SystemExit(f"{pattern!r} matches several kernels: {list(hits)}")
    return next(iter(hits.items()))


def report_kernels(a):
    ks = kernel_stats(a.dir)
    lines = [f"# Kernel trace: {a.title}", "", "Command:", "", "```", a.cmd, "```", "",
             "| kernel | calls | avg us | min us | max us | % GPU time |",
             "|---|---:|---:|---:|---:|---:|"]
    for k in ks:
        lines.append(f"| `{_short(k['name'])}` | {k['calls']} | {k['avg_us']:.2f} | "
                     f"{k['min_us']:.2f} | {k['max_us']:.2f} | {k['pct']:.1f} |")
    Path(a.out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def report_counters(a):
    rows = _rows(a.dir, "counter_collection.csv")
    per = {}
    for r in rows:
        d = per.setdefault(r["Kernel_Name"], {}).setdefault(r["Dispatch_Id"], {})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    simds = a.simds
    lines = [f"# SQ counters: {a.title}", "", "Command:", "", "```", a.cmd, "```", "",
             f"Per-dispatch means over the kernel's dispatches; {simds} SIMDs, {a.xcds} XCDs.", "",
             "| kernel | dispatches | counter | mean per dispatch |", "|---|---:|---|---:|"]
    derived = ["", "| kernel | MFMA busy | VALU busy | VALU instr / wave | LDS bank-conflict share |",
               "|---|---:|---:|---:|---:|"]
    for pat in a.kernel:
        hits = {k: v for k, v in per.items() if pat in k}
        if not hits:
            raise SystemExit(f"no kernel matching {pat!r}")
        for kname, disp in hits.items():
            names = sorted({c for d in disp.values() for c in d})
            mean = {c: statistics.mean(d.get(c, 0.0) for d in disp.values()) for c in names}
            for c in names:
                lines.append(f"| `{_short(kname)}` | {len(disp)} | {c} | {mean[c]:.1f} |")
            gui = mean.get("GRBM_GUI_ACTIVE", 0.0) / a.xcds
            mf = mean.get("SQ_VALU_MFMA_BUSY_CYCLES")
            va = mean.get("SQ_ACTIVE_INST_VALU")
            waves = mean.get("SQ_WAVES")
            lds = mean.get("SQ_LDS_IDX_ACTIVE")
            cells = [
                f"{mf / (gui * simds):.3f}" if mf is not None and gui else "-",
                f"{4 * va / (gui * simds):.3f}" if va is not None and gui else "-",
                f"{mean['SQ_INSTS_VALU'] / waves:.0f}" if waves and "SQ_INSTS_VALU" in mean else "-",
                f"{mean['SQ_LDS_BANK_CONFLICT'] / lds:.3f}" if lds and "SQ_LDS_BANK_CONFLICT" in mean else "-",
            ]
            derived.append(f"| `{_short(kname)}` | " + " | ".join(cells) + " |")
    out = lines + derived
    Path(a.out).write_text("\n".join(out) + "\n")
    print("\n".join(out))


def report_traffic(a):
    fetch = counter_values(a.fetch, "FETCH_SIZE")
    write = counter_values(a.write, "WRITE_SIZE")
    kname, kf = _pick(fetch, a.kernel)
    _, kw = _pick(write, a.kernel)
    cname, cf = _pick(fetch, a.copy_kernel, largest=True)
    _, cw = _pick(write, cname)
    # the probe's dispatches are the large ones (the same kernel also serves
    # small runtime copies)
    cf = [v for v in cf if v >= 0.5 * max(cf)]
    cw = [v for v in cw if v >= 0.5 * max(cw)]
    cb = a.copy_bytes
    f_read = cb / (statistics.mean(cf) * 1024.0)
    f_write = cb / (statistics.mean(cw) * 1024.0)
    rd = statistics.mean(kf) * 1024.0 * f_read
    wr = statistics.mean(kw) * 1024.0 * f_write
    traffic = int(round(rd + wr))
    lines = [
        f"# HBM traffic: {a.title}", "",
        "Commands (one counter per run):", "", "```", a.cmd_fetch, a.cmd_write, "```", "",
        f"kernel: `{_short(kname, 120)}` ({len(kf)} dispatches with FETCH_SIZE, "
        f"{len(kw)} with WRITE_SIZE)",
        f"calibration kernel: `{_short(cname, 120)}` copying {cb} bytes "
        f"({len(cf)} dispatches)", "",
        "| quantity | value |", "|---|---:|",
        f"| copy FETCH_SIZE, KiB/dispatch | {statistics.mean(cf):.1f} |",
        f"| copy WRITE_SIZE, KiB/dispatch | {statistics.mean(cw):.1f} |",
        f"| read scale (bytes per counted byte) | {f_read:.4f} |",
        f"| write scale (bytes per counted byte) | {f_write:.4f} |",
        f"| kernel FETCH_SIZE, KiB/dispatch (mean / min / max) | {statistics.mean(kf):.1f} / "
        f"{min(kf):.1f} / {max(kf):.1f} |",
        f"| kernel WRITE_SIZE, KiB/dispatch (mean / min / max) | {statistics.mean(kw):.1f} / "
        f"{min(kw):.1f} / {max(kw):.1f} |",
        f"| kernel HBM read, bytes/launch (scaled) | {rd:.0f} |",
        f"| kernel HBM write, bytes/launch (scaled) | {wr:.0f} |",
    ]
    if a.algorithmic_bytes:
        lines.append(f"| algorithmic bytes/launch | {a.algorithmic_bytes} |")
        lines.append(f"| traffic / algorithmic | {traffic / a.algorithmic_bytes:.3f} |")
    lines += ["", f"traffic_bytes_per_launch: {traffic}"]
    Path(a.out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="what", required=True)
    k = sub.add_parser("kernels")
    k.add_argument("--dir", required=True)
    k.add_argument("--cmd", required=True)
    k.add_argument("--title", default="")
    k.add_argument("--out", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-kernel", default="copy")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--cmd-fetch", required=True)
    t.add_argument("--cmd-write", required=True)
    t.add_argument("--algorithmic-bytes", type=int, default=0)
    t.add_argument("--title", default="")
    t.add_argument("--out", required=True)
    c = sub.add_parser("counters")
    c.add_argument("--dir", required=True)
    c.add_argument("--kernel", action="append", required=True, help="name pattern (repeatable)")
    c.add_argument("--simds", type=int, default=1024, help="SIMDs of the GPU (MI355X: 256 CUs x 4)")
    c.add_argument("--xcds", type=int, default=8, help="XCDs whose busy cycles GRBM_GUI_ACTIVE sums")
    c.add_argument("--cmd", required=True)
    c.add_argument("--title", default="")
    c.add_argument("--out", required=True)
    a = ap.parse_args()
    {"kernels": report_kernels, "traffic": report_traffic, "counters": report_counters}[a.what](a)


if __name__ == "__main__":
    main()
