"""Build libdmoe.so (the HIP product library) in-tree for gfx950.

    python diffuse-cpp_amd/build.py            # incremental
    python diffuse-cpp_amd/build.py --force    # rebuild everything

Every HIP source is compiled by hipcc with
``-Xclang -target-feature -Xclang -packed-fp32-ops`` (no packed FP32 ops are
emitted), objects go to ``diffuse-cpp_amd/_build/`` and the shared library to
``diffuse-cpp_amd/libdmoe.so``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB = PKG / "libdmoe.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]

SOURCES = ["k_router.hip", "k_quant.hip", "k_gemv.hip", "k_prep.hip", "k_expert.hip", "k_expert_tile.hip", "k_expert_gemm.hip", "k_down_span.hip", "k_expert_q80.hip",
           "k_gemm.hip", "k_norm.hip", "k_down_rows.hip", "k_head.hip", "k_attn.hip", "k_proj.hip",
           "dmoe_api.cpp", "dmoe_gguf.cpp"]
HEADERS = ["dmoe_internal.h", "dmoe_device.h", "dmoe_prep.h", "dmoe_q4k.h"]


def _needs(obj: Path, deps: list[Path]) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _compile(src: Path, force: bool) -> Path:
    obj = OUT_DIR / (src.name + ".o")
    deps = [src] + [CSRC / h for h in HEADERS] + [ROOT / "include" / "dmoe.h"]
    if force or _needs(obj, deps):
        lang = ["-x", "hip"] if src.suffix in (".hip", ".cpp") else []
        cmd = [HIPCC, *CFLAGS, *lang, "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
        noise = "is not a recognized feature for this target"
        msgs = [l for l in (r.stderr or "").splitlines() if noise not in l and l.strip()]
        if msgs:
            sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(force: bool = False, jobs: int = 8) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    if force or _needs(LIB, objs):
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=8)
    a = ap.parse_args()
    print(build(force=a.force, jobs=a.jobs))
