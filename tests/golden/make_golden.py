"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

These vectors are self-pinned: the reference has no golden vectors for this
path (its ggml submodule is absent and its tests never exercise the router),
so the fixtures freeze the oracle's output on fixed synthetic inputs — any
later change to the oracle, the block codecs or the input generators shows up
as a mismatch in tests/test_golden.py.

    python tests/golden/make_golden.py
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "diffuse-cpp_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

CASES = {
    # name: (config builder, seed, n_tokens)
    "tiny_seed7": ("tiny", 7, 32),
    "small_q4k_seed8": ("small_q4k", 8, 64),
    "small_q8_0_seed9": ("small_q8_0", 9, 64),
}


def config(name):
    from dmoe import synth
    if name == "tiny":
        return synth.CONFIGS["tiny"]
    t = {"small_q4k": 12, "small_q8_0": 8}[name]
    return synth.LayerConfig(name, 512, 16, 256, 6, 4, 32, 256, t, t, 64, -0.05, 0.05)


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def compute(case):
    import oracle as O
    from dmoe import synth
    cname, seed, n = CASES[case]
    cfg = config(cname)
    w = synth.host_layer(cfg, seed, O.quantize_rows)
    x = synth.make_x(cfg, seed, n)
    y, d = O.layer_forward(w, x, debug=True, n_threads=1)
    return {
        "inputs_sha256": digest(x, w.gate_w, w.gate_bias, w.exp_gate, w.exp_up, w.exp_down,
                                w.sh_gate, w.sh_up, w.sh_down),
        "logits": d["logits"], "probs": d["probs"], "bmax": d["bmax"], "thr": d["thr"],
        "allowed": d["allowed"], "idx": d["idx"], "weights": d["weights"],
        "counts": d["counts"], "offsets": d["offsets"], "perm": d["perm"], "y": y,
    }


if __name__ == "__main__":
    for case in CASES:
        out = compute(case)
        np.savez_compressed(HERE / f"{case}.npz", **out)
        print(case, out["inputs_sha256"][:16], "y max", float(np.abs(out["y"]).max()))
