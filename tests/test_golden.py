"""CPU: the oracle reproduces the committed golden fixtures bit for bit
(self-pinned vectors written by tests/golden/make_golden.py)."""
import sys
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(HERE))

import make_golden  # noqa: E402


@pytest.mark.parametrize("case", sorted(make_golden.CASES))
def test_golden_fixture(O, case):
    ref = np.load(HERE / f"{case}.npz", allow_pickle=False)
    got = make_golden.compute(case)
    assert str(ref["inputs_sha256"]) == got["inputs_sha256"], "synthetic inputs changed"
    for k in ("logits", "probs", "bmax", "thr", "allowed", "idx", "weights", "counts", "offsets",
              "perm", "y"):
        assert np.array_equal(np.asarray(ref[k]).view(np.uint8), np.asarray(got[k]).view(np.uint8)), k
