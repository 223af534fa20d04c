"""Shared test set-up.

Markers: `gpu` — needs an MI355X (HIP device 0); everything else runs on the
CPU.  Every parity test compares against the CPU oracle (oracle/).
"""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "diffuse-cpp_amd"))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X, gfx950)")


@pytest.fixture(scope="session")
def O():
    import oracle
    oracle.build()
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    import dmoe
    c = dmoe.Context(0)
    yield c
    c.close()


def max_rel_err(y, ref):
    """max |y - ref| / max |ref|: the layer-output tolerance measure."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))
