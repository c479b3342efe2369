"""Shared pytest set-up.

Marker `gpu`: tests that need an MI355X (they call libnmoe_hip.so's kernels
through the C ABI).  Everything else runs on the CPU.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "nano-metal-moe-qwen36_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# max-abs / relative-L2 bounds for floating-point outputs (the path's stated tolerance)
MAX_ABS = 2e-3
REL_L2 = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (runs the HIP kernels)")
    # the CPU oracle is test infrastructure; build it if this checkout has not
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def assert_close(got, want, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    import numpy as np
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    mx = float(err.max()) if err.size else 0.0
    denom = float(np.linalg.norm(want)) or 1.0
    rl2 = float(np.linalg.norm(got - want)) / denom
    assert mx <= max_abs and rl2 <= rel_l2, f"{what}: max-abs {mx:.3g} (<= {max_abs}), rel-L2 {rl2:.3g} (<= {rel_l2})"
    return mx, rl2


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", "math_ref_golden.npz"))
