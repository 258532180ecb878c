import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def rel_l2(actual, expected):
    actual = np.asarray(actual, np.float64).ravel()
    expected = np.asarray(expected, np.float64).ravel()
    denom = np.linalg.norm(expected)
    return float(np.linalg.norm(actual - expected) / (denom if denom > 0 else 1.0))


@pytest.fixture(scope="session")
def device():
    """Initialises the HIP library once per session (GPU tests only)."""
    from floyd_amd import native
    name = native.init()
    print(f"[gpu] device: {name}", flush=True)
    return name
