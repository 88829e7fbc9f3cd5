import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through librsllm_hip.so)")


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max|got - want| / max|want| — the parity metric for float outputs."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = np.abs(want).max() if want.size else 0.0
    if denom == 0.0:
        return float(np.abs(got - want).max()) if got.size else 0.0
    return float(np.abs(got - want).max() / denom)


# Output tolerance stated by the north star: max|Δ|/max|y| <= 1e-3 with fp32
# accumulation.
REL_TOL = 1e-3


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def hip():
    from rsllm_amd import backend as B
    return B
