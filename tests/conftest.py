import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libpssa_hip.so")


def rel_err(actual, expected) -> float:
    """max |actual - expected| / max |expected|: the normwise relative error
    the parity gates are stated in (1e-4 fp32, 2e-2 bf16 weights)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.all(np.isfinite(a)), "non-finite output"
    scale = max(float(np.max(np.abs(e))) if e.size else 0.0, 1e-30)
    return float(np.max(np.abs(a - e))) / scale if e.size else 0.0


@pytest.fixture(scope="session")
def hip():
    """The GPU context, shared by every GPU test of the session."""
    from pssa_amd import HipDevice

    dev = HipDevice(0)
    yield dev
    dev.close()
