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


def elem_rel_err(actual, expected, floor=None) -> float:
    """max over elements of |actual - expected| / max(|expected|, floor): the
    element-wise relative error, with an absolute floor for elements near
    zero.  The floor defaults to the root mean square of `expected` (a
    typical element's magnitude), so elements above it are held to a true
    relative bound and the smaller ones to tol * rms absolute."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.all(np.isfinite(a)), "non-finite output"
    if not e.size:
        return 0.0
    if floor is None:
        floor = float(np.sqrt(np.mean(e * e)))
    return float(np.max(np.abs(a - e) / np.maximum(np.abs(e), max(floor, 1e-30))))


def assert_parity(actual, expected, tol, what="", floor=None):
    """The parity gate: normwise (max |d| / max |expected|) and element-wise
    relative errors both below `tol`.  The element-wise floor (elem_rel_err)
    is the RMS of `expected` at the fp32 gates (tol < 1e-2) and four times
    it at the bf16 gates: rounding a product's operands to bf16 moves each
    element by a fraction of the terms that formed it, which is the typical
    element's size rather than its own, and the bf16 gate (2e-2) leaves about
    ten units of bf16 roundoff where the fp32 gate leaves some 1700 of fp32's."""
    if floor is None:
        e = np.asarray(expected, dtype=np.float64)
        floor = (4.0 if tol >= 1e-2 else 1.0) * float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    nw = rel_err(actual, expected)
    ew = elem_rel_err(actual, expected, floor)
    # At the bf16 gate the error at the one-RMS floor is reported beside the
    # gated one (it is not gated).
    ew1 = f", element-wise at the RMS floor {elem_rel_err(actual, expected):.3e}" if tol >= 1e-2 else ""
    assert nw < tol and ew < tol, f"{what}: normwise {nw:.3e}, element-wise {ew:.3e}, tolerance {tol:g}{ew1}"
    print(f"[parity] {what}: normwise {nw:.3e}, element-wise {ew:.3e}, tolerance {tol:g}{ew1}", flush=True)
    return nw, ew


@pytest.fixture(scope="session")
def hip():
    """The GPU context, shared by every GPU test of the session."""
    from pssa_amd import HipDevice

    dev = HipDevice(0)
    yield dev
    dev.close()
