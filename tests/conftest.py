import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "jdm-ghassan_v1_flach_amd"))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")
    config.addinivalue_line("markers", "slow: CPU test of tens of seconds")


@pytest.fixture(scope="session")
def gh():
    import ghassan_hip
    ghassan_hip.load(init_device=True)
    return ghassan_hip


def golden(name):
    import numpy as np
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


_STATS = []


def elemerr(a, b, floor=0.1):
    """Elementwise relative error max |a-b|/|b| over the entries with
    |b| >= floor * max|b| (small entries are left to the normwise metric)."""
    import numpy as np
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    m = np.max(np.abs(b)) if b.size else 0.0
    if m == 0:
        return float(np.max(np.abs(a - b))) if a.size else 0.0
    sel = np.abs(b) >= floor * m
    return float(np.max(np.abs(a[sel] - b[sel]) / np.abs(b[sel])))


def relerr(a, b):
    """Normwise relative error max|a-b| / max|b| (the parity metric used for
    floating-point outputs)."""
    import numpy as np
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.max(np.abs(b))
    r = float(np.max(np.abs(a - b)) / (den if den > 0 else 1.0))
    if os.environ.get("GH_ERR_LOG"):
        _STATS.append((os.environ.get("PYTEST_CURRENT_TEST", "?"), r, elemerr(a, b, 0.1), elemerr(a, b, 0.01)))
    return r


def close(a, b, tol):
    """The parity check for floating-point outputs: normwise relative error
    <= tol AND elementwise relative error <= elem_tol(tol) on the entries with
    |b| >= 10 % of max|b|. The elementwise bound is looser than tol because
    the reference's CPU path rounds every dequantised weight to fp16
    (core/ops.cpp:304-338) while the GPU multiplies the exact codes:
    tests/test_gpu_exact.py measures the GPU within 2e-4 elementwise of the
    float64 product over the exact weights and the oracle further away than
    that, and chained layers (a model step's logits) add such differences up to
    about 5.6e-3 elementwise at the 1e-3 normwise level."""
    n = relerr(a, b)
    e = elemerr(a, b, 0.1)
    assert n <= tol, f"normwise rel-err {n:.3g} > {tol:g}"
    assert e <= elem_tol(tol), f"elementwise rel-err {e:.3g} > {elem_tol(tol):g} (entries >= 10% of max)"
    return True


def elem_tol(tol):
    return 7.5 * tol if tol <= 1e-3 else 3 * tol


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("GH_ERR_LOG")
    if path and _STATS:
        import json
        with open(path, "w") as f:
            for t, r, e1, e2 in _STATS:
                f.write(json.dumps({"test": t, "norm": r, "elem10": e1, "elem1": e2}) + "\n")
