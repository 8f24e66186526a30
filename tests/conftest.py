import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def rel_err(actual, expected):
    """max |a - e| / max |e|: the error criterion used by every parity test.

    The reference's own tests use a max-abs criterion (backward_kernels_test.exs:1427-1432);
    normalising by max |e| turns the north-star tolerances (1e-4 f32, 2e-2 bf16)
    into a scale-free bound.
    """
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    if e.size == 0:
        return 0.0
    scale = max(np.abs(e).max(), 1e-30)
    return float(np.abs(a - e).max() / scale)


def assert_close(actual, expected, tol, what=""):
    err = rel_err(actual, expected)
    assert np.isfinite(err) and err <= tol, f"{what}: rel err {err:.3e} > {tol:.1e}"


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
