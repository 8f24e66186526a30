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
    """max |a - e| / max |e|: the scale-free max-abs error.

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


# Element-wise floor of assert_close, as a fraction of max |e|: entries at least this large
# are held to (about) the tolerance relative to themselves.  At the float32 tolerance 1%; at
# the bf16 tolerance 5% (the scans, convolution and cross entropy compute in float32 and round
# only their inputs and outputs).  Kernels that round MFMA operands to bf16 (attention's P and
# dS, the chunked delta rule's states and chunk products) take mfma_bf16=True and a floor of
# 25%: an output that sums many such terms carries an error of order 2^-9 of the largest
# terms, whatever its own size, so near-zero outputs are held to 2e-2 * 0.25 = 5e-3 of the
# largest entry, about one bf16 ulp.  (Measured on the GPU suite: every bf16 scan test holds at
# a 5% floor; the MFMA-operand tests need about 20%.)
ELEM_FLOOR = 1e-2
ELEM_FLOOR_BF16 = 0.05
ELEM_FLOOR_MFMA_BF16 = 0.25


def elem_rel_err(actual, expected, floor=ELEM_FLOOR):
    """max over elements of |a - e| / (|e| + floor * max |e|): a relative error per element.

    The north star states rtol; a pure rtol is undefined at entries that are zero or that
    cancel, so each entry's own magnitude is floored at `floor` of the tensor's largest.
    Gradients whose entries span orders of magnitude (dA, dalpha, dbeta, dB) are then
    checked entry by entry, not only against their largest entry.
    """
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    if e.size == 0:
        return 0.0
    den = np.abs(e) + floor * max(np.abs(e).max(), 1e-30)
    return float((np.abs(a - e) / den).max())


def assert_close(actual, expected, tol, what="", elementwise=True, elem_tol=None, mfma_bf16=False):
    """Both criteria at the same tolerance: max |a - e| / max |e| <= tol and, element by
    element, |a - e| <= tol (|e| + floor max |e|), floor ELEM_FLOOR (float32 tolerances),
    ELEM_FLOOR_BF16, or ELEM_FLOOR_MFMA_BF16 for bf16 outputs of kernels that round MFMA
    operands to bf16 (mfma_bf16=True).

    elementwise=False keeps only the first, for whole bf16 models compared with float32
    references: there every weight and activation of the block is rounded to bf16 (a
    relative 2^-9 per rounding, many roundings deep), so outputs near zero cannot hold a
    per-element 2e-2; the fused ops inside those models are checked element-wise in their
    own tests.  elem_tol overrides the element-wise tolerance where a test says why."""
    err = rel_err(actual, expected)
    assert np.isfinite(err) and err <= tol, f"{what}: rel err {err:.3e} > {tol:.1e}"
    if elementwise:
        etol = tol if elem_tol is None else elem_tol
        floor = ELEM_FLOOR if tol < 1e-3 else (ELEM_FLOOR_MFMA_BF16 if mfma_bf16 else ELEM_FLOOR_BF16)
        eerr = elem_rel_err(actual, expected, floor)
        assert np.isfinite(eerr) and eerr <= etol, f"{what}: element-wise rel err {eerr:.3e} > {etol:.1e}"


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
