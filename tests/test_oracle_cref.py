"""Pin the C restatement (oracle/cref.c, the timed CPU baseline) against the numpy oracle."""
import ctypes

import numpy as np
import pytest

from oracle import cbuild, scans
from tests.conftest import assert_close


@pytest.fixture(scope="module")
def cref():
    return cbuild.lib()


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def test_cref_mingru(cref, rng):
    B, T, H = 2, 37, 19
    z = rng.uniform(0.05, 0.95, size=(B, T, H)).astype(np.float32)
    c, dy = (rng.normal(size=(B, T, H)).astype(np.float32) for _ in range(2))
    h0 = rng.normal(size=(B, H)).astype(np.float32)
    out = np.empty_like(z)
    cref.cref_mingru_fwd(P(z), P(c), P(h0), P(out), B, T, H)
    assert_close(out, scans.mingru_scan(z, c, h0), 1e-5, "h")
    dz, dc, dh0 = np.empty_like(z), np.empty_like(z), np.empty_like(h0)
    cref.cref_mingru_bwd(P(z), P(c), P(h0), P(out), P(dy), P(dz), P(dc), P(dh0), B, T, H)
    ez, ec, eh = scans.mingru_scan_backward(z, c, h0, out, dy)
    for a, e, n in ((dz, ez, "dz"), (dc, ec, "dc"), (dh0, eh, "dh0")):
        assert_close(a, e, 1e-5, n)


@pytest.mark.parametrize("extras", [False, True])
def test_cref_selective_scan(cref, rng, extras):
    B, T, D, N = 2, 29, 11, 8
    f32 = np.float32
    x = rng.normal(size=(B, T, D)).astype(f32)
    dt = rng.uniform(0, 0.15, size=(B, T, D)).astype(f32)
    A = (-np.exp(rng.uniform(0, 2.7, size=(D, N)))).astype(f32)
    Bm, Cm = (rng.normal(size=(B, T, N)).astype(f32) for _ in range(2))
    Dv = rng.normal(size=D).astype(f32) if extras else None
    z = rng.normal(size=(B, T, D)).astype(f32) if extras else None
    dy = rng.normal(size=(B, T, D)).astype(f32)
    out = np.empty_like(x)
    nul = ctypes.c_void_p(None)
    cref.cref_selective_scan_fwd(P(x), P(dt), P(A), P(Bm), P(Cm), P(Dv) if extras else nul,
                                 P(z) if extras else nul, P(out), B, T, D, N)
    assert_close(out, scans.selective_scan(x, dt, A, Bm, Cm, Dv, z), 1e-5, "y")
    dx, ddt, dz = np.empty_like(x), np.empty_like(x), np.empty_like(x)
    dA, dB, dC = np.zeros_like(A), np.zeros_like(Bm), np.zeros_like(Cm)
    dD = np.zeros(D, f32)
    cref.cref_selective_scan_bwd(P(x), P(dt), P(A), P(Bm), P(Cm), P(Dv) if extras else nul,
                                 P(z) if extras else nul, P(dy), P(dx), P(ddt), P(dA), P(dB), P(dC),
                                 P(dD) if extras else nul, P(dz) if extras else nul, B, T, D, N)
    g = scans.selective_scan_backward(x, dt, A, Bm, Cm, dy, Dv, z)
    pairs = [("dx", dx), ("ddt", ddt), ("dA", dA), ("dB", dB), ("dC", dC)]
    if extras:
        pairs += [("dD", dD), ("dz", dz)]
    for n, a in pairs:
        assert_close(a, g[n], 1e-4, n)
