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


@pytest.mark.parametrize("gated,per_head", [(False, False), (True, True), (True, False)])
def test_cref_delta_rule(cref, rng, gated, per_head):
    """Forward and the checkpointed reverse pass (T spans three 64-step chunks, the last one
    ragged) against the numpy oracle."""
    B, T, H, d = 2, 150, 2, 12
    f32 = np.float32
    q, v, do = (rng.normal(size=(B, T, H, d)).astype(f32) for _ in range(3))
    k = scans.l2_normalize_keys(rng.normal(size=(B, T, H, d))).astype(f32)
    beta = rng.uniform(0.1, 0.9, size=(B, T, H) if per_head else (B, T, H, d)).astype(f32)
    alpha = rng.uniform(0.8, 1.0, size=(B, T, H)).astype(f32) if gated else None
    nul = ctypes.c_void_p(None)
    out = np.empty_like(q)
    cref.cref_delta_rule_fwd(P(q), P(k), P(v), P(beta), P(alpha) if gated else nul, P(out), B, T, H, d,
                             int(per_head))
    assert_close(out, scans.delta_rule(q, k, v, beta, alpha), 1e-4, "o")
    dq, dk, dv = (np.empty_like(q) for _ in range(3))
    dbeta = np.empty_like(beta)
    dalpha = np.empty((B, T, H), f32)
    cref.cref_delta_rule_bwd(P(q), P(k), P(v), P(beta), P(alpha) if gated else nul, P(do), P(dq), P(dk), P(dv),
                             P(dbeta), P(dalpha) if gated else nul, B, T, H, d, int(per_head))
    g = scans.delta_rule_backward(q, k, v, beta, do, alpha)
    pairs = [("dq", dq), ("dk", dk), ("dv", dv), ("dbeta", dbeta)] + ([("dalpha", dalpha)] if gated else [])
    for n, a in pairs:
        assert_close(a, g[n], 1e-4, n)


@pytest.mark.parametrize("causal", [True, False])
def test_cref_attention(cref, rng, causal):
    BH, T, d = 3, 45, 16
    f32 = np.float32
    q, k, v, do = (rng.normal(size=(1, BH, T, d)).astype(f32) for _ in range(4))
    out, dq, dk, dv = (np.empty_like(q) for _ in range(4))
    lse = np.empty((BH, T), f32)
    cref.cref_attention_fwd(P(q), P(k), P(v), P(out), P(lse), BH, T, d, int(causal))
    eo, el = scans.flash_attention(q, k, v, causal=causal, return_lse=True)
    assert_close(out, eo, 1e-5, "o")
    assert_close(lse, el[0], 1e-5, "lse")
    cref.cref_attention_bwd(P(q), P(k), P(v), P(out), P(do), P(lse), P(dq), P(dk), P(dv), BH, T, d, int(causal))
    for n, a, e in zip(("dq", "dk", "dv"), (dq, dk, dv), scans.flash_attention_backward(q, k, v, do, causal=causal)):
        assert_close(a, e, 1e-4, n)
