"""GPU parity: Mamba selective scan (HIP) vs the CPU oracle, forward and backward."""
import numpy as np
import pytest
import torch

from oracle import scans
from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host, rounded, to_dev

pytestmark = pytest.mark.gpu


def make_inputs(rng, bsz, T, D, N):
    """Config-2 distributions at a chosen shape."""
    x = rng.normal(size=(bsz, T, D))
    dt = np.log1p(np.exp(rng.normal(size=(bsz, T, D)) - 4.0))  # softplus(N(0,1) - 4)
    A = -np.exp(rng.uniform(np.log(1.0), np.log(16.0), size=(D, N)))
    B = rng.normal(size=(bsz, T, N))
    C = rng.normal(size=(bsz, T, N))
    Dv = rng.normal(size=D)
    z = rng.normal(size=(bsz, T, D))
    return x, dt, A, B, C, Dv, z


CASES = [
    # (bsz, T, D, N, io dtype, param dtype, with D/z, dt mode)
    (2, 70, 48, 16, torch.float32, torch.float32, False, "channel"),
    (2, 70, 48, 16, torch.float32, torch.float32, True, "channel"),
    (2, 96, 40, 8, torch.float32, torch.float32, True, "channel"),
    (1, 33, 20, 4, torch.float32, torch.float32, True, "channel"),
    (2, 64, 48, 16, torch.bfloat16, torch.float32, True, "channel"),
    (2, 50, 24, 16, torch.bfloat16, torch.bfloat16, False, "channel"),
    (2, 45, 32, 8, torch.float32, torch.float32, False, "mean"),
    (2, 45, 32, 16, torch.float32, torch.float32, True, "mean"),
    (1, 1, 16, 16, torch.float32, torch.float32, True, "channel"),
    # every state size up to the reference's 32, powers of two or not (padded inside)
    (2, 40, 24, 1, torch.float32, torch.float32, True, "channel"),
    (2, 40, 24, 2, torch.float32, torch.float32, False, "channel"),
    (2, 37, 24, 3, torch.float32, torch.float32, True, "channel"),
    (2, 50, 40, 12, torch.float32, torch.float32, True, "channel"),
    (1, 45, 72, 12, torch.bfloat16, torch.float32, True, "channel"),
    (2, 33, 24, 12, torch.float32, torch.float32, True, "mean"),
    (2, 41, 24, 24, torch.float32, torch.float32, True, "channel"),
    (2, 70, 48, 32, torch.float32, torch.float32, True, "channel"),
    (1, 64, 80, 32, torch.bfloat16, torch.float32, True, "channel"),
    (2, 35, 24, 32, torch.float32, torch.float32, False, "mean"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_selective_scan_fwd_bwd(case, rng):
    from edifice_amd import fused_scan as fs
    bsz, T, D, N, io, par, extras, mode = case
    announce("selective_scan", case=case)
    x, dt, A, B, C, Dv, z = make_inputs(rng, bsz, T, D, N)
    if not extras:
        Dv = z = None
    dy = rng.normal(size=x.shape)
    tx, tdt = to_dev(x, io).requires_grad_(), to_dev(dt, io).requires_grad_()
    tz = to_dev(z, io).requires_grad_() if extras else None
    tA, tB, tC = (to_dev(a, par).requires_grad_() for a in (A, B, C))
    tD = to_dev(Dv, par).requires_grad_() if extras else None
    out = fs.selective_scan(tx, tdt, tA, tB, tC, tD, tz, dt_mode=mode)
    out.backward(to_dev(dy, io))

    xr, dtr, zr, dyr = (None if a is None else rounded(a, io) for a in (x, dt, z, dy))
    Ar, Br, Cr, Dr = (None if a is None else rounded(a, par) for a in (A, B, C, Dv))
    tol = max(TOL[io], TOL[par])
    assert_close(host(out), scans.selective_scan(xr, dtr, Ar, Br, Cr, Dr, zr, mode), tol, "y")
    g = scans.selective_scan_backward(xr, dtr, Ar, Br, Cr, dyr, Dr, zr, mode)
    pairs = [("dx", tx), ("ddt", tdt), ("dA", tA), ("dB", tB), ("dC", tC)]
    if extras:
        pairs += [("dD", tD), ("dz", tz)]
    for name, t in pairs:
        assert_close(host(t.grad), g[name], tol, name)


SP_CASES = [
    (2, 45, 32, 16, torch.float32, torch.float32, True, "mean"),
    (2, 33, 24, 8, torch.float32, torch.float32, False, "mean"),
    (2, 64, 48, 16, torch.bfloat16, torch.float32, True, "mean"),   # the Mamba block's form
    (1, 40, 40, 4, torch.bfloat16, torch.bfloat16, True, "mean"),
]


@pytest.mark.parametrize("case", SP_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_selective_scan_dt_softplus(case, rng):
    """dt given before its softplus (dt_softplus=True, the EDF_SS_DT_SOFTPLUS mode flag): y and
    every gradient against the oracle run on softplus(dt_pre) in float64, dt's gradient chained
    through sigmoid(dt_pre); dt_pre = N(0, 1) - 4 puts softplus(dt_pre) on both sides of
    the clip range."""
    from edifice_amd import fused_scan as fs
    bsz, T, D, N, io, par, extras, mode = case
    announce("selective_scan_dt_softplus", case=case)
    x, _, A, B, C, Dv, z = make_inputs(rng, bsz, T, D, N)
    if not extras:
        Dv = z = None
    dtp = rng.normal(size=x.shape) - 4.0
    dy = rng.normal(size=x.shape)
    tx, tdt = to_dev(x, io).requires_grad_(), to_dev(dtp, io).requires_grad_()
    tz = to_dev(z, io).requires_grad_() if extras else None
    tA, tB, tC = (to_dev(a, par).requires_grad_() for a in (A, B, C))
    tD = to_dev(Dv, par).requires_grad_() if extras else None
    out = fs.selective_scan(tx, tdt, tA, tB, tC, tD, tz, dt_mode=mode, dt_softplus=True)
    out.backward(to_dev(dy, io))

    xr, dtpr, zr, dyr = (None if a is None else rounded(a, io) for a in (x, dtp, z, dy))
    Ar, Br, Cr, Dr = (None if a is None else rounded(a, par) for a in (A, B, C, Dv))
    dtr = np.log1p(np.exp(dtpr))
    tol = max(TOL[io], TOL[par])
    assert_close(host(out), scans.selective_scan(xr, dtr, Ar, Br, Cr, Dr, zr, mode), tol, "y")
    g = scans.selective_scan_backward(xr, dtr, Ar, Br, Cr, dyr, Dr, zr, mode)
    g["ddt"] = g["ddt"] / (1.0 + np.exp(-dtpr))
    pairs = [("dx", tx), ("ddt", tdt), ("dA", tA), ("dB", tB), ("dC", tC)]
    if extras:
        pairs += [("dD", tD), ("dz", tz)]
    for name, t in pairs:
        assert_close(host(t.grad), g[name], tol, name)


def test_selective_scan_dt_softplus_needs_mean_mode(rng):
    """The softplus flag is built for dt-mean mode: with the per-channel mode the library
    refuses it (EDF_ERR_UNSUPPORTED) rather than reading dt as already activated."""
    from edifice_amd import fused_scan as fs
    from edifice_amd._native import EdificeHipError
    announce("selective_scan_dt_softplus_channel")
    x, dt, A, B, C, Dv, z = make_inputs(rng, 1, 8, 16, 4)
    args = [to_dev(a, torch.float32) for a in (x, dt, A, B, C, Dv, z)]
    with pytest.raises(EdificeHipError, match="dt-mean mode"):
        fs.selective_scan(*args, dt_mode="channel", dt_softplus=True)


def test_selective_scan_config2_full_size_properties(rng):
    """C2 shape (B=8, T=2048, D=1536, N=16, bf16 u/dt/z, f32 A/B/C/D): B == 0 gives
    y == D x silu(z) exactly (size-independent closed form), and one batch row agrees
    with the oracle over the whole sequence."""
    from edifice_amd import fused_scan as fs
    bsz, T, D, N = 8, 2048, 1536, 16
    announce("selective_scan_c2_full")
    x, dt, A, B, C, Dv, z = make_inputs(rng, bsz, T, D, N)
    tx, tdt, tz = (to_dev(a, torch.bfloat16) for a in (x, dt, z))
    tA, tB, tC, tD = (to_dev(a, torch.float32) for a in (A, B, C, Dv))
    y0 = fs.selective_scan(tx, tdt, tA, torch.zeros_like(tB), tC, tD, tz)
    xr, zr = rounded(x, torch.bfloat16), rounded(z, torch.bfloat16)
    expect = Dv * xr * zr / (1 + np.exp(-zr))
    assert_close(host(y0), expect, TOL[torch.bfloat16], "B=0 closed form")
    y = fs.selective_scan(tx, tdt, tA, tB, tC, tD, tz)
    b = 3
    ref = scans.selective_scan(xr[b:b + 1, :, :256], rounded(dt, torch.bfloat16)[b:b + 1, :, :256], A[:256],
                               B[b:b + 1], C[b:b + 1], Dv[:256], zr[b:b + 1, :, :256])
    assert_close(host(y)[b:b + 1, :, :256], ref, TOL[torch.bfloat16], "row 3 vs oracle")


# Every compiled (state size, channel groups) instantiation, forced through EDF_SS_PLAN: the
# wide plan (G = 4 at N = 4 and 8, G = 3 at N = 16) and the narrow one (G = 1), forward and
# backward, in both dt modes.  D = 100 spans several tiles of either plan with a ragged last
# one; T = 70 ends off the 16-step checkpoint interval.
PLAN_CASES = [
    (n, plan, mode, io)
    for n, io in ((3, torch.float32), (8, torch.float32), (16, torch.bfloat16), (16, torch.float32))
    for plan in ("narrow", "wide")
    for mode in ("channel", "mean")
]


@pytest.mark.parametrize("case", PLAN_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_selective_scan_each_plan(case, rng, monkeypatch):
    from edifice_amd import fused_scan as fs
    n, plan, mode, io = case
    monkeypatch.setenv("EDF_SS_PLAN", plan)
    announce("selective_scan_plan", n=n, plan=plan, mode=mode, io=io)
    bsz, T, D = 2, 70, 100
    x, dt, A, B, C, Dv, z = make_inputs(rng, bsz, T, D, n)
    dy = rng.normal(size=x.shape)
    par = torch.float32
    tx, tdt, tz = (to_dev(a, io).requires_grad_() for a in (x, dt, z))
    tA, tB, tC, tD = (to_dev(a, par).requires_grad_() for a in (A, B, C, Dv))
    out = fs.selective_scan(tx, tdt, tA, tB, tC, tD, tz, dt_mode=mode)
    out.backward(to_dev(dy, io))
    xr, dtr, zr, dyr = (rounded(a, io) for a in (x, dt, z, dy))
    tol = TOL[io]
    assert_close(host(out), scans.selective_scan(xr, dtr, A, B, C, Dv, zr, mode), tol, "y")
    g = scans.selective_scan_backward(xr, dtr, A, B, C, dyr, Dv, zr, mode)
    for name, t in (("dx", tx), ("ddt", tdt), ("dA", tA), ("dB", tB), ("dC", tC), ("dD", tD), ("dz", tz)):
        assert_close(host(t.grad), g[name], tol, name)


def test_selective_scan_plans_agree_without_gate(rng, monkeypatch):
    """No D, no gate: both plans give the oracle's result (the kernels' Z = false instances)."""
    from edifice_amd import fused_scan as fs
    x, dt, A, B, C, _, _ = make_inputs(rng, 2, 45, 72, 16)
    dy = rng.normal(size=x.shape)
    g = scans.selective_scan_backward(x, dt, A, B, C, dy)
    for plan in ("narrow", "wide"):
        monkeypatch.setenv("EDF_SS_PLAN", plan)
        announce("selective_scan_plan_nogate", plan=plan)
        tx, tdt, tA, tB, tC = (to_dev(a, torch.float32).requires_grad_() for a in (x, dt, A, B, C))
        out = fs.selective_scan(tx, tdt, tA, tB, tC)
        out.backward(to_dev(dy, torch.float32))
        assert_close(host(out), scans.selective_scan(x, dt, A, B, C), TOL[torch.float32], f"y {plan}")
        for name, t in (("dx", tx), ("ddt", tdt), ("dA", tA), ("dB", tB), ("dC", tC)):
            assert_close(host(t.grad), g[name], TOL[torch.float32], f"{name} {plan}")


def test_selective_scan_config5_width(rng, monkeypatch):
    """The hybrid decoder's Mamba shape (config 5: B = 8, d_inner = 2048, N = 16, bf16 x, dt, z;
    f32 A, B, C, D; dt-mean mode with the gate), at a short sequence.  The host's own choice
    there is the narrow plan (G = 1: 1024 even workgroups against the wide plan's 344), which
    the backward workspace size shows.  Row 5 is checked against the oracle over every
    channel (its dt mean couples them all): y, dx, ddt, dz, dB, dC; dA and dD over channels
    0-255, which x = 0 leaves to row 5 alone in the batch sums."""
    from edifice_amd import fused_scan as fs
    from edifice_amd import _native as nat
    bsz, T, D, N, b0, W = 8, 136, 2048, 16, 5, 256
    monkeypatch.delenv("EDF_SS_PLAN", raising=False)
    auto = nat.query("edf_selective_scan_backward_workspace_bytes", bsz, T, D, N, 1, 1)
    monkeypatch.setenv("EDF_SS_PLAN", "narrow")
    narrow = nat.query("edf_selective_scan_backward_workspace_bytes", bsz, T, D, N, 1, 1)
    monkeypatch.setenv("EDF_SS_PLAN", "wide")
    wide = nat.query("edf_selective_scan_backward_workspace_bytes", bsz, T, D, N, 1, 1)
    monkeypatch.delenv("EDF_SS_PLAN")
    assert auto == narrow != wide, (auto, narrow, wide)
    announce("selective_scan_c5_width", B=bsz, T=T, D=D, N=N)
    x, dt, A, B, C, Dv, z = make_inputs(rng, bsz, T, D, N)
    x[np.arange(bsz) != b0, :, :W] = 0.0
    dy = rng.normal(size=x.shape)
    tx, tdt, tz = (to_dev(a, torch.bfloat16).requires_grad_() for a in (x, dt, z))
    tA, tB, tC, tD = (to_dev(a, torch.float32).requires_grad_() for a in (A, B, C, Dv))
    y = fs.selective_scan(tx, tdt, tA, tB, tC, tD, tz, dt_mode="mean")
    y.backward(to_dev(dy, torch.bfloat16))
    torch.cuda.synchronize()
    r = slice(b0, b0 + 1)
    xr, dtr, zr, dyr = (rounded(a, torch.bfloat16)[r] for a in (x, dt, z, dy))
    tol = TOL[torch.bfloat16]
    assert_close(host(y)[r], scans.selective_scan(xr, dtr, A, B[r], C[r], Dv, zr, "mean"), tol, "y row 5")
    g = scans.selective_scan_backward(xr, dtr, A, B[r], C[r], dyr, Dv, zr, "mean")
    for name, t in (("dx", tx), ("ddt", tdt), ("dz", tz)):
        assert_close(host(t.grad)[r], g[name], tol, f"{name} row 5")
    assert_close(host(tB.grad)[r], g["dB"], tol, "dB row 5")
    assert_close(host(tC.grad)[r], g["dC"], tol, "dC row 5")
    # dA / dD: rows other than 5 hold x = 0 on channels 0-255, so only row 5 feeds those sums
    assert_close(host(tA.grad)[:W], g["dA"][:W], tol, "dA channels 0-255")
    assert_close(host(tD.grad)[:W], g["dD"][:W], tol, "dD channels 0-255")
