"""GPU parity: delta rule (DeltaNet / GatedDeltaNet), forward and backward, vs the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import scans
from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host, rounded, to_dev

pytestmark = pytest.mark.gpu


def make_inputs(rng, B, T, H, d, per_head_beta, gated):
    """Config-3 distributions at a chosen shape."""
    q = scans.l2_normalize_keys(rng.normal(size=(B, T, H, d)))
    k = scans.l2_normalize_keys(rng.normal(size=(B, T, H, d)))
    v = rng.normal(size=(B, T, H, d))
    bshape = (B, T, H) if per_head_beta else (B, T, H, d)
    beta = 1 / (1 + np.exp(-rng.normal(size=bshape)))
    alpha = np.exp(-np.log1p(np.exp(rng.normal(size=(B, T, H))))) if gated else None
    return q, k, v, beta, alpha


def chunked_path(B, T, H, d, dtype, per_head_beta):
    """Whether the library runs this shape on the chunked MFMA path (it reports a chunked
    workspace only then)."""
    from edifice_amd import _native as nat
    dt = 1 if dtype == torch.bfloat16 else 0
    return nat.query("edf_delta_rule_workspace_bytes", B, T, H, d, dt, 1 if per_head_beta else 0) > 0


CASES = [
    # (B, T, H, d, dtype, per_head_beta, gated)
    (2, 9, 2, 4, torch.float32, False, False),     # reference test sizes (head_dim 4)
    (2, 33, 3, 16, torch.float32, False, True),
    (1, 40, 2, 32, torch.float32, True, True),
    (1, 50, 2, 64, torch.float32, False, False),
    (1, 37, 1, 128, torch.float32, True, False),
    (1, 48, 2, 128, torch.float32, False, True),
    (2, 20, 2, 32, torch.bfloat16, False, True),
    # chunked MFMA forward and backward (bf16, per-head beta, d=128, T >= 64)
    (1, 64, 2, 128, torch.bfloat16, True, True),
    (1, 200, 2, 128, torch.bfloat16, True, True),    # partial last chunk
    (2, 130, 1, 128, torch.bfloat16, True, False),
    (1, 640, 2, 128, torch.bfloat16, True, True),    # ten chunks: state and gradient carried across
    # head_dim 64 and 96 on the chunked path (zero-padded to 128 inside the kernels)
    (1, 200, 2, 64, torch.bfloat16, True, True),
    (2, 130, 1, 64, torch.bfloat16, True, False),
    (1, 192, 2, 96, torch.bfloat16, True, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_delta_rule_fwd_bwd(case, rng):
    from edifice_amd import fused_scan as fs
    B, T, H, d, dtype, phb, gated = case
    announce("delta_rule", case=case)
    q, k, v, beta, alpha = make_inputs(rng, B, T, H, d, phb, gated)
    do = rng.normal(size=v.shape)
    tq, tk, tv, tb = (to_dev(a, dtype).requires_grad_() for a in (q, k, v, beta))
    ta = to_dev(alpha, dtype).requires_grad_() if gated else None
    out = fs.gated_delta_net_scan(tq, tk, tv, tb, ta) if gated else fs.delta_net_scan(tq, tk, tv, tb)
    out.backward(to_dev(do, dtype))
    qr, kr, vr, br, dor = (rounded(a, dtype) for a in (q, k, v, beta, do))
    ar = rounded(alpha, dtype) if gated else None
    tol = TOL[dtype]
    mf = chunked_path(B, T, H, d, dtype, phb)  # the chunked path rounds its MFMA operands to bf16
    assert_close(host(out), scans.delta_rule(qr, kr, vr, br, ar), tol, "o", mfma_bf16=mf)
    g = scans.delta_rule_backward(qr, kr, vr, br, dor, ar)
    pairs = [("dq", tq), ("dk", tk), ("dv", tv), ("dbeta", tb)] + ([("dalpha", ta)] if gated else [])
    for name, t in pairs:
        assert_close(host(t.grad), g[name], tol, name, mfma_bf16=mf)


@pytest.mark.parametrize("case", [(1, 200, 2, 128, torch.bfloat16, True, True),
                                  (2, 130, 1, 128, torch.bfloat16, False, True),
                                  (1, 200, 2, 64, torch.bfloat16, True, True), (1, 40, 2, 32, torch.float32, True, True),
                                  (1, 70, 2, 128, torch.bfloat16, False, False),  # per-element beta (config 5)
                                  (2, 45, 1, 40, torch.float32, True, False)],
                         ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_delta_rule_backward_entry_points_agree(case, rng):
    """The reference-shaped backward entry points (which recompute the forward context) and
    edf_fused_delta_rule_scan_backward_saved (which reads the forward's workspace) give the
    same gradients: chunked path (gated and not) and the per-step path, whose forward workspace
    of edf_delta_rule_forward_context_bytes() keeps the 16-step states the saved backward
    reads instead of recomputing them.  Same kernels on the same inputs, and every kernel
    sums in a fixed order (the chunked gradient kernel adds the dbeta and decay terms of a
    chunk per wave, then over the waves in order), so the two agree bit for bit."""
    import ctypes

    from edifice_amd import _native as nat
    B, T, H, d, dtype, gated, per_head = case
    announce("delta_rule_entry_points", case=case)
    q, k, v, beta, alpha = make_inputs(rng, B, T, H, d, per_head, gated)
    mode = 1 if per_head else 0
    do = rng.normal(size=v.shape)
    tq, tk, tv, tb, tdo = (to_dev(a, dtype) for a in (q, k, v, beta, do))
    ta = to_dev(alpha, dtype) if gated else None
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dt = 1 if dtype == torch.bfloat16 else 0
    wsf = nat.query("edf_delta_rule_forward_context_bytes", B, T, H, d, dt, mode)
    wsr = nat.query("edf_delta_rule_backward_workspace_bytes", B, T, H, d, dt, mode)
    wss = nat.query("edf_delta_rule_saved_backward_workspace_bytes", B, T, H, d, dt, mode)
    chunked = nat.query("edf_delta_rule_workspace_bytes", B, T, H, d, dt, mode) > 0
    f_ws = torch.empty(max(wsf, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(tv)
    if gated:
        nat.call("edf_fused_gated_delta_net_scan", st, P(tq), P(tk), P(tv), P(tb), P(ta), P(out), P(f_ws), wsf,
                 B, T, H, d, dt, mode)
    else:
        nat.call("edf_fused_delta_net_scan", st, P(tq), P(tk), P(tv), P(tb), P(out), P(f_ws), wsf, B, T, H, d, dt,
                 mode)
    grads = []
    for saved in (False, True):
        g = [torch.empty_like(t) for t in (tq, tk, tv, tb)] + ([torch.empty_like(ta)] if gated else [None])
        if saved:
            ws = torch.empty(max(wss, 1), dtype=torch.uint8, device="cuda")
            nat.call("edf_fused_delta_rule_scan_backward_saved", st, P(tq), P(tk), P(tv), P(tb), P(ta), P(tdo),
                     *(P(x) for x in g), P(f_ws), wsf, P(ws), wss, B, T, H, d, dt, mode)
        elif gated:
            ws = torch.empty(max(wsr, 1), dtype=torch.uint8, device="cuda")
            nat.call("edf_fused_gated_delta_net_scan_backward", st, P(tq), P(tk), P(tv), P(tb), P(ta), P(out),
                     P(tdo), *(P(x) for x in g), P(ws), wsr, B, T, H, d, dt, mode)
        else:
            ws = torch.empty(max(wsr, 1), dtype=torch.uint8, device="cuda")
            nat.call("edf_fused_delta_rule_scan_backward", st, P(tq), P(tk), P(tv), P(tb), P(out), P(tdo),
                     *(P(x) for x in g[:4]), P(ws), wsr, B, T, H, d, dt, mode)
        torch.cuda.synchronize()
        grads.append([None if x is None else host(x) for x in g])
    for name, a, b_ in zip(("dq", "dk", "dv", "dbeta", "dalpha"), *grads):
        if a is not None:
            assert np.array_equal(a, b_), f"{name}: saved and recomputed context disagree"
    # and the saved path against the oracle
    qr, kr, vr, br, dor = (rounded(a, dtype) for a in (q, k, v, beta, do))
    ar = rounded(alpha, dtype) if gated else None
    ref = scans.delta_rule_backward(qr, kr, vr, br, dor, ar)
    for name, x in zip(("dq", "dk", "dv", "dbeta", "dalpha"), grads[1]):
        if x is not None:
            assert_close(x, ref[name], TOL[dtype], name, mfma_bf16=chunked)


def test_delta_rule_invariants(rng):
    """beta == 0 gives o == 0; alpha == 1 reproduces DeltaNet; T = 1 closed form."""
    from edifice_amd import fused_scan as fs
    announce("delta_invariants")
    B, T, H, d = 1, 70, 2, 128
    q, k, v, beta, alpha = make_inputs(rng, B, T, H, d, True, True)
    tq, tk, tv, tb = (to_dev(a, torch.bfloat16) for a in (q, k, v, beta))
    zero = fs.gated_delta_net_scan(tq, tk, tv, torch.zeros_like(tb), to_dev(alpha, torch.bfloat16))
    assert host(zero).max() == 0 and host(zero).min() == 0
    ones = torch.ones(B, T, H, dtype=torch.bfloat16, device="cuda")
    assert_close(host(fs.gated_delta_net_scan(tq, tk, tv, tb, ones)), host(fs.delta_net_scan(tq, tk, tv, tb)),
                 TOL[torch.bfloat16], "alpha == 1")
    t1 = [to_dev(a[:, :1], torch.float32) for a in (q, k, v, beta)]
    o1 = host(fs.delta_net_scan(*t1))
    qr, kr, vr, br = (a[:, :1].astype(np.float32).astype(np.float64) for a in (q, k, v, beta))
    expect = (br[..., None] * vr) * (kr * qr).sum(-1, keepdims=True)
    assert_close(o1, expect, 1e-5, "T=1 closed form")


@pytest.mark.parametrize("shape", [(2, 37, 2, 16), (1, 70, 3, 64), (1, 33, 2, 128), (2, 20, 1, 50)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kda_fwd_bwd(shape, dtype, rng):
    """FusedScan.kda_scan/5 and its backward (per-row log decay, per-head beta) against the oracle."""
    from edifice_amd import fused_scan as fs
    bsz, t, h, d = shape
    announce("kda", shape=shape, dtype=dtype)
    q = scans.l2_normalize_keys(rng.normal(size=shape))
    k = scans.l2_normalize_keys(rng.normal(size=shape))
    v = rng.normal(size=shape)
    alpha = -rng.uniform(0.01, 0.3, size=shape)
    beta = rng.uniform(0.1, 0.9, size=(bsz, t, h))
    do = rng.normal(size=shape)
    tq, tk, tv, ta, tb = (to_dev(a, dtype).requires_grad_() for a in (q, k, v, alpha, beta))
    out = fs.kda_scan(tq, tk, tv, ta, tb)
    out.backward(to_dev(do, dtype))
    qr, kr, vr, ar, br, dor = (rounded(a, dtype) for a in (q, k, v, alpha, beta, do))
    tol = TOL[dtype]
    assert_close(host(out), scans.kda_scan(qr, kr, vr, ar, br), tol, "o")
    g = scans.kda_scan_backward(qr, kr, vr, ar, br, dor)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("dalpha", ta), ("dbeta", tb)):
        assert_close(host(tt.grad), g[n], tol, n)



DP_CASES = [
    # (B, T, n_h, H, d, dtype)
    (1, 2, 2, 2, 2, torch.float32),       # reference backward test sizes (head_dim 2)
    # one token: two sub-steps (with one, o_raw = beta (v . q) kn from S = 0 and the RMS norm
    # removes every dependence on q, v, beta but the 1e-6 one: those gradients are ~1e-4 of
    # dk and f32 cancellation, not the kernel, sets their relative error)
    (1, 1, 2, 1, 8, torch.float32),
    (2, 9, 2, 2, 16, torch.float32),
    (1, 37, 3, 2, 64, torch.float32),     # sub-steps not a multiple of the 16-step chunk
    (1, 20, 1, 1, 128, torch.float32),    # n_h = 1
    (2, 33, 2, 2, 50, torch.float32),     # head_dim off the padded widths
    (1, 70, 4, 1, 32, torch.bfloat16),
    (1, 40, 2, 2, 128, torch.bfloat16),
]


@pytest.mark.parametrize("case", DP_CASES)
def test_delta_product_fwd_bwd(case, rng):
    """FusedScan.delta_product_scan/4 and its backward against the oracle (raw keys, the
    kernel normalizes; beta up to 2 as with allow_neg_eigval)."""
    from edifice_amd import fused_scan as fs
    bsz, t, nhh, h, d, dtype = case
    announce("delta_product", case=case)
    q = rng.normal(size=(bsz, t, h, d))
    k, v = rng.normal(size=(bsz, t, nhh, h, d)), rng.normal(size=(bsz, t, nhh, h, d))
    beta = rng.uniform(0.1, 1.9, size=(bsz, t, nhh, h))
    do = rng.normal(size=(bsz, t, h, d))
    tq, tk, tv, tb = (to_dev(a, dtype).requires_grad_() for a in (q, k, v, beta))
    out = fs.delta_product_scan(tq, tk, tv, tb)
    out.backward(to_dev(do, dtype))
    qr, kr, vr, br, dor = (rounded(a, dtype) for a in (q, k, v, beta, do))
    tol = TOL[dtype]
    assert_close(host(out), scans.delta_product(qr, kr, vr, br), tol, "o")
    g = scans.delta_product_backward(qr, kr, vr, br, dor)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("dbeta", tb)):
        assert_close(host(tt.grad), g[n], tol, n)


RLA_CASES = [
    # (B, T, H, d, dtype, variant, clip)
    (1, 5, 2, 3, torch.float32, "rla", 0.6),
    (1, 1, 1, 8, torch.float32, "rdn", 0.6),      # one step
    (2, 21, 2, 16, torch.float32, "rdn", 0.6),
    (1, 37, 2, 64, torch.float32, "rla", 1.0),    # T not a multiple of the 8-step chunk
    (1, 30, 1, 128, torch.float32, "rdn", 1.0),
    (2, 17, 2, 50, torch.float32, "rla", 0.3),    # head_dim off the padded widths
    (1, 40, 2, 64, torch.bfloat16, "rdn", 1.0),
    (1, 33, 1, 128, torch.bfloat16, "rla", 1.0),
]


@pytest.mark.parametrize("case", RLA_CASES)
def test_rla_fwd_bwd(case, rng):
    """FusedScan.rla_scan/7 (RLA and RDN) and its backward against the oracle; keys scaled
    so that the retrievals stay O(1) and part of the residual errors clip."""
    from edifice_amd import fused_scan as fs
    bsz, t, h, d, dtype, variant, clip = case
    announce("rla", case=case)
    q = rng.normal(size=(bsz, t, h, d))
    k = scans.l2_normalize_keys(rng.normal(size=(bsz, t, h, d)))
    v = rng.normal(size=(bsz, t, h, d))
    alpha, beta, gamma = (rng.uniform(0.3, 0.95, size=(bsz, t, h)) for _ in range(3))
    do = rng.normal(size=(bsz, t, h, d))
    tq, tk, tv, ta, tb, tg = (to_dev(x, dtype).requires_grad_() for x in (q, k, v, alpha, beta, gamma))
    out = fs.rla_scan(tq, tk, tv, ta, tb, tg, variant, clip)
    out.backward(to_dev(do, dtype))
    xs = [rounded(x, dtype) for x in (q, k, v, alpha, beta, gamma)]
    var = scans.RLA_VARIANTS[variant]
    tol = TOL[dtype]
    assert_close(host(out), scans.rla_scan(*xs, var, clip), tol, "o")
    g = scans.rla_scan_backward(*xs, rounded(do, dtype), var, clip)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("dalpha", ta), ("dbeta", tb), ("dgamma", tg)):
        assert_close(host(tt.grad), g[n], tol, n)


TTT_CASES = [
    # (B, T, D, dtype)
    (2, 5, 4, torch.float32),
    (1, 1, 8, torch.float32),       # one step
    (2, 37, 16, torch.float32),     # T not a multiple of the 8-step chunk
    (3, 20, 50, torch.float32),     # D off the padded widths
    (1, 30, 64, torch.float32),
    (2, 24, 128, torch.float32),
    (2, 33, 64, torch.bfloat16),
    (1, 16, 128, torch.bfloat16),
]


@pytest.mark.parametrize("case", TTT_CASES)
def test_ttt_fwd_bwd(case, rng):
    """FusedScan.ttt_scan/7 and its backward (dq, dk, dv, deta, dw0, dln_g, dln_b) against
    the oracle; eta ~ sigmoid / D as the reference block feeds it."""
    from edifice_amd import fused_scan as fs
    bsz, t, d, dtype = case
    announce("ttt", case=case)
    q, k, v, do = (rng.normal(size=(bsz, t, d)) for _ in range(4))
    k = k / np.sqrt(d)
    eta = rng.uniform(0.2, 0.8, size=(bsz, t, d)) / d * 4
    w0 = rng.normal(size=(bsz, d, d)) / np.sqrt(d)
    g, b = 1 + 0.2 * rng.normal(size=d), 0.2 * rng.normal(size=d)
    ts = [to_dev(x, dtype).requires_grad_() for x in (q, k, v, eta, w0, g, b)]
    out = fs.ttt_scan(*ts)
    out.backward(to_dev(do, dtype))
    xs = [rounded(x, dtype) for x in (q, k, v, eta, w0, g, b)]
    tol = TOL[dtype]
    assert_close(host(out), scans.ttt_scan(*xs), tol, "o")
    gr = scans.ttt_scan_backward(*xs, rounded(do, dtype))
    for n, tt in zip(("dq", "dk", "dv", "deta", "dw0", "dln_g", "dln_b"), ts):
        assert_close(host(tt.grad), gr[n], tol, n)


@pytest.mark.parametrize("case", [(2, 37, 16, torch.float32), (2, 33, 64, torch.bfloat16)],
                         ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_ttt_context_entry_points_agree(case, rng):
    """edf_fused_ttt_scan_with_context (the training forward, recording the backward's context
    in the same pass) gives the plain forward's output, and edf_fused_ttt_scan_backward_saved
    from that context gives the recomputing backward's gradients, bit for bit (same kernels)."""
    import ctypes

    from edifice_amd import _native as nat
    bsz, t, d, dtype = case
    announce("ttt_context", case=case)
    q, k, v, do = (rng.normal(size=(bsz, t, d)) for _ in range(4))
    eta = rng.uniform(0.2, 0.8, size=(bsz, t, d)) / d * 4
    w0 = rng.normal(size=(bsz, d, d)) / np.sqrt(d)
    g, b = 1 + 0.2 * rng.normal(size=d), 0.2 * rng.normal(size=d)
    ins = [to_dev(x, dtype) for x in (q, k / np.sqrt(d), v, eta, w0, g, b)]
    tdo = to_dev(do, dtype)
    P = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dt = 1 if dtype == torch.bfloat16 else 0
    wsb = nat.query("edf_ttt_scan_backward_workspace_bytes", bsz, t, d, dt)
    recb = nat.query("edf_ttt_scan_context_bytes", bsz, t, d, dt)
    rec = torch.empty(recb, dtype=torch.uint8, device="cuda")
    outs, grads = [], []
    for saved in (False, True):
        out = torch.empty_like(ins[0])
        if saved:
            nat.call("edf_fused_ttt_scan_with_context", st, *(P(x) for x in ins), P(out), P(rec), recb, bsz, t, d, dt)
        else:
            nat.call("edf_fused_ttt_scan", st, *(P(x) for x in ins), P(out), bsz, t, d, dt)
        gs = [torch.empty_like(x) for x in ins]
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        if saved:
            nat.call("edf_fused_ttt_scan_backward_saved", st, *(P(x) for x in ins), P(tdo), *(P(x) for x in gs),
                     P(rec), recb, P(ws), wsb, bsz, t, d, dt)
        else:
            nat.call("edf_fused_ttt_scan_backward", st, *(P(x) for x in ins), P(tdo), *(P(x) for x in gs), P(ws), wsb,
                     bsz, t, d, dt)
        torch.cuda.synchronize()
        outs.append(out)
        grads.append(gs)
    assert torch.equal(outs[0], outs[1])
    for a, c in zip(*grads):
        assert torch.equal(a, c)


@pytest.mark.parametrize("case", [(2, 13, 2, 2, 16, torch.float32), (1, 40, 3, 2, 128, torch.bfloat16)],
                         ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_delta_product_context_entry_points_agree(case, rng):
    """edf_fused_delta_product_scan_with_context gives the plain forward's output, and
    edf_fused_delta_product_scan_backward_saved from its context the recomputing backward's
    gradients, bit for bit (same kernels)."""
    import ctypes

    from edifice_amd import _native as nat
    B, T, NH, H, d, dtype = case
    announce("delta_product_context", case=case)
    q = rng.normal(size=(B, T, H, d))
    k = rng.normal(size=(B, T, NH, H, d))
    v = rng.normal(size=(B, T, NH, H, d))
    beta = 1 / (1 + np.exp(-rng.normal(size=(B, T, NH, H))))
    do = rng.normal(size=(B, T, H, d))
    tq, tk, tv, tb, tdo = (to_dev(x, dtype) for x in (q, k, v, beta, do))
    P = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dt = 1 if dtype == torch.bfloat16 else 0
    wsf = nat.query("edf_delta_product_workspace_bytes", B, T, NH, H, d, dt)
    wsb = nat.query("edf_delta_product_backward_workspace_bytes", B, T, NH, H, d, dt)
    recb = nat.query("edf_delta_product_context_bytes", B, T, NH, H, d, dt)
    rec = torch.empty(recb, dtype=torch.uint8, device="cuda")
    outs, grads = [], []
    for saved in (False, True):
        out = torch.empty_like(tq)
        if saved:
            nat.call("edf_fused_delta_product_scan_with_context", st, P(tq), P(tk), P(tv), P(tb), P(out), P(rec), recb,
                     B, T, NH, H, d, dt)
        else:
            ws = torch.empty(wsf, dtype=torch.uint8, device="cuda")
            nat.call("edf_fused_delta_product_scan", st, P(tq), P(tk), P(tv), P(tb), P(out), P(ws), wsf,
                     B, T, NH, H, d, dt)
        gs = [torch.empty_like(x) for x in (tq, tk, tv, tb)]
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        if saved:
            nat.call("edf_fused_delta_product_scan_backward_saved", st, P(tq), P(tk), P(tv), P(tb), P(tdo),
                     *(P(x) for x in gs), P(rec), recb, P(ws), wsb, B, T, NH, H, d, dt)
        else:
            nat.call("edf_fused_delta_product_scan_backward", st, P(tq), P(tk), P(tv), P(tb), P(out), P(tdo),
                     *(P(x) for x in gs), P(ws), wsb, B, T, NH, H, d, dt)
        torch.cuda.synchronize()
        outs.append(out)
        grads.append(gs)
    assert torch.equal(outs[0], outs[1])
    for a, c in zip(*grads):
        assert torch.equal(a, c)


@pytest.mark.parametrize("case", [(2, 21, 2, 16, torch.float32, 0), (1, 40, 2, 128, torch.bfloat16, 1)],
                         ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_rla_context_entry_points_agree(case, rng):
    """edf_fused_rla_scan_with_context gives the plain forward's output (within rounding: it
    walks the sequence in 8-step chunks instead of 16, the same arithmetic per step) and
    edf_fused_rla_scan_backward_saved from its context the recomputing backward's gradients bit
    for bit (the same checkpointing pass writes the states)."""
    import ctypes

    from edifice_amd import _native as nat
    B, T, H, d, dtype, variant = case
    announce("rla_context", case=case)
    q, k, v, do = (rng.normal(size=(B, T, H, d)) for _ in range(4))
    k = scans.l2_normalize_keys(k)
    alpha, beta, gamma = (1 / (1 + np.exp(-rng.normal(size=(B, T, H)))) for _ in range(3))
    ins = [to_dev(x, dtype) for x in (q, k, v, alpha, beta, gamma)]
    tdo = to_dev(do, dtype)
    P = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dt = 1 if dtype == torch.bfloat16 else 0
    wsb = nat.query("edf_rla_scan_backward_workspace_bytes", B, T, H, d, dt)
    recb = nat.query("edf_rla_scan_context_bytes", B, T, H, d, dt)
    rec = torch.empty(recb, dtype=torch.uint8, device="cuda")
    outs, grads = [], []
    for saved in (False, True):
        out = torch.empty_like(ins[0])
        if saved:
            nat.call("edf_fused_rla_scan_with_context", st, *(P(x) for x in ins), P(out), P(rec), recb,
                     B, T, H, d, variant, 1.0, dt)
        else:
            nat.call("edf_fused_rla_scan", st, *(P(x) for x in ins), P(out), B, T, H, d, variant, 1.0, dt)
        gs = [torch.empty_like(x) for x in ins]
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        if saved:
            nat.call("edf_fused_rla_scan_backward_saved", st, *(P(x) for x in ins), P(tdo), *(P(x) for x in gs),
                     P(rec), recb, P(ws), wsb, B, T, H, d, variant, 1.0, dt)
        else:
            nat.call("edf_fused_rla_scan_backward", st, *(P(x) for x in ins), P(out), P(tdo), *(P(x) for x in gs),
                     P(ws), wsb, B, T, H, d, variant, 1.0, dt)
        torch.cuda.synchronize()
        outs.append(host(out))
        grads.append(gs)
    assert_close(outs[1], outs[0], TOL[dtype], "o")
    for a, c in zip(*grads):
        assert torch.equal(a, c)


def test_kda_context_entry_points_agree(rng):
    """edf_fused_kda_scan_with_context gives the plain forward's output and
    edf_fused_kda_scan_backward_saved from its context the recomputing backward's gradients,
    bit for bit (same kernels)."""
    import ctypes

    from edifice_amd import _native as nat
    B, T, H, d, dtype = 2, 45, 2, 64, torch.bfloat16
    announce("kda_context")
    q, k, v, do = (rng.normal(size=(B, T, H, d)) for _ in range(4))
    k = scans.l2_normalize_keys(k)
    alpha = -rng.uniform(0.01, 0.3, size=(B, T, H, d))  # log decay, as test_kda_fwd_bwd
    beta = rng.uniform(0.1, 0.9, size=(B, T, H))
    ins = [to_dev(x, dtype) for x in (q, k, v, alpha, beta)]
    tdo = to_dev(do, dtype)
    P = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    wsb = nat.query("edf_kda_scan_backward_workspace_bytes", B, T, H, d, 1)
    recb = nat.query("edf_kda_scan_context_bytes", B, T, H, d, 1)
    rec = torch.empty(recb, dtype=torch.uint8, device="cuda")
    outs, grads = [], []
    for saved in (False, True):
        out = torch.empty_like(ins[0])
        if saved:
            nat.call("edf_fused_kda_scan_with_context", st, *(P(x) for x in ins), P(out), P(rec), recb, B, T, H, d, 1)
        else:
            nat.call("edf_fused_kda_scan", st, *(P(x) for x in ins), P(out), B, T, H, d, 1)
        gs = [torch.empty_like(x) for x in ins]
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        if saved:
            nat.call("edf_fused_kda_scan_backward_saved", st, *(P(x) for x in ins), P(tdo), *(P(x) for x in gs),
                     P(rec), recb, P(ws), wsb, B, T, H, d, 1)
        else:
            nat.call("edf_fused_kda_scan_backward", st, *(P(x) for x in ins), P(out), P(tdo), *(P(x) for x in gs),
                     P(ws), wsb, B, T, H, d, 1)
        torch.cuda.synchronize()
        outs.append(out)
        grads.append(gs)
    assert torch.equal(outs[0], outs[1])
    for a, c in zip(*grads):
        assert torch.equal(a, c)
