"""Pin the oracle's hand-derived backward passes against torch autograd (float64).

The autograd side differentiates a torch restatement of the FORWARD only, so it is
independent of the hand-derived backward in oracle/scans.py (which follows the
reference's *_backward_fallback functions).  Finite differences back both up.
CPU only.
"""
import numpy as np
import pytest
import torch

from oracle import scans
from tests.conftest import assert_close

F64 = torch.float64  # explicit everywhere: never change torch's global default dtype


def _t(a, grad=True):
    return torch.tensor(np.asarray(a), dtype=torch.float64, requires_grad=grad)


def torch_mingru(z, c, h0):
    h, out = h0, []
    for t in range(z.shape[1]):
        h = (1 - z[:, t]) * h + z[:, t] * c[:, t]
        out.append(h)
    return torch.stack(out, 1)


def torch_minlstm(f, i, c, h0):
    s = f + i + 1e-6
    fn, inn = f / s, i / s
    h, out = h0, []
    for t in range(f.shape[1]):
        h = fn[:, t] * h + inn[:, t] * c[:, t]
        out.append(h)
    return torch.stack(out, 1)


def test_mingru_backward_vs_autograd(rng):
    z = rng.uniform(0.05, 0.95, size=(2, 13, 6))
    c = rng.normal(size=z.shape)
    h0 = rng.normal(size=(2, 6))
    dy = rng.normal(size=z.shape)
    tz, tc, th = _t(z), _t(c), _t(h0)
    torch_mingru(tz, tc, th).backward(torch.from_numpy(dy))
    fwd = scans.mingru_scan(z, c, h0)
    dz, dc, dh0 = scans.mingru_scan_backward(z, c, h0, fwd, dy)
    for a, e, n in ((dz, tz.grad, "dz"), (dc, tc.grad, "dc"), (dh0, th.grad, "dh0")):
        assert_close(a, e.numpy(), 1e-12, n)
    # logit-level chain rule
    g = rng.normal(size=z.shape)
    tg = _t(g)
    torch_mingru(torch.sigmoid(tg), tc.detach(), torch.zeros(2, 6, dtype=F64)).backward(torch.from_numpy(dy))
    dg, _ = scans.min_gru_scan_backward(g, c, dy)
    assert_close(dg, tg.grad.numpy(), 1e-12, "dgates")


def torch_linear_closed_form(a, b, h0):
    """h_t = sum_{s<=t} (prod_{s<r<=t} a_r) b_s + (prod_{r<=t} a_r) h0, built from
    cumulative products (not the recurrence the oracle restates)."""
    T = a.shape[1]
    out = []
    for t in range(T):
        h = torch.prod(a[:, :t + 1], dim=1) * h0
        for s in range(t + 1):
            h = h + torch.prod(a[:, s + 1:t + 1], dim=1) * b[:, s]
        out.append(h)
    return torch.stack(out, 1)


def test_linear_scan_forward_backward_vs_autograd(rng):
    a = rng.uniform(-1.1, 1.1, size=(2, 9, 4))
    b = rng.normal(size=a.shape)
    h0 = rng.normal(size=(2, 4))
    dy = rng.normal(size=a.shape)
    ta, tb, th = _t(a), _t(b), _t(h0)
    out = torch_linear_closed_form(ta, tb, th)
    fwd = scans.linear_scan(a, b, h0)
    assert_close(fwd, out.detach().numpy(), 1e-12, "h")
    out.backward(torch.from_numpy(dy))
    da, db, dh0 = scans.linear_scan_backward(a, h0, fwd, dy)
    for x, e, n in ((da, ta.grad, "da"), (db, tb.grad, "db"), (dh0, th.grad, "dh0")):
        assert_close(x, e.numpy(), 1e-12, n)


def test_linear_scan_backward_finite_difference(rng):
    """backward_kernels_test.exs:52-74 (finite differences of sum(forward))."""
    a = rng.uniform(0.2, 0.8, size=(1, 5, 3))
    b = rng.uniform(-0.5, 0.5, size=a.shape)
    h0 = rng.normal(size=(1, 3))
    dy = rng.normal(size=a.shape)
    da, db, dh0 = scans.linear_scan_backward(a, h0, scans.linear_scan(a, b, h0), dy)
    eps = 1e-6
    for name, arr, g in (("da", a, da), ("db", b, db), ("dh0", h0, dh0)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            old = arr[idx]
            arr[idx] = old + eps
            fp = (scans.linear_scan(a, b, h0) * dy).sum()
            arr[idx] = old - eps
            fm = (scans.linear_scan(a, b, h0) * dy).sum()
            arr[idx] = old
            num[idx] = (fp - fm) / (2 * eps)
        assert_close(g, num, 1e-7, name)


def test_minlstm_backward_vs_autograd(rng):
    f = rng.uniform(0.05, 0.95, size=(2, 11, 5))
    i = rng.uniform(0.05, 0.95, size=f.shape)
    c = rng.normal(size=f.shape)
    h0 = rng.normal(size=(2, 5))
    dy = rng.normal(size=f.shape)
    tf, ti, tc, th = _t(f), _t(i), _t(c), _t(h0)
    torch_minlstm(tf, ti, tc, th).backward(torch.from_numpy(dy))
    fwd = scans.minlstm_scan(f, i, c, h0)
    df, di, dc, dh0 = scans.minlstm_scan_backward(f, i, c, h0, fwd, dy)
    for a, e, n in ((df, tf.grad, "df"), (di, ti.grad, "di"), (dc, tc.grad, "dc"), (dh0, th.grad, "dh0")):
        assert_close(a, e.numpy(), 1e-12, n)


def torch_selective_assoc(x, dt, A, B, C, D, z, mode):
    """Independent forward: the scan as cumulative sums in log-decay space,
    h_t = sum_{s<=t} exp(A (cum_t - cum_s)) dtb_s B_s x_s (no recurrence)."""
    dtc = torch.clamp(dt, 1e-3, 0.1)
    dtb = dtc.mean(-1, keepdim=True).expand_as(dtc) if mode == "mean" else dtc
    cum = torch.cumsum(dtc, 1)  # [b, t, d]
    T = x.shape[1]
    ys = []
    for t in range(T):
        decay = torch.exp(A[None, None] * (cum[:, t:t + 1, :, None] - cum[:, :t + 1, :, None]))  # [b,s,d,n]
        h = (decay * (dtb[:, :t + 1, :, None] * B[:, :t + 1, None, :] * x[:, :t + 1, :, None])).sum(1)
        ys.append((h * C[:, t, None, :]).sum(-1))
    y = torch.stack(ys, 1)
    if D is not None:
        y = y + D * x
    if z is not None:
        y = y * z * torch.sigmoid(z)
    return y


@pytest.mark.parametrize("mode", ["channel", "mean"])
@pytest.mark.parametrize("extras", [False, True])
def test_selective_scan_forward_backward_vs_autograd(rng, mode, extras):
    bsz, T, D, N = 2, 9, 5, 4
    x = rng.normal(size=(bsz, T, D))
    dt = rng.uniform(0.0, 0.15, size=(bsz, T, D))  # some entries outside [1e-3, 0.1]
    A = -np.exp(rng.uniform(0, np.log(16), size=(D, N)))
    B, C = rng.normal(size=(bsz, T, N)), rng.normal(size=(bsz, T, N))
    Dv = rng.normal(size=D) if extras else None
    z = rng.normal(size=x.shape) if extras else None
    dy = rng.normal(size=x.shape)
    tx, tdt, tA, tB, tC = _t(x), _t(dt), _t(A), _t(B), _t(C)
    tD = _t(Dv) if extras else None
    tz = _t(z) if extras else None
    y_t = torch_selective_assoc(tx, tdt, tA, tB, tC, tD, tz, mode)
    y = scans.selective_scan(x, dt, A, B, C, Dv, z, mode)
    assert_close(y, y_t.detach().numpy(), 1e-12, "forward")
    y_t.backward(torch.from_numpy(dy))
    g = scans.selective_scan_backward(x, dt, A, B, C, dy, Dv, z, mode)
    pairs = [("dx", tx), ("ddt", tdt), ("dA", tA), ("dB", tB), ("dC", tC)]
    if extras:
        pairs += [("dD", tD), ("dz", tz)]
    for name, tt in pairs:
        assert_close(g[name], tt.grad.numpy(), 1e-10, name)


def torch_delta(q, k, v, beta, alpha):
    bsz, T, H, d = q.shape
    S = torch.zeros(bsz, H, v.shape[-1], d, dtype=F64)
    out = []
    for t in range(T):
        if alpha is not None:
            S = alpha[:, t, :, None, None] * S
        r = torch.einsum("bhij,bhj->bhi", S, k[:, t])
        b = beta[:, t] if beta.dim() == 4 else beta[:, t, :, None]
        S = S + (b * (v[:, t] - r))[..., None] * k[:, t, :, None, :]
        out.append(torch.einsum("bhij,bhj->bhi", S, q[:, t]))
    return torch.stack(out, 1)


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("per_head_beta", [False, True])
def test_delta_rule_backward_vs_autograd(rng, gated, per_head_beta):
    bsz, T, H, d = 2, 7, 2, 4
    q = rng.normal(size=(bsz, T, H, d))
    k = scans.l2_normalize_keys(rng.normal(size=(bsz, T, H, d)))
    v = rng.normal(size=(bsz, T, H, d))
    beta = rng.uniform(size=(bsz, T, H) if per_head_beta else (bsz, T, H, d))
    alpha = rng.uniform(0.5, 1.0, size=(bsz, T, H)) if gated else None
    do = rng.normal(size=v.shape)
    tq, tk, tv, tb = _t(q), _t(k), _t(v), _t(beta)
    ta = _t(alpha) if gated else None
    o_t = torch_delta(tq, tk, tv, tb, ta)
    assert_close(scans.delta_rule(q, k, v, beta, alpha), o_t.detach().numpy(), 1e-12, "forward")
    o_t.backward(torch.from_numpy(do))
    g = scans.delta_rule_backward(q, k, v, beta, do, alpha)
    pairs = [("dq", tq), ("dk", tk), ("dv", tv), ("dbeta", tb)] + ([("dalpha", ta)] if gated else [])
    for name, tt in pairs:
        assert_close(g[name], tt.grad.numpy(), 1e-10, name)


@pytest.mark.parametrize("causal", [False, True])
def test_flash_backward_vs_sdpa_autograd(rng, causal):
    bsz, H, T, d = 2, 2, 9, 8
    q, k, v, do = (rng.normal(size=(bsz, H, T, d)) for _ in range(4))
    tq, tk, tv = _t(q), _t(k), _t(v)
    torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).backward(torch.from_numpy(do))
    dq, dk, dv = scans.flash_attention_backward(q, k, v, do, causal)
    for a, tt, n in ((dq, tq, "dq"), (dk, tk, "dk"), (dv, tv, "dv")):
        assert_close(a, tt.grad.numpy(), 1e-10, n)


def test_selective_scan_backward_finite_difference(rng):
    bsz, T, D, N = 1, 6, 3, 2
    x = rng.normal(size=(bsz, T, D))
    dt = rng.uniform(0.01, 0.09, size=(bsz, T, D))
    A = -np.exp(rng.uniform(0, 2, size=(D, N)))
    B, C = rng.normal(size=(bsz, T, N)), rng.normal(size=(bsz, T, N))
    dy = rng.normal(size=x.shape)
    g = scans.selective_scan_backward(x, dt, A, B, C, dy)
    eps = 1e-6
    for name, arr in (("dx", x), ("ddt", dt), ("dA", A), ("dB", B), ("dC", C)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            old = arr[idx]
            arr[idx] = old + eps
            fp = (scans.selective_scan(x, dt, A, B, C) * dy).sum()
            arr[idx] = old - eps
            fm = (scans.selective_scan(x, dt, A, B, C) * dy).sum()
            arr[idx] = old
            num[idx] = (fp - fm) / (2 * eps)
        assert_close(g[name], num, 1e-6, name)


def test_fox_attention_vs_torch_autograd(rng):
    """FoX forward and backward against torch autograd of an independent torch forward
    (scores + cs_i - cs_j, causal softmax)."""
    b, h, t, d = 1, 2, 9, 4
    q, k, v, do = (rng.normal(size=(b, h, t, d)) for _ in range(4))
    cs = np.cumsum(np.log(1 / (1 + np.exp(-rng.normal(size=(b, h, t))))), axis=-1)
    tq, tk, tv, tc = _t(q), _t(k), _t(v), _t(cs)
    sc = tq @ tk.transpose(-1, -2) / np.sqrt(d) + tc[..., :, None] - tc[..., None, :]
    mask = torch.ones(t, t, dtype=torch.bool).tril()
    sc = sc.masked_fill(~mask, float("-inf"))
    out = torch.softmax(sc, -1) @ tv
    out.backward(torch.from_numpy(do))
    assert_close(scans.fox_attention(q, k, v, cs), out.detach().numpy(), 1e-12, "o")
    dq, dk, dv, dcs = scans.fox_attention_backward(q, k, v, cs, do)
    for a, e, n in ((dq, tq.grad, "dq"), (dk, tk.grad, "dk"), (dv, tv.grad, "dv"), (dcs, tc.grad, "dcs")):
        assert_close(a, e.numpy(), 1e-10, n)


@pytest.mark.parametrize("causal", [True, False])
def test_laser_attention_vs_torch_autograd(rng, causal):
    b, h, t, d = 1, 2, 8, 4
    q, k, v, do = (rng.normal(size=(b, h, t, d)) for _ in range(4))
    tq, tk, tv = _t(q), _t(k), _t(v)
    sc = tq @ tk.transpose(-1, -2) / np.sqrt(d)
    if causal:
        sc = sc.masked_fill(~torch.ones(t, t, dtype=torch.bool).tril(), float("-inf"))
    vmax = tv.detach().amax(dim=2, keepdim=True)
    out = torch.log(torch.softmax(sc, -1) @ torch.exp(tv - vmax)) + vmax
    out.backward(torch.from_numpy(do))
    assert_close(scans.laser_attention(q, k, v, causal), out.detach().numpy(), 1e-12, "o")
    dq, dk, dv = scans.laser_attention_backward(q, k, v, do, causal)
    for a, e, n in ((dq, tq.grad, "dq"), (dk, tk.grad, "dk"), (dv, tv.grad, "dv")):
        assert_close(a, e.numpy(), 1e-10, n)


def test_kda_backward_vs_autograd(rng):
    """KDA backward (oracle) against torch autograd of an independent torch forward."""
    bsz, t, h, d = 1, 5, 2, 3
    q, k, v, do = (rng.normal(size=(bsz, t, h, d)) for _ in range(4))
    alpha = -rng.uniform(0.05, 0.6, size=(bsz, t, h, d))
    beta = rng.uniform(0.1, 0.9, size=(bsz, t, h))
    tq, tk, tv, ta, tb = _t(q), _t(k), _t(v), _t(alpha), _t(beta)
    S = torch.zeros(bsz, h, d, d, dtype=F64)
    outs = []
    for s in range(t):
        S = torch.exp(ta[:, s])[..., :, None] * S
        err = tv[:, s] - torch.einsum("bhij,bhj->bhi", S, tk[:, s])
        S = S + tb[:, s][..., None, None] * err[..., :, None] * tk[:, s][..., None, :]
        outs.append(torch.einsum("bhij,bhj->bhi", S, tq[:, s]))
    out = torch.stack(outs, 1)
    out.backward(torch.from_numpy(do))
    assert_close(scans.kda_scan(q, k, v, alpha, beta), out.detach().numpy(), 1e-12, "o")
    g = scans.kda_scan_backward(q, k, v, alpha, beta, do)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("dalpha", ta), ("dbeta", tb)):
        assert_close(g[n], tt.grad.numpy(), 1e-10, n)



def test_delta_product_backward_vs_autograd(rng):
    """DeltaProduct backward (oracle) against torch autograd of the reference-convention
    forward (state [key][value], matrix Householder form, RMS-normalized S q)."""
    bsz, t, nhh, h, d = 1, 4, 2, 2, 3
    q, do = rng.normal(size=(bsz, t, h, d)), rng.normal(size=(bsz, t, h, d))
    k, v = rng.normal(size=(bsz, t, nhh, h, d)), rng.normal(size=(bsz, t, nhh, h, d))
    beta = rng.uniform(0.1, 1.9, size=(bsz, t, nhh, h))
    tq, tk, tv, tb = _t(q), _t(k), _t(v), _t(beta)
    S = torch.zeros(bsz, h, d, d, dtype=F64)
    eye = torch.eye(d, dtype=F64)
    outs = []
    for s in range(t):
        for j in range(nhh):
            kv = tk[:, s, j]
            kn = kv / torch.sqrt((kv * kv).sum(-1, keepdim=True) + 1e-6)
            be = tb[:, s, j][..., None, None]
            S = (eye - be * kn[..., :, None] * kn[..., None, :]) @ S + be * kn[..., :, None] * tv[:, s, j][..., None, :]
        o = (S @ tq[:, s][..., None])[..., 0]
        outs.append(o / torch.sqrt((o * o).mean(-1, keepdim=True) + 1e-6))
    out = torch.stack(outs, 1)
    out.backward(torch.from_numpy(do))
    assert_close(scans.delta_product(q, k, v, beta), out.detach().numpy(), 1e-12, "o")
    g = scans.delta_product_backward(q, k, v, beta, do)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("dbeta", tb)):
        assert_close(g[n], tt.grad.numpy(), 1e-10, n)


@pytest.mark.parametrize("variant", [0, 1])
def test_rla_backward_vs_autograd(rng, variant):
    """RLA / RDN backward (oracle) against torch autograd of an independent forward written
    from the reference's matrix statement (fused_rla_scan.cu:1-20); the threshold 0.6
    clips part of the errors."""
    bsz, t, h, d = 1, 5, 2, 3
    q, k, v, do = (rng.normal(size=(bsz, t, h, d)) for _ in range(4))
    alpha, beta, gamma = (rng.uniform(0.3, 0.95, size=(bsz, t, h)) for _ in range(3))
    tq, tk, tv, ta, tb, tg = _t(q), _t(k), _t(v), _t(alpha), _t(beta), _t(gamma)
    S = torch.zeros(bsz, h, d, d, dtype=F64)
    R = torch.zeros(bsz, h, d, d, dtype=F64)
    outs, clipped = [], 0
    for s in range(t):
        kk, vv = tk[:, s], tv[:, s]
        a, b, g = (x[:, s][..., None, None] for x in (ta, tb, tg))
        err = vv - (S @ kk[..., None])[..., 0]
        clipped += int((err.abs() > 0.6).sum())
        re = torch.clamp(err, -0.6, 0.6)
        if variant == 0:
            S2 = a * S + b * vv[..., :, None] * kk[..., None, :]
            R2 = a * R + g * re[..., :, None] * kk[..., None, :]
        else:
            rr = (R @ kk[..., None])[..., 0]
            S2 = a * S + b * err[..., :, None] * kk[..., None, :]
            R2 = a * R + g * (re - rr)[..., :, None] * kk[..., None, :]
        S, R = S2, R2
        outs.append(((S + R) @ tq[:, s][..., None])[..., 0])
    assert clipped > 0
    out = torch.stack(outs, 1)
    out.backward(torch.from_numpy(do))
    assert_close(scans.rla_scan(q, k, v, alpha, beta, gamma, variant, 0.6), out.detach().numpy(), 1e-12, "o")
    gr = scans.rla_scan_backward(q, k, v, alpha, beta, gamma, do, variant, 0.6)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("dalpha", ta), ("dbeta", tb), ("dgamma", tg)):
        assert_close(gr[n], tt.grad.numpy(), 1e-10, n)


def test_ttt_backward_vs_autograd(rng):
    """TTT-Linear backward (oracle) against torch autograd of an independent forward using
    torch.nn.functional.layer_norm (population variance, eps 1e-6)."""
    bsz, t, d = 2, 4, 5
    q, k, v, do = (rng.normal(size=(bsz, t, d)) for _ in range(4))
    eta = rng.uniform(0.05, 0.3, size=(bsz, t, d))
    w0 = 0.5 * rng.normal(size=(bsz, d, d))
    g, b = 1 + 0.3 * rng.normal(size=d), 0.3 * rng.normal(size=d)
    tq, tk, tv, te, tw, tg, tb = (_t(x) for x in (q, k, v, eta, w0, g, b))
    W = tw
    outs = []
    for s in range(t):
        pred = (W @ tk[:, s][..., None])[..., 0]
        err = torch.nn.functional.layer_norm(pred, (d,), tg, tb, eps=1e-6) - tv[:, s]
        W = W - (te[:, s] * err)[..., :, None] * tk[:, s][:, None, :]
        outs.append((W @ tq[:, s][..., None])[..., 0])
    out = torch.stack(outs, 1)
    out.backward(torch.from_numpy(do))
    assert_close(scans.ttt_scan(q, k, v, eta, w0, g, b), out.detach().numpy(), 1e-12, "o")
    gr = scans.ttt_scan_backward(q, k, v, eta, w0, g, b, do)
    for n, tt in (("dq", tq), ("dk", tk), ("dv", tv), ("deta", te), ("dw0", tw), ("dln_g", tg), ("dln_b", tb)):
        assert_close(gr[n], tt.grad.numpy(), 1e-10, n)
