"""Pins for the CPU oracle (oracle/scans.py): reference fixtures, known answers, invariants.

Each check is chosen so that a plausible restatement mistake (dropped term, wrong
sign or index, transposed operand) fails it.  CPU only.
"""
import os

import numpy as np
import pytest
import torch

from oracle import blocks, scans
from tests.conftest import GOLDEN, assert_close


# ---------------------------------------------------------------------------
# reference fixtures (test/fixtures/numerical/*_random.safetensors, checked by
# test/edifice/pretrained/architecture_numerical_test.exs at atol 1e-4)
# ---------------------------------------------------------------------------

MODELS = {
    "min_gru": blocks.min_gru_model,
    "delta_net": blocks.delta_net_model,
    "mamba": blocks.mamba_model,
    "gqa": blocks.gqa_model,
}


@pytest.mark.parametrize("name", sorted(MODELS))
def test_oracle_matches_reference_fixture(name):
    w = blocks.load_fixture(os.path.join(GOLDEN, f"{name}_random.safetensors"))
    out = MODELS[name](w, w["input.state_sequence"], blocks.oracle_ops())
    err = (out - w["expected_output"]).abs().max().item()
    assert err < 1e-4, f"{name}: max abs err {err}"


def test_mamba_fixture_saturates_the_dt_clip():
    """In the Mamba fixture every softplus(dt) exceeds 0.1, so clip(dt) == 0.1 everywhere and
    the dt-mean (common.ex:402-445) and per-channel (fused_selective_scan.cu:68-90)
    discretisations coincide: the fixture pins the clip, A = -(1..N) and the block wiring,
    not the choice between the two modes (the autograd tests pin each mode's formula)."""
    w = blocks.load_fixture(os.path.join(GOLDEN, "mamba_random.safetensors"))
    seen = []
    ops = blocks.oracle_ops()
    mean_op = ops["selective_scan_mean"]

    def spy(x, dt, A, B, C):
        seen.append(dt.min().item())
        return mean_op(x, dt, A, B, C)

    ops["selective_scan_mean"] = spy
    blocks.mamba_model(w, w["input.state_sequence"], ops)
    assert min(seen) > 0.1
    ops["selective_scan_mean"] = lambda x, dt, A, B, C: torch.from_numpy(
        scans.selective_scan(x.numpy(), dt.numpy(), A.numpy(), B.numpy(), C.numpy(), mode="channel"))
    out = blocks.mamba_model(w, w["input.state_sequence"], ops)
    assert (out - w["expected_output"]).abs().max().item() < 1e-4


def test_delta_net_fixture_gradient_is_degenerate_but_consistent():
    """gradient.input of the DeltaNet fixture (generate_random_weight_fixtures.py:516-541)
    is the gradient of sum(final LayerNorm output) with unit gamma, which is ~0; it is
    reproduced, but cannot pin the delta-rule backward (autograd tests do that)."""
    w = blocks.load_fixture(os.path.join(GOLDEN, "delta_net_random.safetensors"))
    x = w["input.state_sequence"].clone().requires_grad_(True)
    blocks.delta_net_model(w, x, blocks.oracle_ops()).sum().backward()
    assert (x.grad - w["gradient.input"]).abs().max().item() < 1e-5


# ---------------------------------------------------------------------------
# known answers from the reference tests
# ---------------------------------------------------------------------------

def test_mingru_seq1_known_answer():
    """backward_kernels_test.exs:271-287."""
    z = np.array([[[0.3, 0.7]]])
    cand = np.array([[[2.0, -1.0]]])
    h0 = np.zeros((1, 2))
    fwd = scans.mingru_scan(z, cand, h0)
    np.testing.assert_allclose(fwd, [[[0.6, -0.7]]], atol=1e-12)
    dz, dc, dh0 = scans.mingru_scan_backward(z, cand, h0, fwd, np.ones((1, 1, 2)))
    np.testing.assert_allclose(dz, [[[2.0, -1.0]]], atol=1e-12)
    np.testing.assert_allclose(dc, [[[0.3, 0.7]]], atol=1e-12)
    np.testing.assert_allclose(dh0, [[0.7, 0.3]], atol=1e-12)


def test_linear_scan_seq1_known_answer_via_mingru():
    """backward_kernels_test.exs:76-93 (h = a h + b with a=0.5, b=1): MinGRU with
    1-z = a and z cand = b gives dh0 = a = 0.5 and d(b) = 1."""
    z = np.array([[[0.5]]])
    cand = np.array([[[2.0]]])  # z * cand = 1
    h0 = np.zeros((1, 1))
    fwd = scans.mingru_scan(z, cand, h0)
    assert fwd[0, 0, 0] == pytest.approx(1.0)
    _, dc, dh0 = scans.mingru_scan_backward(z, cand, h0, fwd, np.ones((1, 1, 1)))
    assert dh0[0, 0] == pytest.approx(0.5)
    assert dc[0, 0, 0] / z[0, 0, 0] == pytest.approx(1.0)


def test_linear_scan_seq1_known_answer():
    """backward_kernels_test.exs:76-95: a = 0.5, b = 1, h0 = 0 -> h = 1, da = 0, db = 1,
    dh0 = 0.5."""
    a, b, h0 = np.array([[[0.5]]]), np.array([[[1.0]]]), np.zeros((1, 1))
    fwd = scans.linear_scan(a, b, h0)
    assert fwd[0, 0, 0] == 1.0
    da, db, dh0 = scans.linear_scan_backward(a, h0, fwd, np.ones((1, 1, 1)))
    assert (da[0, 0, 0], db[0, 0, 0], dh0[0, 0]) == (0.0, 1.0, 0.5)


# ---------------------------------------------------------------------------
# invariants / closed forms
# ---------------------------------------------------------------------------

def test_mingru_invariants(rng):
    cand = rng.normal(size=(2, 9, 5))
    h0 = rng.normal(size=(2, 5))
    np.testing.assert_allclose(scans.mingru_scan(np.ones_like(cand), cand, h0), cand)
    np.testing.assert_allclose(scans.mingru_scan(np.zeros_like(cand), cand, h0),
                               np.broadcast_to(h0[:, None], cand.shape))
    # closed form h_T = sum_s prod_{r>s}(1-z_r) z_s c_s + prod_r (1-z_r) h0
    z = rng.uniform(size=cand.shape)
    h = scans.mingru_scan(z, cand, h0)
    T = cand.shape[1]
    expect = np.prod(1 - z, axis=1) * h0
    for s in range(T):
        expect = expect + np.prod(1 - z[:, s + 1:], axis=1) * z[:, s] * cand[:, s]
    np.testing.assert_allclose(h[:, -1], expect, rtol=1e-12)


def test_linear_scan_invariants(rng):
    b = rng.normal(size=(2, 9, 5))
    h0 = rng.normal(size=(2, 5))
    # a = 1: cumulative sum from h0;  a = 0: h_t = b_t
    np.testing.assert_allclose(scans.linear_scan(np.ones_like(b), b, h0), h0[:, None] + np.cumsum(b, axis=1),
                               rtol=1e-12)
    np.testing.assert_allclose(scans.linear_scan(np.zeros_like(b), b, h0), b)
    # a constant alpha, b constant beta, h0 = 0: h_t = beta (1 - alpha^(t+1)) / (1 - alpha)
    alpha, beta = 0.7, -1.3
    out = scans.linear_scan(np.full((1, 12, 1), alpha), np.full((1, 12, 1), beta))
    t = np.arange(12)
    np.testing.assert_allclose(out[0, :, 0], beta * (1 - alpha ** (t + 1)) / (1 - alpha), rtol=1e-12)
    # a = 1 - z, b = z c is MinGRU (forward and backward)
    z = rng.uniform(0.05, 0.95, size=b.shape)
    fwd = scans.linear_scan(1 - z, z * b, h0)
    np.testing.assert_allclose(fwd, scans.mingru_scan(z, b, h0), rtol=1e-12)
    dy = rng.normal(size=b.shape)
    da, db, dh0 = scans.linear_scan_backward(1 - z, h0, fwd, dy)
    dz, dc, dh0_g = scans.mingru_scan_backward(z, b, h0, fwd, dy)
    np.testing.assert_allclose(db * z, dc, rtol=1e-12)  # d/dc = db dz c/dc
    np.testing.assert_allclose(-da + db * b, dz, rtol=1e-10, atol=1e-12)  # d/dz = -da + db c
    np.testing.assert_allclose(dh0, dh0_g, rtol=1e-12)


def _block_weights(rng, hid, layers, scale=0.3, nproj=2):
    return rng.normal(scale=scale, size=layers * (nproj * (hid * hid + hid) + 2 * hid))


@pytest.mark.parametrize("kind", ["mingru", "minlstm", "linear"])
def test_block_formulations_agree(rng, kind):
    """Layer-parallel restatement (the reference fallbacks) == the per-timestep walk of the
    reference kernels (fused_*_block_scan.cu)."""
    x = rng.normal(size=(2, 7, 6))
    w = _block_weights(rng, 6, 3, nproj=scans.BLOCK_PROJECTIONS[kind])
    h0 = rng.normal(size=(2, 3, 6))
    np.testing.assert_allclose(scans.block(kind, x, w, h0, 3), scans.block_stepwise(kind, x, w, h0, 3),
                               rtol=1e-12, atol=1e-12)


def test_minlstm_and_linear_block_one_layer_written_out(rng):
    hid = 4
    x = rng.normal(size=(2, 5, hid))
    h0 = rng.normal(size=(2, 1, hid))
    mean = x.mean(-1, keepdims=True)
    sd = np.sqrt(x.var(-1, keepdims=True) + 1e-5)

    def proj(w, k):
        o = k * (hid * hid + hid)
        return w[o:o + hid * hid].reshape(hid, hid), w[o + hid * hid:o + hid * hid + hid]

    w3 = _block_weights(rng, hid, 1, nproj=3)
    gamma, beta = w3[3 * 20:3 * 20 + hid], w3[3 * 20 + hid:]
    n = (x - mean) / sd * gamma + beta
    (wf, bf), (wi, bi), (wh, bh) = proj(w3, 0), proj(w3, 1), proj(w3, 2)
    expect = x + scans.minlstm_scan(scans.sigmoid(n @ wf + bf), scans.sigmoid(n @ wi + bi), n @ wh + bh, h0[:, 0])
    np.testing.assert_allclose(scans.block("minlstm", x, w3, h0, 1), expect, rtol=1e-12)
    w2 = _block_weights(rng, hid, 1, nproj=2)
    gamma, beta = w2[2 * 20:2 * 20 + hid], w2[2 * 20 + hid:]
    n = (x - mean) / sd * gamma + beta
    (wa, ba), (wb, bb) = proj(w2, 0), proj(w2, 1)
    expect = x + scans.linear_scan(n @ wa + ba, n @ wb + bb, h0[:, 0])
    np.testing.assert_allclose(scans.block("linear", x, w2, h0, 1), expect, rtol=1e-12)


def test_mingru_block_one_layer_written_out(rng):
    x = rng.normal(size=(2, 5, 4))
    w = _block_weights(rng, 4, 1)
    h0 = rng.normal(size=(2, 1, 4))
    wz, bz, wh, bh, gamma, beta = (w[0:16].reshape(4, 4), w[16:20], w[20:36].reshape(4, 4), w[36:40], w[40:44],
                                   w[44:48])
    mean = x.mean(-1, keepdims=True)
    sd = np.sqrt(x.var(-1, keepdims=True) + 1e-5)
    n = (x - mean) / sd * gamma + beta
    expect = x + scans.mingru_scan(scans.sigmoid(n @ wz + bz), n @ wh + bh, h0[:, 0])
    np.testing.assert_allclose(scans.mingru_block(x, w, h0, 1), expect, rtol=1e-12)
    # L layers == one layer applied L times with that layer's slice of weights and h0
    w2 = _block_weights(rng, 4, 2)
    h02 = rng.normal(size=(2, 2, 4))
    y = scans.mingru_block(x, w2[:48], h02[:, :1], 1)
    y = scans.mingru_block(y, w2[48:], h02[:, 1:], 1)
    np.testing.assert_allclose(scans.mingru_block(x, w2, h02, 2), y, rtol=1e-12)


def test_mingru_block_zero_projection_closed_form(rng):
    """W = 0: z = sigmoid(b_z), c = b_h for every step, so one layer gives
    h_t = b_h + (1 - z)^(t+1) (h0 - b_h) and out = x + h."""
    hid = 3
    x = rng.normal(size=(1, 6, hid))
    w = np.zeros(2 * hid * hid + 4 * hid)
    bz, bh = rng.normal(size=hid), rng.normal(size=hid)
    w[hid * hid:hid * hid + hid] = bz
    w[2 * hid * hid + hid:2 * hid * hid + 2 * hid] = bh
    w[2 * hid * hid + 2 * hid:2 * hid * hid + 3 * hid] = 1.0  # gamma
    h0 = rng.normal(size=(1, 1, hid))
    z = scans.sigmoid(bz)
    t = np.arange(6)[:, None]
    h = bh + (1 - z) ** (t + 1) * (h0[0, 0] - bh)
    np.testing.assert_allclose(scans.mingru_block(x, w, h0, 1)[0], x[0] + h, rtol=1e-12)


def test_minlstm_invariants(rng):
    f = rng.uniform(0.05, 1, size=(2, 7, 4))
    i = rng.uniform(0.05, 1, size=(2, 7, 4))
    cand = rng.normal(size=f.shape)
    h0 = rng.normal(size=(2, 4))
    # i == 0 -> state constant (f' = f/(f+eps) ~ 1)
    out = scans.minlstm_scan(f, np.zeros_like(i), cand, h0)
    np.testing.assert_allclose(out, np.broadcast_to(h0[:, None], out.shape), rtol=1e-4)
    # T = 1 closed form
    o1 = scans.minlstm_scan(f[:, :1], i[:, :1], cand[:, :1], h0)
    s = f[:, 0] + i[:, 0] + 1e-6
    np.testing.assert_allclose(o1[:, 0], f[:, 0] / s * h0 + i[:, 0] / s * cand[:, 0])


def test_selective_scan_invariants(rng):
    bsz, T, D, N = 2, 11, 6, 4
    x = rng.normal(size=(bsz, T, D))
    dt = rng.uniform(0.0, 0.2, size=(bsz, T, D))
    A = -np.exp(rng.uniform(0, np.log(16), size=(D, N)))
    B = rng.normal(size=(bsz, T, N))
    C = rng.normal(size=(bsz, T, N))
    Dv = rng.normal(size=D)
    z = rng.normal(size=x.shape)
    # B == 0 -> y == 0 (and with D, z: y == D x silu(z))
    np.testing.assert_allclose(scans.selective_scan(x, dt, A, np.zeros_like(B), C), 0)
    np.testing.assert_allclose(scans.selective_scan(x, dt, A, np.zeros_like(B), C, Dv, z),
                               Dv * x * z / (1 + np.exp(-z)), rtol=1e-12)
    # N = 1, A = 0 -> y_t = C_t sum_{s<=t} clip(dt_s) B_s x_s
    y = scans.selective_scan(x, dt, np.zeros((D, 1)), B[..., :1], C[..., :1])
    dtc = np.clip(dt, 1e-3, 0.1)
    expect = C[..., :1] * np.cumsum(dtc * B[..., :1] * x, axis=1)
    np.testing.assert_allclose(y, expect, rtol=1e-12)
    # the reference kernel restatement at one step: y = C . (clip(dt) B x)
    y1 = scans.selective_scan(x[:, :1], dt[:, :1], A, B[:, :1], C[:, :1])
    np.testing.assert_allclose(y1[:, 0], dtc[:, 0] * x[:, 0] * (B[:, 0] * C[:, 0]).sum(-1)[:, None])


def test_selective_scan_clip_mask(rng):
    bsz, T, D, N = 1, 6, 5, 4
    x = rng.normal(size=(bsz, T, D))
    dt = rng.uniform(0.0, 0.2, size=(bsz, T, D))
    dt[0, 0, 0] = 1e-5
    dt[0, 1, 1] = 0.5
    A = -np.ones((D, N))
    B, C = rng.normal(size=(bsz, T, N)), rng.normal(size=(bsz, T, N))
    g = scans.selective_scan_backward(x, dt, A, B, C, np.ones_like(x))
    out_of_range = (dt < 1e-3) | (dt > 0.1)
    assert np.all(g["ddt"][out_of_range] == 0)
    assert np.all(g["ddt"][~out_of_range] != 0)


def test_delta_rule_invariants(rng):
    bsz, T, H, d = 2, 5, 3, 4
    q = rng.normal(size=(bsz, T, H, d))
    k = scans.l2_normalize_keys(rng.normal(size=(bsz, T, H, d)))
    v = rng.normal(size=(bsz, T, H, d))
    beta = rng.uniform(size=(bsz, T, H, d))
    alpha = rng.uniform(0.5, 1, size=(bsz, T, H))
    np.testing.assert_allclose(scans.delta_rule(q, k, v, np.zeros_like(beta)), 0)
    np.testing.assert_allclose(scans.delta_rule(q, k, v, beta, np.ones((bsz, T, H))),
                               scans.delta_rule(q, k, v, beta))
    # T = 1: o = (beta * v) (k . q)  (||k|| ~ 1, S0 = 0)
    o1 = scans.delta_rule(q[:, :1], k[:, :1], v[:, :1], beta[:, :1], alpha[:, :1])
    np.testing.assert_allclose(o1[:, 0], beta[:, 0] * v[:, 0] * (k[:, 0] * q[:, 0]).sum(-1, keepdims=True))
    # per-head beta == per-element beta broadcast
    bh = rng.uniform(size=(bsz, T, H))
    np.testing.assert_allclose(scans.delta_rule(q, k, v, bh, alpha),
                               scans.delta_rule(q, k, v, np.repeat(bh[..., None], d, -1), alpha))
    # a key stored with beta = 1 is retrieved exactly: S k = v after the update
    o = scans.delta_rule(k[:, :1], k[:, :1], v[:, :1], np.ones_like(beta[:, :1]))
    np.testing.assert_allclose(o[:, 0], v[:, 0] * (k[:, 0] ** 2).sum(-1, keepdims=True), rtol=1e-12)


def _gdn_two_step(q, k, v, beta, alpha):
    """GatedDeltaNet at T = 2 written out from gated_delta_net.ex:322-344 (S0 = 0), in torch.

    Step 1 stores S1 = (beta1 v1) k1^T (decaying the empty state does nothing).  Step 2
    decays BEFORE the retrieval: s_gated = alpha2 S1 (:327), retrieval = s_gated k2
    (:330-332), S2 = s_gated + (beta2 (v2 - retrieval)) k2^T (:335-338), o2 = S2 q2
    (:341-344), so
        o1 = beta1 v1 (k1.q1)
        o2 = alpha2 beta1 v1 (k1.q2) + beta2 (v2 - alpha2 beta1 v1 (k1.k2)) (k2.q2).
    q, k, v, beta: [B, 2, H, d] (beta may be [B, 2, H]); alpha: [B, 2, H]."""
    if beta.dim() == 3:
        beta = beta[..., None].expand(v.shape)

    def dot(a, b):
        return (a * b).sum(-1, keepdim=True)

    q1, q2, k1, k2, v1, v2 = q[:, 0], q[:, 1], k[:, 0], k[:, 1], v[:, 0], v[:, 1]
    b1, b2, a2 = beta[:, 0], beta[:, 1], alpha[:, 1, :, None]
    o1 = b1 * v1 * dot(k1, q1)
    o2 = a2 * b1 * v1 * dot(k1, q2) + b2 * (v2 - a2 * b1 * v1 * dot(k1, k2)) * dot(k2, q2)
    return torch.stack([o1, o2], dim=1)


@pytest.mark.parametrize("beta_per_head", [False, True])
def test_gated_delta_rule_two_step_closed_form(rng, beta_per_head):
    """Pins the GatedDeltaNet decay order (decay, then retrieve from the decayed state) and,
    through torch autograd of the written-out closed form, every gradient of the oracle's
    backward at T = 2.  alpha2 != 1 and per-element beta make the alternative orders
    (retrieve from the undecayed state; decay after the update) differ visibly."""
    bsz, H, d = 2, 3, 4
    q, k, v = (rng.normal(size=(bsz, 2, H, d)) for _ in range(3))
    beta = rng.uniform(0.2, 0.9, size=(bsz, 2, H) if beta_per_head else (bsz, 2, H, d))
    alpha = rng.uniform(0.3, 0.7, size=(bsz, 2, H))
    do = rng.normal(size=(bsz, 2, H, d))
    tq, tk, tv, tb, ta = (torch.tensor(a, dtype=torch.float64, requires_grad=True)
                          for a in (q, k, v, beta, alpha))
    closed = _gdn_two_step(tq, tk, tv, tb, ta)
    np.testing.assert_allclose(scans.delta_rule(q, k, v, beta, alpha), closed.detach().numpy(),
                               rtol=1e-12, atol=1e-12)

    # the closed form tells the orders apart: retrieval from the undecayed state differs
    b4 = np.broadcast_to(beta[..., None], v.shape) if beta_per_head else beta
    kk = (k[:, 0] * k[:, 1]).sum(-1, keepdims=True)
    kq = (k[:, 1] * q[:, 1]).sum(-1, keepdims=True)
    undecayed_retrieval = (alpha[:, 1, :, None] * b4[:, 0] * v[:, 0] * (k[:, 0] * q[:, 1]).sum(-1, keepdims=True)
                           + b4[:, 1] * (v[:, 1] - b4[:, 0] * v[:, 0] * kk) * kq)
    assert np.abs(undecayed_retrieval - closed.detach().numpy()[:, 1]).max() > 1e-2

    closed.backward(torch.from_numpy(do))
    g = scans.delta_rule_backward(q, k, v, beta, do, alpha)
    for name, t in (("dq", tq), ("dk", tk), ("dv", tv), ("dbeta", tb), ("dalpha", ta)):
        np.testing.assert_allclose(g[name], t.grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)


def _ss_mean_two_step(x, dt, A, B, C):
    """The block CPU (dt-mean) selective scan at T = 2 written out from common.ex:402-445
    (discretize_ssm), :492-513 (sequential_scan, h[-1] = 0) and :462-471
    (compute_ssm_output), in torch, with an arbitrary A[d, n] in place of the block's
    fixed -(1..N):
      clip first (:413): c = clip(dt, 1e-3, 0.1); m_t = mean_d c_t (:439-441)
      h1 = m1 B1 x1;  h2 = exp(c2 A) h1 + m2 B2 x2;  y_t = sum_n C_t,n h_t,n
    x, dt: [B, 2, D]; A: [D, N]; B, C: [B, 2, N]."""
    c = dt.clamp(scans.DT_MIN, scans.DT_MAX)
    m = c.mean(dim=2, keepdim=True)  # [B, 2, 1]
    h1 = m[:, 0, :, None] * B[:, 0, None, :] * x[:, 0, :, None]  # [B, D, N]
    h2 = torch.exp(c[:, 1, :, None] * A[None]) * h1 + m[:, 1, :, None] * B[:, 1, None, :] * x[:, 1, :, None]
    y1 = (C[:, 0, None, :] * h1).sum(-1)
    y2 = (C[:, 1, None, :] * h2).sum(-1)
    return torch.stack([y1, y2], dim=1)


def test_selective_scan_mean_mode_closed_forms(rng):
    """Pins the dt-mean mode: (1) with A = 0, y_t,d = sum_n C_t,n sum_{s<=t} m_s B_s,n x_s,d
    over a long sequence; (2) at T = 2 with A != 0, the decay uses each channel's own clipped
    dt while the input term uses the channel mean of the clipped dt — forward and (torch
    autograd of the written-out form) every gradient.  dt spreads over [1e-3, 0.1] with a few
    values outside it, so the clip acts before the mean and mean mode differs from channel
    mode."""
    bsz, D, N = 2, 6, 3
    # (1) A = 0 over T = 9
    T = 9
    x = rng.normal(size=(bsz, T, D))
    dt = rng.uniform(0.002, 0.095, size=(bsz, T, D))
    dt[0, 2, 1], dt[1, 4, 3] = 0.4, 1e-4  # clipped to 0.1 and 1e-3 before the mean
    B, C = rng.normal(size=(bsz, T, N)), rng.normal(size=(bsz, T, N))
    m = np.clip(dt, 1e-3, 0.1).mean(axis=2)  # [B, T]
    acc = np.cumsum(m[:, :, None, None] * B[:, :, None, :] * x[:, :, :, None], axis=1)  # [B,T,D,N]
    want = np.einsum("btdn,btn->btd", acc, C)
    got = scans.selective_scan(x, dt, np.zeros((D, N)), B, C, mode="mean")
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    chan = scans.selective_scan(x, dt, np.zeros((D, N)), B, C, mode="channel")
    assert np.abs(chan - got).max() > 1e-2 * np.abs(got).max()

    # (2) T = 2, arbitrary negative A, forward and gradients
    x2 = rng.normal(size=(bsz, 2, D))
    dt2 = rng.uniform(0.002, 0.095, size=(bsz, 2, D))
    dt2[0, 1, 2] = 0.3
    A = -np.exp(rng.uniform(0.0, np.log(16.0), size=(D, N)))
    B2, C2 = rng.normal(size=(bsz, 2, N)), rng.normal(size=(bsz, 2, N))
    dy = rng.normal(size=(bsz, 2, D))
    tx, tdt, tA, tB, tC = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x2, dt2, A, B2, C2))
    closed = _ss_mean_two_step(tx, tdt, tA, tB, tC)
    np.testing.assert_allclose(scans.selective_scan(x2, dt2, A, B2, C2, mode="mean"),
                               closed.detach().numpy(), rtol=1e-12, atol=1e-12)
    closed.backward(torch.from_numpy(dy))
    g = scans.selective_scan_backward(x2, dt2, A, B2, C2, dy, mode="mean")
    for name, t in (("dx", tx), ("ddt", tdt), ("dA", tA), ("dB", tB), ("dC", tC)):
        np.testing.assert_allclose(g[name], t.grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)
    assert g["ddt"][0, 1, 2] == 0.0  # clipped entry gets no gradient


def test_flash_attention_matches_sdpa_and_invariants(rng):
    bsz, H, T, d = 2, 3, 7, 8
    q, k, v = (rng.normal(size=(bsz, H, T, d)) for _ in range(3))
    for causal in (False, True):
        o = scans.flash_attention(q, k, v, causal)
        ref = torch.nn.functional.scaled_dot_product_attention(
            *(torch.from_numpy(t) for t in (q, k, v)), is_causal=causal).numpy()
        np.testing.assert_allclose(o, ref, rtol=1e-10, atol=1e-12)
    oc = scans.flash_attention(q, k, v, True)
    np.testing.assert_allclose(oc[:, :, 0], v[:, :, 0])  # causal row 0 sees only key 0
    same_k = np.broadcast_to(k[:, :, :1], k.shape)
    np.testing.assert_allclose(scans.flash_attention(q, same_k, v, False),
                               np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape))
    _, lse = scans.flash_attention(q, k, v, True, return_lse=True)
    s = np.einsum("bhid,bhjd->bhij", q, k) / np.sqrt(d)
    np.testing.assert_allclose(lse[:, :, 0], s[:, :, 0, 0])


def test_fox_attention_invariants(rng):
    """cs constant ==> causal attention; a shift of cs changes nothing; d cs sums to zero
    over the sequence (every score's gradient enters once with + and once with -)."""
    b, h, t, d = 1, 2, 7, 4
    q, k, v, do = (rng.normal(size=(b, h, t, d)) for _ in range(4))
    cs = np.cumsum(-np.abs(rng.normal(size=(b, h, t))), axis=-1)
    np.testing.assert_allclose(scans.fox_attention(q, k, v, np.full((b, h, t), 3.0)),
                               scans.flash_attention(q, k, v, causal=True), rtol=1e-12)
    np.testing.assert_allclose(scans.fox_attention(q, k, v, cs + 5.0), scans.fox_attention(q, k, v, cs), rtol=1e-12)
    dcs = scans.fox_attention_backward(q, k, v, cs, do)[3]
    np.testing.assert_allclose(dcs.sum(-1), 0.0, atol=1e-12)


def test_laser_attention_identical_rows(rng):
    """All value rows equal c: exp(V - vmax) = 1 for every key, so O = c for any weights."""
    b, h, t, d = 1, 1, 6, 3
    q, k = rng.normal(size=(b, h, t, d)), rng.normal(size=(b, h, t, d))
    row = rng.normal(size=d)
    v = np.broadcast_to(row, (b, h, t, d)).copy()
    np.testing.assert_allclose(scans.laser_attention(q, k, v, causal=True), v, rtol=1e-12, atol=1e-12)


def test_kda_reduces_to_deltanet_and_gated(rng):
    """KDA with alpha = 0 is DeltaNet; with every row sharing log decay c it is
    GatedDeltaNet with alpha = exp(c)."""
    bsz, t, h, d = 1, 6, 2, 4
    q, k, v = (rng.normal(size=(bsz, t, h, d)) for _ in range(3))
    beta = rng.uniform(0.1, 0.9, size=(bsz, t, h))
    np.testing.assert_allclose(scans.kda_scan(q, k, v, np.zeros((bsz, t, h, d)), beta),
                               scans.delta_rule(q, k, v, beta), rtol=1e-12)
    c = -rng.uniform(0.05, 0.5, size=(bsz, t, h))
    np.testing.assert_allclose(scans.kda_scan(q, k, v, np.broadcast_to(c[..., None], (bsz, t, h, d)), beta),
                               scans.delta_rule(q, k, v, beta, np.exp(c)), rtol=1e-12)



def _dp_reference_form(q, k, v, beta):
    """DeltaProduct written literally as the reference states it, in its own [key][value]
    state: S = (I - beta kn kn^T) S + beta kn v^T per sub-step, o = RMS_norm(S q)."""
    bsz, t, nhh, h, d = k.shape
    out = np.empty(q.shape)
    for b in range(bsz):
        for hh in range(h):
            S = np.zeros((d, d))
            for s in range(t):
                for j in range(nhh):
                    kv = k[b, s, j, hh]
                    kn = kv / np.sqrt(kv @ kv + 1e-6)
                    be = beta[b, s, j, hh]
                    S = (np.eye(d) - be * np.outer(kn, kn)) @ S + be * np.outer(kn, v[b, s, j, hh])
                o = S @ q[b, s, hh]
                out[b, s, hh] = o / np.sqrt(np.mean(o * o) + 1e-6)
    return out


def test_delta_product_matches_reference_matrix_form(rng):
    """The oracle's row-wise update in the [value][key] state against the reference's own
    matrix statement (fused_delta_product_scan.cu:1-13, delta_product.ex:333-343)."""
    bsz, t, nhh, h, d = 2, 5, 3, 2, 4
    q = rng.normal(size=(bsz, t, h, d))
    k, v = (rng.normal(size=(bsz, t, nhh, h, d)) for _ in range(2))
    beta = rng.uniform(0.1, 1.9, size=(bsz, t, nhh, h))
    np.testing.assert_allclose(scans.delta_product(q, k, v, beta), _dp_reference_form(q, k, v, beta),
                               rtol=1e-11, atol=1e-12)


def test_delta_product_one_step_closed_form(rng):
    """One token, one sub-step from S = 0: S_ref = beta kn v^T, so S_ref q = beta (v . q) kn
    and out = c kn / sqrt(c^2 mean(kn^2) + 1e-6) with c = beta (v . q): the output follows
    the KEY, which a contraction over the wrong state axis would not give."""
    d = 6
    q, k, v = rng.normal(size=(1, 1, 1, d)), rng.normal(size=(1, 1, 1, 1, d)), rng.normal(size=(1, 1, 1, 1, d))
    beta = np.full((1, 1, 1, 1), 0.7)
    kn = k[0, 0, 0, 0] / np.sqrt(k[0, 0, 0, 0] @ k[0, 0, 0, 0] + 1e-6)
    c = 0.7 * (v[0, 0, 0, 0] @ q[0, 0, 0])
    np.testing.assert_allclose(scans.delta_product(q, k, v, beta)[0, 0, 0],
                               c * kn / np.sqrt(c * c * np.mean(kn * kn) + 1e-6), rtol=1e-12)


def test_delta_product_reduces_to_delta_rule(rng):
    """n_h = 1 runs the delta rule's states (normalized keys, per-head beta); a second
    sub-step with beta = 0 is the identity."""
    bsz, t, h, d = 1, 6, 2, 4
    q = rng.normal(size=(bsz, t, h, d))
    k, v = rng.normal(size=(bsz, t, 1, h, d)), rng.normal(size=(bsz, t, 1, h, d))
    beta = rng.uniform(0.1, 0.9, size=(bsz, t, 1, h))
    _, states = scans.delta_rule(q, scans.l2_normalize_keys(k[:, :, 0]), v[:, :, 0], beta[:, :, 0],
                                 return_states=True)
    raw = np.einsum("bthij,bthi->bthj", states, q)
    np.testing.assert_allclose(scans.delta_product(q, k, v, beta, return_raw=True)[1], raw, rtol=1e-12)
    k2 = np.concatenate([k, rng.normal(size=k.shape)], axis=2)
    v2 = np.concatenate([v, rng.normal(size=v.shape)], axis=2)
    b2 = np.concatenate([beta, np.zeros_like(beta)], axis=2)
    np.testing.assert_allclose(scans.delta_product(q, k2, v2, b2), scans.delta_product(q, k, v, beta), rtol=1e-12)


def _rla_inputs(rng, bsz=1, t=6, h=2, d=4):
    q, k, v = (rng.normal(size=(bsz, t, h, d)) for _ in range(3))
    alpha, beta, gamma = (rng.uniform(0.3, 0.95, size=(bsz, t, h)) for _ in range(3))
    return q, k, v, alpha, beta, gamma


def test_rla_without_residual_is_decayed_linear_attention(rng):
    """RLA with gamma = 0 is S_t = a_t S + b_t v_t k_t^T, so
    o_t = sum_{s<=t} (prod_{u=s+1..t} a_u) b_s (k_s . q_t) v_s."""
    q, k, v, alpha, beta, _ = _rla_inputs(rng)
    bsz, t, h, d = q.shape
    want = np.zeros_like(q)
    for tt in range(t):
        for s in range(tt + 1):
            w = np.prod(alpha[:, s + 1:tt + 1], axis=1) * beta[:, s] * (k[:, s] * q[:, tt]).sum(-1)
            want[:, tt] += w[..., None] * v[:, s]
    np.testing.assert_allclose(scans.rla_scan(q, k, v, alpha, beta, np.zeros_like(beta), 0), want, rtol=1e-12)


def test_rdn_reduces_to_delta_rule(rng):
    """RDN with alpha = 1 and gamma = 0 is DeltaNet with a per-head beta."""
    q, k, v, _, beta, _ = _rla_inputs(rng)
    np.testing.assert_allclose(scans.rla_scan(q, k, v, np.ones_like(beta), beta, np.zeros_like(beta), 1),
                               scans.delta_rule(q, k, v, beta), rtol=1e-12)


@pytest.mark.parametrize("variant", [0, 1])
def test_rla_zero_clip_keeps_residual_empty(rng, variant):
    """clip threshold 0: the residual error is 0, R stays 0 and the output is the gamma = 0
    one; a huge threshold differs from it (the residual state is live)."""
    q, k, v, alpha, beta, gamma = _rla_inputs(rng)
    base = scans.rla_scan(q, k, v, alpha, beta, np.zeros_like(gamma), variant)
    np.testing.assert_allclose(scans.rla_scan(q, k, v, alpha, beta, gamma, variant, clip=0.0), base, rtol=1e-12)
    assert np.abs(scans.rla_scan(q, k, v, alpha, beta, gamma, variant, clip=1e9) - base).max() > 1e-3


def test_ttt_closed_forms(rng):
    """eta = 0: W stays w0, so o_t = w0 q_t.  w0 = 0, one step: pred = 0 normalizes to 0,
    so err = ln_b - v and o = -(eta (ln_b - v)) (k . q)."""
    bsz, t, d = 2, 5, 6
    q, k, v = (rng.normal(size=(bsz, t, d)) for _ in range(3))
    w0 = rng.normal(size=(bsz, d, d))
    g, b = rng.normal(size=d), rng.normal(size=d)
    np.testing.assert_allclose(scans.ttt_scan(q, k, v, np.zeros((bsz, t, d)), w0, g, b),
                               np.einsum("bij,btj->bti", w0, q), rtol=1e-12)
    eta = rng.uniform(0.0, 0.1, size=(bsz, 1, d))
    got = scans.ttt_scan(q[:, :1], k[:, :1], v[:, :1], eta, np.zeros((bsz, d, d)), g, b)
    want = -(eta[:, 0] * (b - v[:, 0])) * (k[:, 0] * q[:, 0]).sum(-1, keepdims=True)
    np.testing.assert_allclose(got[:, 0], want, rtol=1e-12)


def _rnn_weights(rng, kind, hid, layers, scale=0.3):
    g = scans.RNN_BLOCK_GATES[kind] * hid
    per = []
    for _ in range(layers):
        per += [scale * rng.normal(size=hid * g), scale * rng.normal(size=g), scale * rng.normal(size=hid * g),
                1 + 0.2 * rng.normal(size=hid), 0.2 * rng.normal(size=hid)]
    return np.concatenate(per)


@pytest.mark.parametrize("kind", ["lstm", "gru"])
def test_rnn_block_layerwise_equals_stepwise(rng, kind):
    """The reference's two formulations (fallback layer by layer, kernel step by step) agree."""
    bsz, t, hid, layers = 2, 7, 5, 3
    x = rng.normal(size=(bsz, t, hid))
    w = _rnn_weights(rng, kind, hid, layers)
    h0, c0 = rng.normal(size=(bsz, layers, hid)), rng.normal(size=(bsz, layers, hid))
    np.testing.assert_allclose(scans.rnn_block(kind, x, w, h0, c0, layers),
                               scans.rnn_block_stepwise(kind, x, w, h0, c0, layers), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kind", ["lstm", "gru"])
def test_rnn_block_one_layer_is_torch_rnn(rng, kind):
    """One layer = LayerNorm + torch.nn.LSTM / torch.nn.GRU (gate orders i,f,g,o and r,z,n;
    weight_ih = W_x^T, weight_hh = R^T, no recurrent bias) + residual.  torch's GRU mixes
    h' = (1 - z) n + z h, the reference (1 - z) h + z n, so the z rows are negated
    (sigmoid(-a) = 1 - sigmoid(a))."""
    bsz, t, hid = 2, 6, 4
    x = rng.normal(size=(bsz, t, hid))
    w = _rnn_weights(rng, kind, hid, 1)
    h0, c0 = rng.normal(size=(bsz, 1, hid)), rng.normal(size=(bsz, 1, hid))
    wx, bx, r, gamma, beta = scans._rnn_layer_weights(w, 0, hid, scans.RNN_BLOCK_GATES[kind])
    n = scans._block_norm(x, gamma, beta)
    wih, whh, bih = wx.T.copy(), r.T.copy(), bx.copy()
    if kind == "gru":
        for m in (wih, whh):
            m[hid:2 * hid] *= -1
        bih[hid:2 * hid] *= -1
        net = torch.nn.GRU(hid, hid, batch_first=True).double()
    else:
        net = torch.nn.LSTM(hid, hid, batch_first=True).double()
    with torch.no_grad():
        net.weight_ih_l0.copy_(torch.from_numpy(wih))
        net.weight_hh_l0.copy_(torch.from_numpy(whh))
        net.bias_ih_l0.copy_(torch.from_numpy(bih))
        net.bias_hh_l0.zero_()
        hh = torch.from_numpy(h0.transpose(1, 0, 2).copy())
        init = (hh, torch.from_numpy(c0.transpose(1, 0, 2).copy())) if kind == "lstm" else hh
        y, _ = net(torch.from_numpy(n), init)
    np.testing.assert_allclose(scans.rnn_block(kind, x, w, h0, c0, 1), x + y.numpy(), rtol=1e-10, atol=1e-12)
