"""GPU parity: flash attention forward/backward (HIP) vs the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import scans
from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host, rounded, to_dev

pytestmark = pytest.mark.gpu

CASES = [
    # (B, H, T, d, dtype, causal)
    (2, 2, 64, 32, torch.bfloat16, True),
    (1, 2, 200, 64, torch.bfloat16, True),
    (1, 2, 130, 128, torch.bfloat16, False),
    (2, 2, 256, 128, torch.bfloat16, False),  # whole key and query tiles: the unmasked instances
    (1, 2, 160, 128, torch.bfloat16, False),  # whole 32-query tiles, a partial 64-key tile
    (2, 1, 256, 128, torch.bfloat16, True),
    (1, 1, 1, 128, torch.bfloat16, True),
    (1, 3, 33, 24, torch.bfloat16, True),     # odd head_dim: wave-per-row path
    (2, 2, 40, 16, torch.float32, True),
    (1, 2, 77, 64, torch.float32, False),
    (1, 1, 96, 128, torch.float32, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_flash_attention_fwd_bwd(case, rng):
    from edifice_amd import fused_scan as fs
    B, H, T, d, dtype, causal = case
    announce("flash_attention", case=case)
    std = d ** -0.25  # config-4 distribution N(0, 1/sqrt(d))
    q, k, v, do = (rng.normal(scale=std, size=(B, H, T, d)) for _ in range(4))
    tq, tk, tv = (to_dev(a, dtype).requires_grad_() for a in (q, k, v))
    out = fs.flash_attention(tq, tk, tv, causal=causal)
    out.backward(to_dev(do, dtype))
    qr, kr, vr, dor = (rounded(a, dtype) for a in (q, k, v, do))
    tol = TOL[dtype]
    assert_close(host(out), scans.flash_attention(qr, kr, vr, causal), tol, "O", mfma_bf16=True)
    dq, dk, dv = scans.flash_attention_backward(qr, kr, vr, dor, causal)
    if T == 1:
        # One key: O = V[0] exactly, so dP - D = dO . (V[0] - O) = 0 and dQ = dK = 0
        # analytically; the kernel's float32 dP and D (different summation orders) leave a
        # rounding residue, bounded here by the tolerance times the size of one gradient
        # term, sqrt(d) max|dO| max|V| max|K| (a ratio to max |expected| ~ 0 is undefined).
        term = np.sqrt(d) * np.abs(dor).max() * np.abs(vr).max() * max(np.abs(kr).max(), np.abs(qr).max())
        for name, got in (("dQ", host(tq.grad)), ("dK", host(tk.grad))):
            assert np.abs(got).max() <= tol * term, f"{name}: |{name}| {np.abs(got).max():.3e} > {tol * term:.3e}"
    else:
        assert_close(host(tq.grad), dq, tol, "dQ", mfma_bf16=True)
        assert_close(host(tk.grad), dk, tol, "dK", mfma_bf16=True)
    assert_close(host(tv.grad), dv, tol, "dV", mfma_bf16=True)


def test_flash_attention_lse_and_invariants(rng):
    """lse equals logsumexp of the scaled scores; causal row 0 returns V[0];
    identical keys give the mean of V (non-causal)."""
    from edifice_amd import _native as nat
    import ctypes
    announce("flash_lse")
    B, H, T, d = 1, 2, 96, 128
    q, k, v = (rng.normal(scale=0.3, size=(B, H, T, d)) for _ in range(3))
    tq, tk, tv = (to_dev(a, torch.bfloat16) for a in (q, k, v))
    out = torch.empty_like(tq)
    lse = torch.empty(B, H, T, dtype=torch.float32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.call("edf_fused_flash_attention", stream, P(tq), P(tk), P(tv), P(out), P(lse), B, H, T, d, 1, 1)
    qr, kr, vr = (rounded(a, torch.bfloat16) for a in (q, k, v))
    o_ref, lse_ref = scans.flash_attention(qr, kr, vr, True, return_lse=True)
    assert_close(host(lse), lse_ref, 1e-3, "lse")
    assert_close(host(out)[:, :, 0], vr[:, :, 0], TOL[torch.bfloat16], "causal row 0", mfma_bf16=True)
    same_k = tk[:, :, :1].expand(-1, -1, T, -1).contiguous()
    nat.call("edf_fused_flash_attention", stream, P(tq), P(same_k), P(tv), P(out), P(lse), B, H, T, d, 0, 1)
    assert_close(host(out), np.broadcast_to(vr.mean(axis=2, keepdims=True), vr.shape), TOL[torch.bfloat16],
                 "identical keys", mfma_bf16=True)


def test_flash_attention_config4_head_slice(rng):
    """Config-4 sequence length (T=4096, d=128, causal, bf16) on one (b, h) pair:
    forward and gradients against the oracle."""
    from edifice_amd import fused_scan as fs
    B, H, T, d = 1, 1, 4096, 128
    announce("flash_c4_slice")
    q, k, v, do = (rng.normal(scale=d ** -0.25, size=(B, H, T, d)) for _ in range(4))
    tq, tk, tv = (to_dev(a, torch.bfloat16).requires_grad_() for a in (q, k, v))
    out = fs.flash_attention(tq, tk, tv, causal=True)
    out.backward(to_dev(do, torch.bfloat16))
    qr, kr, vr, dor = (rounded(a, torch.bfloat16) for a in (q, k, v, do))
    tol = TOL[torch.bfloat16]
    assert_close(host(out), scans.flash_attention(qr, kr, vr, True), tol, "O", mfma_bf16=True)
    dq, dk, dv = scans.flash_attention_backward(qr, kr, vr, dor, True)
    assert_close(host(tq.grad), dq, tol, "dQ", mfma_bf16=True)
    assert_close(host(tk.grad), dk, tol, "dK", mfma_bf16=True)
    assert_close(host(tv.grad), dv, tol, "dV", mfma_bf16=True)


FOX_CASES = [
    # (B, H, T, d, dtype): the MFMA path (bf16, d = 32/64/128) and the wave-per-row path
    (2, 2, 64, 32, torch.bfloat16),
    (1, 2, 200, 64, torch.bfloat16),
    (2, 1, 256, 128, torch.bfloat16),
    (1, 2, 130, 128, torch.bfloat16),
    (1, 1, 1, 128, torch.bfloat16),
    (1, 3, 33, 24, torch.bfloat16),
    (2, 2, 40, 16, torch.float32),
    (1, 1, 96, 128, torch.float32),
]


@pytest.mark.parametrize("case", FOX_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_fox_attention_fwd_bwd(case, rng):
    """FusedScan.fox_attention/4 and its backward (dq, dk, dv, d cs) against the oracle."""
    from edifice_amd import fused_scan as fs
    B, H, T, d, dtype = case
    announce("fox_attention", case=case)
    std = d ** -0.25
    q, k, v, do = (rng.normal(scale=std, size=(B, H, T, d)) for _ in range(4))
    # cumulative log forget gates, as FoX builds them (sigmoid of logits around +2)
    cs = np.cumsum(-np.log1p(np.exp(-(rng.normal(size=(B, H, T)) + 2.0))), axis=-1)
    tq, tk, tv, tc = (to_dev(a, dtype).requires_grad_() for a in (q, k, v, cs))
    out = fs.fox_attention(tq, tk, tv, tc)
    out.backward(to_dev(do, dtype))
    qr, kr, vr, cr, dor = (rounded(a, dtype) for a in (q, k, v, cs, do))
    tol = TOL[dtype]
    assert_close(host(out), scans.fox_attention(qr, kr, vr, cr), tol, "O", mfma_bf16=True)
    dq, dk, dv, dcs = scans.fox_attention_backward(qr, kr, vr, cr, dor)
    assert_close(host(tq.grad), dq, tol, "dQ", mfma_bf16=True)
    assert_close(host(tk.grad), dk, tol, "dK", mfma_bf16=True)
    assert_close(host(tv.grad), dv, tol, "dV", mfma_bf16=True)
    assert_close(host(tc.grad), dcs, tol, "dcs", mfma_bf16=True)


def test_fox_with_constant_cs_is_causal_flash(rng):
    """cs constant: the bias vanishes and FoX equals causal flash attention exactly (same
    kernels, bias 0)."""
    from edifice_amd import fused_scan as fs
    announce("fox_constant_cs")
    B, H, T, d = 1, 2, 192, 128
    q, k, v = (to_dev(rng.normal(scale=d ** -0.25, size=(B, H, T, d)), torch.bfloat16) for _ in range(3))
    cs = torch.zeros(B, H, T, dtype=torch.bfloat16, device="cuda")
    assert torch.equal(fs.fox_attention(q, k, v, cs), fs.flash_attention(q, k, v, causal=True))


LASER_CASES = [
    # (B, H, T, d, dtype, causal)
    (2, 2, 64, 32, torch.bfloat16, True),
    (1, 2, 200, 128, torch.bfloat16, True),
    (1, 2, 130, 64, torch.bfloat16, False),
    (1, 3, 33, 24, torch.bfloat16, True),
    (2, 2, 40, 16, torch.float32, True),
    (1, 1, 96, 128, torch.float32, False),
]


@pytest.mark.parametrize("case", LASER_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_laser_attention_fwd_bwd(case, rng):
    """FusedScan.laser_attention and its backward against the oracle."""
    from edifice_amd import fused_scan as fs
    B, H, T, d, dtype, causal = case
    announce("laser_attention", case=case)
    std = d ** -0.25
    q, k, do = (rng.normal(scale=std, size=(B, H, T, d)) for _ in range(3))
    # unit-scale values: with values of scale d^-1/4 and near-uniform attention every output
    # is log(mean exp(v)) ~ 0.06, and the tolerance (relative to max |O|) would measure bf16
    # rounding of a near-constant
    v = rng.normal(size=(B, H, T, d))
    tq, tk, tv = (to_dev(a, dtype).requires_grad_() for a in (q, k, v))
    out = fs.laser_attention(tq, tk, tv, causal=causal)
    out.backward(to_dev(do, dtype))
    qr, kr, vr, dor = (rounded(a, dtype) for a in (q, k, v, do))
    tol = TOL[dtype]
    assert_close(host(out), scans.laser_attention(qr, kr, vr, causal), tol, "O", mfma_bf16=True)
    dq, dk, dv = scans.laser_attention_backward(qr, kr, vr, dor, causal)
    # bf16 gradients pass through one more bf16 rounding than the flash ones (E = exp(V - vmax)
    # is an MFMA operand): element-wise 3e-2, still tighter than the reference's own bf16
    # LASER gradient check (absolute 0.05, attention_backward_test.exs:227-229)
    et = 3e-2 if dtype == torch.bfloat16 else None
    assert_close(host(tq.grad), dq, tol, "dQ", elem_tol=et, mfma_bf16=True)
    assert_close(host(tk.grad), dk, tol, "dK", elem_tol=et, mfma_bf16=True)
    assert_close(host(tv.grad), dv, tol, "dV", elem_tol=et, mfma_bf16=True)
