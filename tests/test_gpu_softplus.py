"""GPU parity: the HIP softplus (the Mamba block's dt activation) and row L2 normalisation (the
DeltaNet key norm) against float64 torch on the same (rounded) inputs, values and gradient."""
import pytest
import torch

from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host

pytestmark = pytest.mark.gpu

CASES = [
    # (shape, dtype, offset): offset 1 starts the tensor one element into a buffer (scalar path)
    ((8, 2048, 64), torch.bfloat16, 0),   # the config-5 dt width, a slice of the batch
    ((3, 70, 48), torch.float32, 0),
    ((1001,), torch.bfloat16, 0),         # a tail past the last 16-byte vector
    ((517,), torch.float32, 1),
    ((5,), torch.bfloat16, 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_softplus(case):
    from edifice_amd import fused_scan as fs
    shape, dtype, off = case
    announce("softplus", case=case)
    g = torch.Generator().manual_seed(6)
    n = 1
    for d in shape:
        n *= d
    x = torch.randn(n, generator=g) * 4.0 - 2.0
    x[:4] = torch.tensor([-100.0, 100.0, 0.0, 25.0])  # both saturated ends and the threshold region
    x = x.to(dtype)
    dy = torch.randn(n, generator=g).to(dtype)
    buf = torch.zeros(n + off, dtype=dtype, device="cuda")
    buf[off:] = x.cuda()
    xd = buf[off:].view(shape).detach().requires_grad_()
    y = fs.softplus(xd)
    y.backward(dy.view(shape).cuda())
    xr = x.double().view(shape).requires_grad_()
    yr = torch.nn.functional.softplus(xr)
    yr.backward(dy.double().view(shape))
    assert y.dtype == dtype and torch.isfinite(y).all()
    assert_close(host(y), yr.detach().numpy(), TOL[dtype], "y")
    assert_close(host(xd.grad), xr.grad.numpy(), TOL[dtype], "dx")


L2_CASES = [
    # (rows, d, dtype, offset)
    (8 * 2048 * 8, 128, torch.bfloat16, 0),  # the config-5 DeltaNet keys
    (300, 128, torch.float32, 0),
    (77, 64, torch.bfloat16, 0),
    (50, 1000, torch.float32, 0),          # beyond the vector path for f32
    (31, 100, torch.bfloat16, 1),          # misaligned: one element per lane
    (5, 8, torch.float32, 0),
]


@pytest.mark.parametrize("case", L2_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_l2_normalize(case):
    """fs.l2_normalize (the DeltaNet key norm) against float64 torch: values and gradient, with
    a zero row (eps keeps it finite)."""
    from edifice_amd import fused_scan as fs
    rows, d, dtype, off = case
    announce("l2_normalize", case=case)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(rows, d, generator=g) * 3.0
    x[0] = 0.0
    x = x.to(dtype)
    dy = torch.randn(rows, d, generator=g).to(dtype)
    buf = torch.zeros(rows * d + off, dtype=dtype, device="cuda")
    buf[off:] = x.cuda().reshape(-1)
    xd = buf[off:].view(rows, d).detach().requires_grad_()
    y = fs.l2_normalize(xd, 1e-6)
    y.backward(dy.cuda())
    xr = x.double().requires_grad_()
    yr = xr / torch.sqrt((xr * xr).sum(-1, keepdim=True) + 1e-6)
    yr.backward(dy.double())
    assert torch.isfinite(y).all() and torch.isfinite(xd.grad).all()
    assert_close(host(y), yr.detach().numpy(), TOL[dtype], "y")
    assert_close(host(xd.grad), xr.grad.numpy(), TOL[dtype], "dx")


SPLIT_CASES = [
    # (batch, seq, heads, head_dim, dtype, offset)
    (2, 64, 8, 128, torch.bfloat16, 0),   # the config-5 layer's heads
    (1, 37, 2, 64, torch.float32, 0),
    (2, 9, 3, 256, torch.float32, 0),     # four vectors per lane
    (1, 11, 2, 33, torch.float32, 0),     # off the vector: one element per lane
    (1, 5, 2, 128, torch.bfloat16, 1),    # misaligned projection
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_delta_net_split(case):
    """fs.delta_net_split against float64 torch (split, head reshape, per-head key L2 norm with eps
    inside the square root, sigmoid of beta_pre): the four outputs and the projection's
    gradient; q and v are copies (bit-identical) and so are their gradients."""
    from edifice_amd import fused_scan as fs
    bsz, seq, nh, d, dtype, off = case
    announce("delta_net_split", case=case)
    g = torch.Generator().manual_seed(21)
    width = 4 * nh * d
    p = torch.randn(bsz * seq * width, generator=g).to(dtype)
    grads = [torch.randn(bsz, seq, nh, d, generator=g).to(dtype) for _ in range(4)]
    buf = torch.zeros(p.numel() + off, dtype=dtype, device="cuda")
    buf[off:] = p.cuda()
    pd = buf[off:].view(bsz, seq, width).detach().requires_grad_()
    outs = fs.delta_net_split(pd, nh, 1e-6)
    torch.autograd.backward(outs, [t.cuda() for t in grads])
    pr = p.double().view(bsz, seq, width).requires_grad_()
    q, k, v, b = (t.reshape(bsz, seq, nh, d) for t in torch.split(pr, nh * d, dim=-1))
    refs = (q, k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6), v, torch.sigmoid(b))
    torch.autograd.backward(refs, [t.double() for t in grads])
    for name, o, r in zip("qkvb", outs, refs):
        assert o.shape == (bsz, seq, nh, d) and o.dtype == dtype
        assert_close(host(o), r.detach().numpy(), TOL[dtype], name)
    pv = p.view(bsz, seq, width)
    assert torch.equal(outs[0].cpu(), pv[..., : nh * d].reshape(bsz, seq, nh, d))
    assert torch.equal(outs[2].cpu(), pv[..., 2 * nh * d: 3 * nh * d].reshape(bsz, seq, nh, d))
    assert_close(host(pd.grad), pr.grad.numpy(), TOL[dtype], "dproj")
    gp = pd.grad.cpu()
    assert torch.equal(gp[..., : nh * d], grads[0].reshape(bsz, seq, nh * d))
    assert torch.equal(gp[..., 2 * nh * d: 3 * nh * d], grads[2].reshape(bsz, seq, nh * d))
