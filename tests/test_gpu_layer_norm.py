"""GPU parity: the HIP layer norm (the block models' pre-norms and final norms) against float64
torch on the same (rounded) inputs: y, dx, dgamma, dbeta."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host

pytestmark = pytest.mark.gpu

CASES = [
    # (leading shape, cols, io dtype, parameter dtype, affine)
    ((8, 2048), 1024, torch.bfloat16, torch.bfloat16, True),   # the config-5 shape, one batch row
    ((3, 70), 1024, torch.float32, torch.float32, True),
    ((5000,), 256, torch.bfloat16, torch.float32, True),       # more rows than the backward's waves
    ((7,), 2048, torch.float32, torch.float32, True),          # eight vectors per lane
    ((9,), 2048, torch.bfloat16, torch.bfloat16, True),        # four vectors per lane
    ((6, 5), 33, torch.float32, torch.float32, True),          # off the vector: row read per pass
    ((4,), 4100, torch.bfloat16, torch.float32, True),         # past the register path
    ((3,), 8192, torch.float32, torch.bfloat16, True),         # the column limit
    ((11,), 96, torch.bfloat16, torch.bfloat16, False),        # no weight, no bias
    ((1,), 8, torch.float32, torch.float32, True),             # one row, one vector
]


def _ref(x, w, b, dy, eps):
    xr = x.double().requires_grad_()
    wr = None if w is None else w.double().requires_grad_()
    br = None if b is None else b.double().requires_grad_()
    y = torch.nn.functional.layer_norm(xr, (x.shape[-1],), wr, br, eps)
    y.backward(dy.double())
    return y, xr.grad, None if wr is None else wr.grad, None if br is None else br.grad


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_layer_norm(case):
    from edifice_amd import fused_scan as fs
    lead, cols, io, par, affine = case
    announce("layer_norm", case=case)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(*lead, cols, generator=g) * 2.0 + 0.5).to(io)
    dy = torch.randn(*lead, cols, generator=g).to(io)
    w = (1.0 + 0.3 * torch.randn(cols, generator=g)).to(par) if affine else None
    b = (0.2 * torch.randn(cols, generator=g)).to(par) if affine else None
    eps = 1e-5
    xd = x.cuda().requires_grad_()
    wd = None if w is None else w.cuda().requires_grad_()
    bd = None if b is None else b.cuda().requires_grad_()
    y = fs.layer_norm(xd, wd, bd, eps)
    y.backward(dy.cuda())
    yr, dxr, dwr, dbr = _ref(x, w, b, dy, eps)
    tol = max(TOL[io], TOL[par])
    assert y.dtype == io and xd.grad.dtype == io
    assert_close(host(y), yr.detach().numpy(), TOL[io], "y")
    assert_close(host(xd.grad), dxr.numpy(), TOL[io], "dx")
    if affine:
        assert wd.grad.dtype == par and bd.grad.dtype == par
        assert_close(host(wd.grad), dwr.numpy(), tol, "dgamma")
        assert_close(host(bd.grad), dbr.numpy(), tol, "dbeta")


def test_layer_norm_matches_nn_layernorm_and_is_deterministic():
    """The blocks' LayerNorm module (nn.LayerNorm's parameters) runs the HIP kernels, gives
    torch's float32 result, and repeated backward passes give bit-identical gradients (fixed
    summation order); a misaligned view takes the any-shape kernels."""
    from edifice_amd import blocks
    from edifice_amd import fused_scan as fs
    announce("layer_norm_module")
    torch.manual_seed(4)
    m = blocks.LayerNorm(1024, eps=1e-5).cuda()
    with torch.no_grad():
        m.weight.uniform_(0.5, 1.5)
        m.bias.uniform_(-0.5, 0.5)
    ref = torch.nn.LayerNorm(1024, eps=1e-5).cuda()
    ref.load_state_dict(m.state_dict())
    x = torch.randn(4, 300, 1024, device="cuda")
    dy = torch.randn_like(x)
    grads = []
    for _ in range(2):
        xd = x.clone().requires_grad_()
        m.zero_grad()
        m(xd).backward(dy)
        grads.append((xd.grad.clone(), m.weight.grad.clone(), m.bias.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    xr = x.clone().requires_grad_()
    yr = ref(xr)
    yr.backward(dy)
    assert_close(host(m(x)), host(yr), TOL[torch.float32], "y vs nn.LayerNorm")
    assert_close(host(grads[0][0]), host(xr.grad), TOL[torch.float32], "dx vs nn.LayerNorm")
    assert_close(host(grads[0][1]), host(ref.weight.grad), TOL[torch.float32], "dgamma vs nn.LayerNorm")
    assert_close(host(grads[0][2]), host(ref.bias.grad), TOL[torch.float32], "dbeta vs nn.LayerNorm")
    # a view one element into a buffer: not 16-byte aligned, so the any-shape kernels run
    buf = torch.randn(1 + 6 * 512, device="cuda")
    xv = buf[1:].view(6, 512)
    w = torch.ones(512, device="cuda")
    yv = fs.layer_norm(xv, w, None, 1e-5)
    assert_close(host(yv), host(torch.nn.functional.layer_norm(xv, (512,), w, None, 1e-5)), TOL[torch.float32],
                 "misaligned view")
    assert np.isfinite(host(yv)).all()


ADD_CASES = [CASES[0], CASES[1], CASES[3], CASES[5], CASES[6], CASES[8]]


@pytest.mark.parametrize("case", ADD_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_add_layer_norm(case):
    """fs.add_layer_norm: the sum bit-identical to torch's add in the io dtype, y the float64
    layer norm of that sum, and the input gradient LN'(dy) + (gradient reaching the sum), the
    same for both addends; the parameter gradients as the plain layer norm's."""
    from edifice_amd import fused_scan as fs
    lead, cols, io, par, affine = case
    announce("add_layer_norm", case=case)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(*lead, cols, generator=g) * 2.0 + 0.5).to(io)
    r = torch.randn(*lead, cols, generator=g).to(io)
    dy = torch.randn(*lead, cols, generator=g).to(io)
    ds = torch.randn(*lead, cols, generator=g).to(io)
    w = (1.0 + 0.3 * torch.randn(cols, generator=g)).to(par) if affine else None
    b = (0.2 * torch.randn(cols, generator=g)).to(par) if affine else None
    eps = 1e-5
    xd, rd = x.cuda().requires_grad_(), r.cuda().requires_grad_()
    wd = None if w is None else w.cuda().requires_grad_()
    bd = None if b is None else b.cuda().requires_grad_()
    s, y = fs.add_layer_norm(xd, rd, wd, bd, eps)
    torch.autograd.backward([s, y], [ds.cuda(), dy.cuda()])
    st = x + r  # torch's add in the io dtype
    assert s.dtype == io and torch.equal(s.cpu(), st)
    yr, dxr, dwr, dbr = _ref(st, w, b, dy, eps)
    tol = max(TOL[io], TOL[par])
    assert_close(host(y), yr.detach().numpy(), TOL[io], "y")
    assert_close(host(xd.grad), (dxr + ds.double()).numpy(), TOL[io], "dx")
    assert torch.equal(xd.grad, rd.grad)
    if affine:
        assert_close(host(wd.grad), dwr.numpy(), tol, "dgamma")
        assert_close(host(bd.grad), dbr.numpy(), tol, "dbeta")


def test_add_layer_norm_one_output_used():
    """Only y used: dx is LN'(dy) alone; only the sum used: its gradient passes through and the
    parameter gradients are zero.  A misaligned addend takes the any-shape kernels."""
    from edifice_amd import fused_scan as fs
    announce("add_layer_norm_one_output")
    torch.manual_seed(6)
    x = torch.randn(5, 256, device="cuda")
    buf = torch.randn(1 + 5 * 256, device="cuda")
    r = buf[1:].view(5, 256)  # not 16-byte aligned
    w = torch.rand(256, device="cuda") + 0.5
    dy = torch.randn(5, 256, device="cuda")
    xd, rd, wd = x.clone().requires_grad_(), r.clone().requires_grad_(), w.clone().requires_grad_()
    _, y = fs.add_layer_norm(xd, r, wd, None, 1e-5)
    y.backward(dy)
    xr, wr = (x + r).requires_grad_(), w.clone().requires_grad_()
    yr = torch.nn.functional.layer_norm(xr, (256,), wr, None, 1e-5)
    yr.backward(dy)
    assert_close(host(y), host(yr), TOL[torch.float32], "y (misaligned addend)")
    assert_close(host(xd.grad), host(xr.grad), TOL[torch.float32], "dx (y only)")
    assert_close(host(wd.grad), host(wr.grad), TOL[torch.float32], "dgamma (y only)")
    xd.grad = None
    wd.grad = None
    s, _ = fs.add_layer_norm(xd, rd, wd, None, 1e-5)
    s.backward(dy)
    assert torch.equal(xd.grad, dy) and torch.equal(rd.grad, dy)
    assert torch.equal(wd.grad, torch.zeros_like(w))
