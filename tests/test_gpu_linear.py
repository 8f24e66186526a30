"""GPU: the blocks' Linear (nn.Linear whose weight gradient splits the row dimension into
slices with float32 partials) against float64 torch, at the config-5 row count."""
import pytest
import torch

from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host

pytestmark = pytest.mark.gpu

CASES = [
    # (rows, in, out, dtype): 8 slices, 4 slices, one product (large output), f32 (one product)
    (16384, 1024, 1024, torch.bfloat16),
    (16384, 1024, 2048, torch.bfloat16),
    (16384, 1024, 32000, torch.bfloat16),
    (16384, 2048, 64, torch.bfloat16),
    (4096, 256, 128, torch.float32),
    (1000, 64, 64, torch.bfloat16),  # rows not divisible into 1024-row slices: one product
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_linear_weight_grad(case):
    from edifice_amd import blocks
    rows, fin, fout, dtype = case
    announce("linear", case=case)
    g = torch.Generator().manual_seed(8)
    lin = blocks.Linear(fin, fout, bias=fout < 32000)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(fout, fin, generator=g) / fin ** 0.5)
        if lin.bias is not None:
            lin.bias.copy_(torch.randn(fout, generator=g))
    lin = lin.to("cuda", dtype)
    x = torch.randn(rows // 8, 8, fin, generator=g).to(dtype)
    dy = torch.randn(rows // 8, 8, fout, generator=g).to(dtype)
    xd = x.cuda().requires_grad_()
    y = lin(xd)
    y.backward(dy.cuda())
    xr = x.double().requires_grad_()
    wr = lin.weight.detach().cpu().double().requires_grad_()
    br = None if lin.bias is None else lin.bias.detach().cpu().double().requires_grad_()
    yr = torch.nn.functional.linear(xr, wr, br)
    yr.backward(dy.double())
    tol = TOL[dtype]
    assert_close(host(y), yr.detach().numpy(), tol, "y", elementwise=False)
    assert_close(host(xd.grad), xr.grad.numpy(), tol, "dx", elementwise=False)
    assert_close(host(lin.weight.grad), wr.grad.numpy(), tol, "dW", elementwise=False)
    if br is not None:
        assert_close(host(lin.bias.grad), br.grad.numpy(), tol, "db", elementwise=False)


COLSUM_CASES = [
    # (rows, cols, dtype, out dtype, offset)
    (16384, 1024, torch.bfloat16, torch.bfloat16, 0),  # the config-5 bias gradients
    (16384, 4096, torch.bfloat16, torch.float32, 0),
    (1000, 301, torch.float32, torch.float32, 0),      # odd width: one element per lane
    (70, 256, torch.bfloat16, torch.bfloat16, 1),      # fewer rows than a slice, misaligned
    (1, 5, torch.float32, torch.bfloat16, 0),
    (8, 1 << 20, torch.float32, torch.bfloat16, 0),  # split-product partials: the one-pass kernel
    (4, 4096, torch.bfloat16, torch.float32, 0),     # one pass, bf16 in
    (32, 1000, torch.float32, torch.float32, 0),     # one pass at its row limit
    (3, 64, torch.float32, torch.bfloat16, 1),       # few rows but misaligned: the sliced kernels
]


@pytest.mark.parametrize("case", COLSUM_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_column_sum(case):
    """fs.column_sum against float64 torch, and bit-identical on a repeated call (fixed order)."""
    from edifice_amd import fused_scan as fs
    rows, cols, dtype, odt, off = case
    announce("column_sum", case=case)
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(rows * cols, generator=g) + 0.25).to(dtype)
    buf = torch.zeros(rows * cols + off, dtype=dtype, device="cuda")
    buf[off:] = x.cuda()
    xd = buf[off:].view(rows, cols)
    out = fs.column_sum(xd, odt)
    assert out.dtype == odt and out.shape == (cols,)
    assert torch.equal(out, fs.column_sum(xd, odt))
    ref = x.double().view(rows, cols).sum(0)
    assert_close(host(out), ref.numpy(), max(TOL[dtype], TOL[odt]), "column sum", elementwise=False)
