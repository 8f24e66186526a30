"""GPU parity: causal depthwise conv1d + bias + SiLU (the Mamba x branch, common.ex:251-252 and
298-309; the GatedDeltaNet short convolution) against a float64 torch reference, forward and
all gradients, including x read in place from a column slice of a wider tensor."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host, torch_causal_conv_silu

pytestmark = pytest.mark.gpu

CASES = [
    # (B, T, C, K, dtype, bias, x a column slice of a [B, T, 2C] tensor)
    (2, 70, 48, 4, torch.bfloat16, True, False),   # 8 channels per thread
    (2, 70, 20, 4, torch.float32, True, False),    # 4 channels per thread
    (1, 33, 13, 3, torch.float32, False, False),   # one channel per thread, no bias
    (2, 100, 64, 4, torch.bfloat16, True, True),   # strided x
    (1, 5, 16, 4, torch.bfloat16, True, False),    # T < K
    (3, 64, 40, 1, torch.float32, True, False),    # K = 1
    (1, 97, 24, 8, torch.float32, True, True),     # K = 8, T off the 32-step runs
    (2, 300, 2048, 4, torch.bfloat16, True, True), # config-5 width, many workgroups
    (2, 1, 16, 4, torch.bfloat16, True, True),     # one step (decode), strided: batch stride 2C
    (3, 1, 24, 3, torch.float32, True, True),      # the same in f32, three batch elements
    (2, 1, 16, 4, torch.float32, False, False),    # one step, contiguous
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_causal_conv1d_silu(case):
    from edifice_amd import fused_scan as fs
    B, T, C, K, dtype, with_bias, strided = case
    announce("causal_conv1d_silu", case=case)
    g = torch.Generator().manual_seed(7)
    xw = torch.randn(B, T, 2 * C if strided else C, generator=g)
    w = torch.randn(C, 1, K, generator=g) / K ** 0.5
    b = torch.randn(C, generator=g) if with_bias else None
    dy = torch.randn(B, T, C, generator=g)
    xd = xw.to("cuda", dtype).requires_grad_()
    wd = w.to("cuda", dtype).requires_grad_()
    bd = b.to("cuda", dtype).requires_grad_() if with_bias else None
    x_in = xd[..., :C] if strided else xd
    y = fs.causal_conv1d_silu(x_in, wd, bd)
    y.backward(dy.to("cuda", dtype))
    # reference on the rounded inputs, float64
    xr = xw.to(dtype).double().requires_grad_()
    wr = w.to(dtype).double().requires_grad_()
    br = b.to(dtype).double().requires_grad_() if with_bias else None
    yr = torch_causal_conv_silu(xr[..., :C] if strided else xr, wr, br)
    yr.backward(dy.to(dtype).double())
    tol = TOL[dtype]
    assert_close(host(y), yr.detach().numpy(), tol, "y")
    gx = host(xd.grad)
    assert_close(gx[..., :C], xr.grad.numpy()[..., :C], tol, "dx")
    if strided:
        assert np.all(gx[..., C:] == 0.0), "gradient outside the slice"
    assert_close(host(wd.grad), wr.grad.numpy(), tol, "dw")
    if with_bias:
        assert_close(host(bd.grad), br.grad.numpy(), tol, "dbias")


def test_causal_conv1d_silu_deterministic():
    """dw and dbias are summed in a fixed order: two calls give identical bits."""
    from edifice_amd import fused_scan as fs
    announce("causal_conv1d_silu_deterministic")
    g = torch.Generator().manual_seed(8)
    x = torch.randn(4, 256, 512, generator=g).to("cuda", torch.bfloat16)
    w = torch.randn(512, 1, 4, generator=g).to("cuda", torch.bfloat16)
    b = torch.randn(512, generator=g).to("cuda", torch.bfloat16)
    dy = torch.randn(4, 256, 512, generator=g).to("cuda", torch.bfloat16)
    grads = []
    for _ in range(2):
        xs, ws, bs = (t.clone().requires_grad_() for t in (x, w, b))
        fs.causal_conv1d_silu(xs, ws, bs).backward(dy)
        grads.append((xs.grad, ws.grad, bs.grad))
    for a, c in zip(*grads):
        assert torch.equal(a, c)
