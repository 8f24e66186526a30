"""GPU parity: the attention blocks' head split / merge kernels are exact permutations."""
import pytest
import torch

from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


HEAD_CASES = [
    # (batch, seq, parts, heads, head_dim, dtype, offset)
    (2, 64, 3, 8, 128, torch.bfloat16, 0),   # the config-5 attention's q | k | v
    (1, 37, 1, 4, 64, torch.float32, 0),     # the output merge
    (2, 9, 4, 2, 12, torch.float32, 0),      # 48-byte head rows
    (1, 5, 2, 3, 7, torch.bfloat16, 0),      # off the vector: one element per thread
    (1, 6, 3, 2, 64, torch.bfloat16, 1),     # misaligned input
]


@pytest.mark.parametrize("case", HEAD_CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_split_merge_heads(case):
    """fs.split_heads / fs.merge_heads are exact permutations (bit-identical to torch's reshape +
    transpose), each the other's backward."""
    from edifice_amd import fused_scan as fs
    bsz, seq, parts, nh, d, dtype, off = case
    announce("split_merge_heads", case=case)
    g = torch.Generator().manual_seed(41)
    width = parts * nh * d
    x = torch.randn(bsz * seq * width, generator=g).to(dtype)
    buf = torch.zeros(x.numel() + off, dtype=dtype, device="cuda")
    buf[off:] = x.cuda()
    xd = buf[off:].view(bsz, seq, width).detach().requires_grad_()
    outs = fs.split_heads(xd, parts, nh)
    ref = x.view(bsz, seq, parts, nh, d).permute(2, 0, 3, 1, 4)
    assert len(outs) == parts
    for p, o in enumerate(outs):
        assert o.shape == (bsz, nh, seq, d) and torch.equal(o.cpu(), ref[p])
    grads = [torch.randn(bsz, nh, seq, d, generator=g).to(dtype) for _ in range(parts)]
    torch.autograd.backward(outs, [t.cuda() for t in grads])
    want = torch.stack(grads).permute(1, 3, 0, 2, 4).reshape(bsz, seq, width)
    assert torch.equal(xd.grad.cpu(), want)
    h = grads[0].cuda().requires_grad_()
    y = fs.merge_heads(h)
    assert torch.equal(y.cpu(), grads[0].transpose(1, 2).reshape(bsz, seq, nh * d))
    dy = torch.randn(bsz, seq, nh * d, generator=g).to(dtype)
    y.backward(dy.cuda())
    assert torch.equal(h.grad.cpu(), dy.view(bsz, seq, nh, d).transpose(1, 2))
