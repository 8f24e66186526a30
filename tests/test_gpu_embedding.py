"""GPU parity: the HIP token-embedding weight gradient (the language models' input embedding)
against float64 torch on the same (rounded) inputs, and bit-identical on a repeated call."""
import pytest
import torch

from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host

pytestmark = pytest.mark.gpu

CASES = [
    # (ids shape, vocab, dim, dtype, padding_idx, id pattern)
    ((8, 257), 32000, 1024, torch.bfloat16, None, "uniform"),   # the config-5 layer, reduced length
    ((5000,), 1000, 256, torch.float32, None, "uniform"),
    ((2, 700), 64, 128, torch.bfloat16, 3, "uniform"),          # long runs, a padding row
    ((3000,), 10, 64, torch.float32, None, "one"),              # every position on one row
    ((300,), 50, 33, torch.float32, None, "uniform"),           # off the vector: one column per lane
    ((0,), 20, 16, torch.float32, None, "uniform"),             # no positions: all rows zero
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_embedding_backward(case):
    from edifice_amd import fused_scan as fs
    shape, vocab, dim, dtype, pad, pattern = case
    announce("embedding_backward", case=case)
    g = torch.Generator().manual_seed(31)
    ids = torch.randint(0, vocab, shape, generator=g) if pattern == "uniform" else torch.full(shape, 7)
    w = torch.randn(vocab, dim, generator=g).to(dtype)
    dy = torch.randn(*shape, dim, generator=g).to(dtype)
    wd = w.cuda().requires_grad_()
    out = fs.embedding(ids.cuda(), wd, pad)
    assert torch.equal(out.cpu(), torch.nn.functional.embedding(ids, w, pad))
    out.backward(dy.cuda())
    first = wd.grad.clone()
    wd.grad = None
    fs.embedding(ids.cuda(), wd, pad).backward(dy.cuda())
    assert torch.equal(first, wd.grad)
    wr = w.double().requires_grad_()
    torch.nn.functional.embedding(ids, wr, pad).backward(dy.double())
    assert first.dtype == dtype and first.shape == (vocab, dim)
    assert_close(host(first), wr.grad.numpy(), TOL[dtype], "dW")
    if pad is not None:
        assert not first[pad].any()
    unused = torch.ones(vocab, dtype=torch.bool)
    unused[ids.reshape(-1)] = False
    assert not first[unused.cuda()].any()


def test_embedding_module_in_model():
    """blocks.Embedding keeps nn.Embedding's parameter and gives torch's float32 gradient."""
    from edifice_amd import blocks
    announce("embedding_module")
    torch.manual_seed(32)
    m = blocks.Embedding(500, 64).cuda()
    ref = torch.nn.Embedding(500, 64).cuda()
    ref.load_state_dict(m.state_dict())
    ids = torch.randint(0, 500, (4, 100), device="cuda")
    dy = torch.randn(4, 100, 64, device="cuda")
    m(ids).backward(dy)
    ref(ids).backward(dy)
    assert_close(host(m.weight.grad), host(ref.weight.grad), TOL[torch.float32], "dW vs nn.Embedding")

