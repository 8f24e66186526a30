"""GPU parity: fused softmax cross entropy (the decoder models' next-token loss) against
float64 torch on the same (rounded) logits: the mean loss and the logits' gradient."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_close
from tests.gpu_util import TOL, announce, host

pytestmark = pytest.mark.gpu

CASES = [
    # (rows, vocab, dtype)
    (64, 1000, torch.bfloat16),
    (37, 333, torch.float32),     # vocab off the 16-byte vector: one element per access
    (16, 32000, torch.bfloat16),  # config-5 vocabulary
    (5, 7, torch.bfloat16),       # vocab below one vector per thread
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v).replace("torch.", "") for v in c))
def test_cross_entropy(case):
    from edifice_amd import fused_scan as fs
    rows, vocab, dtype = case
    announce("cross_entropy", case=case)
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(rows, vocab, generator=g) * 3.0
    targets = torch.randint(0, vocab, (rows,), generator=g)
    targets[0], targets[-1] = 0, vocab - 1
    ld = logits.to("cuda", dtype).requires_grad_()
    loss = fs.cross_entropy(ld, targets.cuda())
    (2.0 * loss).backward()
    lr = logits.to(dtype).double().requires_grad_()
    ref = torch.nn.functional.cross_entropy(lr, targets)
    (2.0 * ref).backward()
    assert loss.dtype == torch.float32
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item()), (loss.item(), ref.item())
    assert_close(host(ld.grad), lr.grad.numpy(), TOL[dtype], "dlogits")
