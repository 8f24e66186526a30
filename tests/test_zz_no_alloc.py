"""The allocation-free flash-attention backward (edf_fused_flash_attention_backward_noalloc)
against the workspace entry point (edf_fused_flash_attention_backward), both through the C
ABI: identical dq, dk, dv on two calls in a row, the second smaller (the library's scratch
still holds the first call's D), for the MFMA kernels (bf16, head_dim 128, causal) and the
wave kernels (float32, head_dim 64, non-causal)."""
import ctypes

import pytest
import torch

from tests.gpu_util import announce

pytestmark = pytest.mark.gpu

P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(nat, B, H, T, d, dtype, causal, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, T, d, device="cuda", generator=g).mul_(d ** -0.25).to(dtype) for _ in range(4))
    flag = 1 if dtype == torch.bfloat16 else 0
    out = torch.empty_like(q)
    lse = torch.empty(B, H, T, dtype=torch.float32, device="cuda")
    nat.call("edf_fused_flash_attention", _stream(), P(q), P(k), P(v), P(out), P(lse), B, H, T, d, causal, flag)
    want = [torch.empty_like(q) for _ in range(3)]
    wsb = nat.query("edf_flash_attention_backward_workspace_bytes", B, H, T, d)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    nat.call("edf_fused_flash_attention_backward", _stream(), P(q), P(k), P(v), P(out), P(do), P(lse),
             *(P(t) for t in want), P(ws), wsb, B, H, T, d, causal, flag)
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    nat.call("edf_fused_flash_attention_backward_noalloc", _stream(), P(q), P(k), P(v), P(out), P(do), P(lse),
             *(P(t) for t in got), B, H, T, d, causal, flag)
    torch.cuda.synchronize()
    for name, a, e in zip(("dq", "dk", "dv"), got, want):
        assert torch.isfinite(e).all(), name
        assert torch.equal(a, e), f"{name}: max |diff| {(a.float() - e.float()).abs().max().item()}"


@pytest.mark.parametrize("dtype, d, causal", [(torch.bfloat16, 128, 1), (torch.float32, 64, 0)],
                         ids=["bf16-d128-causal", "f32-d64"])
def test_noalloc_backward_matches_workspace_entry_point(dtype, d, causal):
    from edifice_amd import _native as nat
    for i, (B, H, T) in enumerate(((2, 4, 300), (1, 2, 130))):  # the second call is smaller
        announce("flash_bwd_noalloc", call=i, B=B, H=H, T=T, d=d, dtype=dtype, causal=causal)
        _case(nat, B, H, T, d, dtype, causal, seed=100 + i)
