"""Helpers shared by the GPU parity tests."""
import numpy as np
import torch

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}  # north-star tolerances (rel. to max |expected|)
DEV = "cuda"


def to_dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV).to(dtype)


def rounded(a, dtype):
    """The values the kernel actually sees (inputs rounded to the storage dtype), as float64."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype).double().numpy()


def host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def announce(name, **kw):
    print(f"[gpu-case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def torch_causal_conv_silu(x, weight, bias=None):
    """Reference for fs.causal_conv1d_silu, differentiable, float64 inside: silu(bias + sum_j
    w[c, j] x[t - (K - 1) + j]) with zeros before t = 0, as Axon.conv with padding
    [{K - 1, 0}] and one group per channel (lib/edifice/ssm/common.ex:298-309), written as K
    shifted products (no float64 convolution on the device); cast back to x's dtype."""
    w = weight.reshape(weight.shape[0], -1).double()
    k, seq = w.shape[1], x.shape[1]
    xp = torch.nn.functional.pad(x.double(), (0, 0, k - 1, 0))
    pre = sum(xp[:, j:j + seq] * w[:, j] for j in range(k))
    if bias is not None:
        pre = pre + bias.double()
    return torch.nn.functional.silu(pre).to(x.dtype)
