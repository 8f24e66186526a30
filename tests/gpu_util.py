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
