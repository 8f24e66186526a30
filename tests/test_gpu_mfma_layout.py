"""Pin the v_mfma_f32_32x32x16_bf16 lane layout the attention/delta-rule kernels assume."""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def test_mfma_32x32x16_layout(rng):
    from edifice_amd import _native as nat
    announce("mfma_layout")
    A = torch.from_numpy(rng.integers(-4, 5, size=(32, 16)).astype(np.float32)).to("cuda", torch.bfloat16)
    B = torch.from_numpy(rng.integers(-4, 5, size=(16, 32)).astype(np.float32)).to("cuda", torch.bfloat16)
    C = torch.empty(32, 32, dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.call("edf_debug_mfma_32x32x16_bf16", stream, ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(B.data_ptr()),
             ctypes.c_void_p(C.data_ptr()))
    expect = A.float().cpu().numpy() @ B.float().cpu().numpy()
    np.testing.assert_array_equal(C.cpu().numpy(), expect)  # small integers: exact
