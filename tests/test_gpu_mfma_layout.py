"""Pin the v_mfma_f32_32x32x16_bf16 lane layout the attention/delta-rule kernels assume,
through the library's layout probes (declared in tests/edifice_hip_probes.h, not part of the
product C ABI, so bound here rather than in edifice_amd._native)."""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_util import announce

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
PROBES = {"edf_debug_mfma_32x32x16_bf16": [P, P, P, P], "edf_debug_acc_kfrag_bf16": [P, P, P],
          "edf_debug_lds_read_tr16": [P, P, P]}


def _probe(name, *args):
    from edifice_amd import _native as nat
    fn = getattr(nat.lib(), name)
    fn.restype, fn.argtypes = ctypes.c_int, PROBES[name]
    rc = fn(*args)
    assert rc == 0, nat.lib().edf_last_error()


def test_mfma_32x32x16_layout(rng):
    announce("mfma_layout")
    A = torch.from_numpy(rng.integers(-4, 5, size=(32, 16)).astype(np.float32)).to("cuda", torch.bfloat16)
    B = torch.from_numpy(rng.integers(-4, 5, size=(16, 32)).astype(np.float32)).to("cuda", torch.bfloat16)
    C = torch.empty(32, 32, dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _probe("edf_debug_mfma_32x32x16_bf16", stream, ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(B.data_ptr()),
             ctypes.c_void_p(C.data_ptr()))
    expect = A.float().cpu().numpy() @ B.float().cpu().numpy()
    np.testing.assert_array_equal(C.cpu().numpy(), expect)  # small integers: exact


def test_acc_kfrag_layout(rng):
    """An accumulator tile reused as an operand over its rows (v_permlane32_swap)."""
    announce("acc_kfrag_layout")
    x = rng.integers(-64, 65, size=(64, 32)).astype(np.float32)  # exact in bf16
    X = torch.from_numpy(x).cuda()
    out = torch.empty(64, 4, 8, dtype=torch.bfloat16, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _probe("edf_debug_acc_kfrag_bf16", stream, ctypes.c_void_p(X.data_ptr()), ctypes.c_void_p(out.data_ptr()))
    got = out.float().cpu().numpy()
    lane = np.arange(64)[:, None, None]
    kk = np.arange(4)[None, :, None]
    e = np.arange(8)[None, None, :]
    expect = x[16 * kk + 8 * (lane // 32) + e, lane % 32]
    np.testing.assert_array_equal(got, expect)


def test_lds_read_tr16_layout(rng):
    """ds_read_b64_tr_b16: the transposed V^T operand read from a row-major LDS tile."""
    announce("lds_read_tr16_layout")
    x = rng.integers(-128, 128, size=(64, 64)).astype(np.float32)  # exact in bf16
    X = torch.from_numpy(x).to("cuda", torch.bfloat16)
    out = torch.empty(64, 2, 4, dtype=torch.bfloat16, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _probe("edf_debug_lds_read_tr16", stream, ctypes.c_void_p(X.data_ptr()), ctypes.c_void_p(out.data_ptr()))
    got = out.float().cpu().numpy()
    lane = np.arange(64)[:, None, None]
    rb = np.arange(2)[None, :, None]
    e = np.arange(4)[None, None, :]
    expect = x[8 * rb + 4 * (lane // 32) + e, lane % 32]
    np.testing.assert_array_equal(got, expect)
