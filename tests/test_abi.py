"""C-ABI checks that need no GPU: the library loads, exports every symbol the public
header declares, and rejects invalid arguments with the reference's error messages
before touching the device."""
import ctypes
import glob
import os
import re

import pytest

from tests.conftest import ROOT


def _declared(pattern=os.path.join(ROOT, "include", "*.h")):
    names = set()
    for hdr in glob.glob(pattern):
        text = open(hdr).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(edf_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from edifice_amd import _native

    return _native.lib()


def test_header_declares_entry_points():
    names = _declared()
    for must in ("edf_fused_mingru_scan", "edf_fused_selective_scan", "edf_fused_flash_attention",
                 "edf_fused_delta_net_scan", "edf_fused_gated_delta_net_scan_backward"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_layout_probes_stay_out_of_the_product_header(lib):
    """The three layout probes live in the test-only header tests/edifice_hip_probes.h."""
    probes = _declared(os.path.join(ROOT, "tests", "*.h"))
    assert probes and not set(probes) & set(_declared())
    assert all(hasattr(lib, n) for n in probes)


def test_ctypes_table_covers_header():
    from edifice_amd import _native

    assert set(_declared()) <= set(_native.SIGNATURES), set(_declared()) - set(_native.SIGNATURES)


def test_version(lib):
    assert lib.edf_version() == 1


@pytest.mark.parametrize("call", [
    lambda L: L.edf_fused_mingru_scan(None, None, None, None, None, 0, 4, 4, 0),
    lambda L: L.edf_fused_minlstm_scan(None, None, None, None, None, None, 2, -1, 4, 0),
    lambda L: L.edf_fused_selective_scan(None, None, None, None, None, None, None, None, None, None, None, 0,
                                         1, 0, 4, 16, 1, 0, 0),
    lambda L: L.edf_fused_flash_attention(None, None, None, None, None, None, 1, 1, 0, 128, 1, 1),
    lambda L: L.edf_fused_delta_net_scan(None, None, None, None, None, None, None, 0, 0, 4, 2, 4, 0, 0),
])
def test_nonpositive_dims_rejected(lib, call):
    """The reference NIFs return {:error, "dimensions must be positive"} (c_src/edifice_cuda_nif.c:657)."""
    rc = call(lib)
    assert rc == 1
    assert lib.edf_last_error() == b"dimensions must be positive"


def test_bad_dtype_and_unsupported_shapes(lib):
    assert lib.edf_fused_mingru_scan(None, None, None, None, None, 1, 1, 1, 7) == 1
    assert b"dtype" in lib.edf_last_error()
    # the selective scan takes state sizes 1..32, as the reference (MAX_STATE 32)
    for fn, nargs in ((lib.edf_fused_selective_scan_backward, 18), (lib.edf_fused_selective_scan, 11)):
        rc = fn(*([None] * nargs), 0, 1, 8, 8, 33, 0, 0, 0)
        assert rc == 2 and b"state size" in lib.edf_last_error()
    # a missing workspace is reported, not dereferenced
    rc = lib.edf_fused_flash_attention_backward(*([ctypes.c_void_p(16)] * 10), None, 0, 1, 1, 8, 64, 1, 1)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    # the MinGRU block takes H <= 256 and needs its workspace
    p = ctypes.c_void_p(16)
    rc = lib.edf_fused_mingru_block_scan(None, p, p, None, p, p, 1 << 30, 2, 4, 257, 1, 0)
    assert rc == 2 and b"hidden" in lib.edf_last_error()
    rc = lib.edf_fused_mingru_block_scan(None, p, p, None, p, None, 0, 2, 4, 64, 1, 0)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    assert lib.edf_mingru_block_workspace_bytes(2, 4, 64, 3, 0) >= 4 * 2 * 4 * 64 * 4 + 2 * 64 * 4


def test_workspace_queries(lib):
    # one float32 state per (b, chunk of 16 timesteps, n, d), padded to 256 bytes, then room
    # for y before the gate (one float32 per (b, t, d))
    a256 = lambda v: (v + 255) // 256 * 256  # noqa: E731
    assert lib.edf_selective_scan_states_bytes(8, 2048, 1536, 16) == 8 * 128 * 16 * 1536 * 4 + 8 * 2048 * 1536 * 4
    assert lib.edf_selective_scan_states_bytes(1, 17, 3, 4) == a256(2 * 4 * 3 * 4) + 17 * 3 * 4
    # other state sizes are held padded to the next power of two
    assert lib.edf_selective_scan_states_bytes(1, 17, 3, 12) == a256(2 * 16 * 3 * 4) + 17 * 3 * 4
    assert lib.edf_selective_scan_states_bytes(1, 16, 3, 32) == a256(1 * 32 * 3 * 4) + 16 * 3 * 4
    assert lib.edf_flash_attention_backward_workspace_bytes(4, 32, 4096, 128) == 4 * 32 * 4096 * 4
    assert lib.edf_delta_rule_workspace_bytes(4, 4096, 16, 128, 1, 1) > 0  # chunked path
    assert lib.edf_delta_rule_workspace_bytes(4, 4096, 16, 128, 0, 1) == 0  # f32: step path
    # head_dim 64 .. 128 in steps of 8 takes the chunked path (padded to 128, same workspace)
    for d in (64, 96, 120):
        assert lib.edf_delta_rule_workspace_bytes(4, 4096, 16, d, 1, 1) == lib.edf_delta_rule_workspace_bytes(
            4, 4096, 16, 128, 1, 1)
    for d in (32, 60, 100):  # below 64 or not a multiple of 8: step path
        assert lib.edf_delta_rule_workspace_bytes(4, 4096, 16, d, 1, 1) == 0


def test_variant_entry_points_validate_before_launch(lib):
    """DeltaProduct, RLA, TTT and the LSTM / GRU blocks reject bad arguments with an error
    code and message before any device work."""
    p = ctypes.c_void_p(16)
    rc = lib.edf_fused_delta_product_scan(None, p, p, p, p, p, p, 1 << 20, 1, 4, 0, 2, 16, 0)
    assert rc == 1 and lib.edf_last_error() == b"dimensions must be positive"
    rc = lib.edf_fused_delta_product_scan(None, p, p, p, p, p, p, 1 << 20, 1, 4, 2, 2, 129, 0)
    assert rc == 2 and b"head_dim" in lib.edf_last_error()
    rc = lib.edf_fused_delta_product_scan(None, p, p, p, p, p, None, 0, 1, 4, 2, 2, 64, 0)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    rc = lib.edf_fused_rla_scan(None, p, p, p, p, p, p, p, 1, 4, 2, 16, 2, 1.0, 0)
    assert rc == 1 and b"variant" in lib.edf_last_error()
    rc = lib.edf_fused_rla_scan(None, p, p, p, p, p, p, p, 1, 4, 2, 16, 0, -0.5, 0)
    assert rc == 1 and b"clip" in lib.edf_last_error()
    rc = lib.edf_fused_rla_scan(None, p, p, p, p, p, p, p, 1, 4, 2, 16, 0, float("nan"), 0)
    assert rc == 1 and b"clip" in lib.edf_last_error()
    rc = lib.edf_fused_ttt_scan(None, p, p, p, p, p, p, p, p, 2, 4, 200, 0)
    assert rc == 2 and b"inner_size" in lib.edf_last_error()
    rc = lib.edf_fused_ttt_scan_backward(None, *([p] * 15), None, 0, 2, 4, 64, 0)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    rc = lib.edf_fused_lstm_block_scan(None, p, p, None, None, p, p, 1 << 30, 2, 4, 300, 1, 0)
    assert rc == 2 and b"hidden" in lib.edf_last_error()
    rc = lib.edf_fused_gru_block_scan(None, p, p, None, p, None, 0, 2, 4, 64, 2, 1)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    assert lib.edf_delta_product_backward_workspace_bytes(1, 5, 3, 2, 16, 0) > \
        lib.edf_delta_product_workspace_bytes(1, 5, 3, 2, 16, 0) > 0
    assert lib.edf_rla_scan_backward_workspace_bytes(0, 5, 2, 16, 0) == 0


def _t(*shape):
    import torch

    return torch.zeros(shape, dtype=torch.float32)


@pytest.mark.parametrize("call, msg", [
    (lambda fs: fs.mingru(_t(2, 5, 8), _t(2, 5, 9)), "candidates"),
    (lambda fs: fs.mingru(_t(2, 5), _t(2, 5)), "gates"),
    (lambda fs: fs.minlstm(_t(2, 5, 8), _t(2, 4, 8), _t(2, 5, 8)), "input_gates"),
    (lambda fs: fs.minlstm(_t(2, 5, 8), _t(2, 5, 8), _t(1, 5, 8)), "candidates"),
    (lambda fs: fs.selective_scan(_t(2, 5, 8), _t(2, 5, 7), _t(8, 4), _t(2, 5, 4), _t(2, 5, 4)), "dt"),
    (lambda fs: fs.selective_scan(_t(2, 5, 8), _t(2, 5, 8), _t(9, 4), _t(2, 5, 4), _t(2, 5, 4)), "A"),
    (lambda fs: fs.selective_scan(_t(2, 5, 8), _t(2, 5, 8), _t(8, 4), _t(2, 5, 3), _t(2, 5, 4)), "B"),
    (lambda fs: fs.selective_scan(_t(2, 5, 8), _t(2, 5, 8), _t(8, 4), _t(2, 5, 4), _t(2, 6, 4)), "C"),
    (lambda fs: fs.selective_scan(_t(2, 5, 8), _t(2, 5, 8), _t(8, 4), _t(2, 5, 4), _t(2, 5, 4), _t(7)), "D"),
    (lambda fs: fs.selective_scan(_t(2, 5, 8), _t(2, 5, 8), _t(8, 4), _t(2, 5, 4), _t(2, 5, 4), None,
                                  _t(2, 5, 1)), "z"),
])
def test_wrappers_reject_mismatched_shapes_before_launch(call, msg):
    """The kernels index every operand by the leading tensor's sizes, so the host mirror
    checks shapes first: the error is raised before device checks or any launch (these
    tensors are on the CPU, which would otherwise fail the device check)."""
    from edifice_amd import fused_scan as fs
    from edifice_amd._native import EdificeHipError

    with pytest.raises(EdificeHipError, match=msg):
        call(fs)


@pytest.mark.parametrize("gated", [False, True])
def test_chunked_delta_rule_forward_requires_workspace(lib, gated):
    """bf16 + per-head beta + head_dim 64..128 + seq >= 64 selects the chunked kernels: the
    forward, like the backward, returns EDF_ERR_WORKSPACE (4) for a missing or short
    workspace instead of silently running the per-step kernels.  The check precedes any
    device call, so dummy host addresses are never dereferenced."""
    from edifice_amd import _native

    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    B, T, H, d, bf16, per_head = 1, 128, 2, 128, 1, 1
    need = lib.edf_delta_rule_workspace_bytes(B, T, H, d, bf16, per_head)
    assert need > 0
    assert lib.edf_delta_rule_workspace_bytes(B, T, H, d, 0, per_head) == 0  # f32: per-step kernels
    for ws, nbytes in ((None, 0), (p, need - 1)):
        if gated:
            rc = lib.edf_fused_gated_delta_net_scan(None, p, p, p, p, p, p, ws, nbytes, B, T, H, d, bf16, per_head)
        else:
            rc = lib.edf_fused_delta_net_scan(None, p, p, p, p, p, ws, nbytes, B, T, H, d, bf16, per_head)
        assert rc == 4, rc
        assert b"workspace too small" in _native.lib().edf_last_error()


def test_noalloc_flash_backward_rejects_sizes_beyond_its_scratch(lib):
    """The allocation-free flash backward holds D in a fixed library-owned array of
    EDF_FA_NOALLOC_SCRATCH_BYTES (16 MiB = 4M rows of batch * heads * seq_len): larger calls get
    EDF_ERR_UNSUPPORTED (2) from the host-side check, before any device work."""
    p = ctypes.c_void_p(16)
    rows_max = (16 << 20) // 4
    rc = lib.edf_fused_flash_attention_backward_noalloc(None, *([p] * 9), 1, 1, rows_max + 1, 64, 1, 1)
    assert rc == 2 and b"no-alloc scratch" in lib.edf_last_error()


def test_context_and_glue_entry_points_validate_before_launch(lib):
    """The training-context forwards and saved backwards, the causal conv and the cross
    entropy reject bad arguments (sizes, null pointers, short contexts and workspaces) with an
    error code and message before any device work."""
    p = ctypes.c_void_p(16)
    # a context smaller than its query: EDF_ERR_WORKSPACE, for every op that records one
    need = lib.edf_ttt_scan_context_bytes(2, 9, 16, 0)
    assert need > 0
    rc = lib.edf_fused_ttt_scan_with_context(None, *([p] * 8), p, need - 1, 2, 9, 16, 0)
    assert rc == 4 and b"context" in lib.edf_last_error()
    rc = lib.edf_fused_ttt_scan_backward_saved(None, *([p] * 15), p, need - 1, p, 1 << 30, 2, 9, 16, 0)
    assert rc == 4 and b"context" in lib.edf_last_error()
    need = lib.edf_delta_product_context_bytes(1, 5, 2, 2, 16, 0)
    rc = lib.edf_fused_delta_product_scan_with_context(None, *([p] * 5), p, need - 1, 1, 5, 2, 2, 16, 0)
    assert rc == 4 and b"context" in lib.edf_last_error()
    rc = lib.edf_fused_delta_product_scan_backward_saved(None, *([p] * 9), None, 0, p, 1 << 30, 1, 5, 2, 2, 16, 0)
    assert rc == 4 and b"context" in lib.edf_last_error()
    need = lib.edf_rla_scan_context_bytes(1, 9, 2, 16, 0)
    rc = lib.edf_fused_rla_scan_with_context(None, *([p] * 7), p, need - 1, 1, 9, 2, 16, 0, 1.0, 0)
    assert rc == 4 and b"context" in lib.edf_last_error()
    rc = lib.edf_fused_rla_scan_with_context(None, *([p] * 7), p, need, 1, 9, 2, 16, 3, 1.0, 0)
    assert rc == 1 and b"variant" in lib.edf_last_error()
    need = lib.edf_kda_scan_context_bytes(1, 9, 2, 16, 0)
    rc = lib.edf_fused_kda_scan_with_context(None, *([p] * 6), p, need - 1, 1, 9, 2, 16, 0)
    assert rc == 4 and b"context" in lib.edf_last_error()
    rc = lib.edf_fused_kda_scan_backward_saved(None, *([p] * 11), p, need, p, 0, 1, 9, 2, 16, 0)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    # the per-step delta rule's training context is its 16-step states; the chunked path's is
    # its forward workspace
    assert lib.edf_delta_rule_forward_context_bytes(1, 40, 2, 32, 0, 0) > 0
    assert lib.edf_delta_rule_workspace_bytes(1, 40, 2, 32, 0, 0) == 0
    assert lib.edf_delta_rule_forward_context_bytes(1, 128, 2, 128, 1, 1) == \
        lib.edf_delta_rule_workspace_bytes(1, 128, 2, 128, 1, 1) > 0
    # causal conv: kernel size, row stride, workspace
    rc = lib.edf_causal_conv1d_silu(None, p, 8, p, p, p, 2, 5, 8, 9, 0)
    assert rc == 2 and b"kernel_size" in lib.edf_last_error()
    rc = lib.edf_causal_conv1d_silu(None, p, 7, p, p, p, 2, 5, 8, 4, 0)
    assert rc == 1 and b"x_row_stride" in lib.edf_last_error()
    rc = lib.edf_causal_conv1d_silu(None, p, 8, p, p, p, 0, 5, 8, 4, 0)
    assert rc == 1 and lib.edf_last_error() == b"dimensions must be positive"
    rc = lib.edf_causal_conv1d_silu_backward(None, p, 8, p, p, p, p, p, p, None, 0, 2, 5, 8, 4, 1)
    assert rc == 4 and b"workspace" in lib.edf_last_error()
    assert lib.edf_causal_conv1d_silu_backward_workspace_bytes(2, 5, 8, 9) == 0
    # cross entropy
    rc = lib.edf_cross_entropy(None, p, p, p, None, 4, 10, 1)
    assert rc == 1 and b"null" in lib.edf_last_error()
    rc = lib.edf_cross_entropy_backward(None, p, p, p, p, 0.25, p, 4, 10, 3)
    assert rc == 1 and b"dtype" in lib.edf_last_error()
