"""ctypes binding of ``libedifice_hip.so`` (the C ABI in ``include/edifice_hip.h``).

The library is loaded lazily; if it has not been built, every op raises
``EdificeHipError`` — there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes
import os

from .build import lib_path

P = ctypes.c_void_p
I = ctypes.c_int
S = ctypes.c_size_t
F = ctypes.c_float
L = ctypes.c_long

# name -> (restype, argtypes); must match include/edifice_hip.h
SIGNATURES = {
    "edf_version": (I, []),
    "edf_last_error": (ctypes.c_char_p, []),
    "edf_fused_mingru_scan": (I, [P, P, P, P, P, I, I, I, I]),
    "edf_fused_mingru_scan_backward": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I]),
    "edf_mingru": (I, [P, P, P, P, I, I, I, I]),
    "edf_mingru_backward": (I, [P, P, P, P, P, P, P, I, I, I, I]),
    "edf_fused_minlstm_scan": (I, [P, P, P, P, P, P, I, I, I, I]),
    "edf_fused_minlstm_scan_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I]),
    "edf_minlstm": (I, [P, P, P, P, P, I, I, I, I]),
    "edf_minlstm_backward": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I]),
    "edf_fused_linear_scan": (I, [P, P, P, P, P, I, I, I, I]),
    "edf_fused_linear_scan_backward": (I, [P, P, P, P, P, P, P, P, I, I, I, I]),
    "edf_mingru_block_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_mingru_block_scan": (I, [P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_minlstm_block_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_minlstm_block_scan": (I, [P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_linear_block_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_linear_block_scan": (I, [P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_lstm_block_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_lstm_block_scan": (I, [P, P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_gru_block_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_lstm_block_status": (I, [P, P, S, I, I, I, I]),
    "edf_gru_block_status": (I, [P, P, S, I, I, I, I]),
    "edf_fused_gru_block_scan": (I, [P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_fused_selective_scan": (I, [P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I, I]),
    "edf_selective_scan_states_bytes": (S, [I, I, I, I]),
    "edf_selective_scan_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_selective_scan_backward": (
        I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I, I]),
    "edf_selective_scan_backward_workspace_bytes": (S, [I, I, I, I, I, I]),
    "edf_fused_flash_attention": (I, [P, P, P, P, P, P, I, I, I, I, I, I]),
    "edf_fused_flash_attention_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_flash_attention_backward_workspace_bytes": (S, [I, I, I, I]),
    "edf_fused_flash_attention_backward_noalloc": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I]),
    "edf_fused_fox_attention": (I, [P, P, P, P, P, P, P, I, I, I, I, I]),
    "edf_fused_fox_attention_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_fox_attention_backward_workspace_bytes": (S, [I, I, I, I]),
    "edf_causal_conv1d_silu": (I, [P, P, I, P, P, P, I, I, I, I, I]),
    "edf_causal_conv1d_silu_backward_workspace_bytes": (S, [I, I, I, I]),
    "edf_causal_conv1d_silu_backward": (I, [P, P, I, P, P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_cross_entropy": (I, [P, P, P, P, P, I, I, I]),
    "edf_cross_entropy_backward": (I, [P, P, P, P, P, F, P, I, I, I]),
    "edf_layer_norm": (I, [P, P, P, P, P, P, P, I, I, F, I, I]),
    "edf_layer_norm_backward_workspace_bytes": (S, [I, I]),
    "edf_layer_norm_backward": (I, [P, P, P, P, P, P, P, P, P, P, S, I, I, I, I]),
    "edf_add_layer_norm": (I, [P, P, P, P, P, P, P, P, P, I, I, F, I, I]),
    "edf_layer_norm_backward_add": (I, [P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I]),
    "edf_heads_split": (I, [P, P, P, L, L, I, I, I, I]),
    "edf_heads_merge": (I, [P, P, P, L, L, I, I, I, I]),
    "edf_embedding_backward_workspace_bytes": (S, [L, L]),
    "edf_embedding_backward": (I, [P, P, P, P, P, S, L, L, I, L, I]),
    "edf_softplus": (I, [P, P, P, L, I]),
    "edf_softplus_backward": (I, [P, P, P, P, L, I]),
    "edf_column_sum_workspace_bytes": (S, [L, I]),
    "edf_column_sum": (I, [P, P, P, P, S, L, I, I, I]),
    "edf_l2_normalize": (I, [P, P, P, L, I, F, I]),
    "edf_l2_normalize_backward": (I, [P, P, P, P, L, I, F, I]),
    "edf_delta_net_split": (I, [P, P, P, P, P, P, L, I, I, F, I]),
    "edf_delta_net_split_backward": (I, [P, P, P, P, P, P, P, L, I, I, F, I]),
    "edf_laser_attention_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_laser_attention": (I, [P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_laser_attention_backward_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_fused_laser_attention_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_delta_rule_workspace_bytes": (S, [I, I, I, I, I, I]),
    "edf_delta_rule_backward_workspace_bytes": (S, [I, I, I, I, I, I]),
    "edf_fused_delta_net_scan": (I, [P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_fused_gated_delta_net_scan": (I, [P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_fused_delta_rule_scan_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_fused_gated_delta_net_scan_backward": (
        I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_delta_rule_forward_context_bytes": (S, [I, I, I, I, I, I]),
    "edf_delta_rule_saved_backward_workspace_bytes": (S, [I, I, I, I, I, I]),
    "edf_fused_delta_rule_scan_backward_saved": (
        I, [P, P, P, P, P, P, P, P, P, P, P, P, P, S, P, S, I, I, I, I, I, I]),
    "edf_fused_kda_scan": (I, [P, P, P, P, P, P, P, I, I, I, I, I]),
    "edf_fused_kda_scan_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_kda_scan_backward_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_kda_scan_context_bytes": (S, [I, I, I, I, I]),
    "edf_fused_kda_scan_with_context": (I, [P, P, P, P, P, P, P, P, S, I, I, I, I, I]),
    "edf_fused_kda_scan_backward_saved": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, S, P, S, I, I, I, I, I]),
    "edf_fused_delta_product_scan": (I, [P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_delta_product_workspace_bytes": (S, [I, I, I, I, I, I]),
    "edf_fused_delta_product_scan_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_delta_product_backward_workspace_bytes": (S, [I, I, I, I, I, I]),
    "edf_delta_product_context_bytes": (S, [I, I, I, I, I, I]),
    "edf_fused_delta_product_scan_with_context": (I, [P, P, P, P, P, P, P, S, I, I, I, I, I, I]),
    "edf_fused_delta_product_scan_backward_saved": (I, [P, P, P, P, P, P, P, P, P, P, P, S, P, S, I, I, I, I, I,
                                                         I]),
    "edf_fused_rla_scan": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, F, I]),
    "edf_fused_rla_scan_backward": (
        I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, F, I]),
    "edf_rla_scan_backward_workspace_bytes": (S, [I, I, I, I, I]),
    "edf_rla_scan_context_bytes": (S, [I, I, I, I, I]),
    "edf_fused_rla_scan_with_context": (I, [P, P, P, P, P, P, P, P, P, S, I, I, I, I, I, F, I]),
    "edf_fused_rla_scan_backward_saved": (
        I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, P, S, I, I, I, I, I, F, I]),
    "edf_fused_ttt_scan": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I]),
    "edf_fused_ttt_scan_backward": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, I, I, I, I]),
    "edf_ttt_scan_backward_workspace_bytes": (S, [I, I, I, I]),
    "edf_ttt_scan_context_bytes": (S, [I, I, I, I]),
    "edf_fused_ttt_scan_with_context": (I, [P, P, P, P, P, P, P, P, P, P, S, I, I, I, I]),
    "edf_fused_ttt_scan_backward_saved": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, S, P, S, I, I,
                                               I, I]),
}


class EdificeHipError(RuntimeError):
    """Raised when the HIP library is missing or an entry point returns an error."""


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not os.path.exists(path):
            raise EdificeHipError(
                f"{path} is not built; run `python -m edifice_amd.build` (edifice_amd has no CPU fallback)")
        handle = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().edf_last_error().decode(errors="replace")
        raise EdificeHipError(f"{name} failed (code {rc}): {msg}")


def query(name: str, *args) -> int:
    return int(getattr(lib(), name)(*args))
