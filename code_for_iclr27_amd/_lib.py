"""Loader for liblazyrecall_hip.so, the C ABI declared in include/lazyrecall.h.

torch is imported before the library is opened so that the library's libamdhip64.so.7
dependency binds to the HIP runtime torch already loaded (one runtime per process). There is
no CPU fallback: if the library is missing every op raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIBRARY_PATH = Path(__file__).resolve().parent / "liblazyrecall_hip.so"

LR_OK = 0
LR_DTYPE_F32, LR_DTYPE_F64, LR_DTYPE_F16, LR_DTYPE_BF16 = 0, 1, 2, 3
LR_SEG_WORDS = 12
LR_HEAD_WORDS = 6
LR_REINSERT_WORDS = 8
LR_APPEND_WORDS = 12
LR_REINSERT_MAX_PER_HEAD = 4096
LR_HISTORY_MAX_LAYERS = 128

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t

# name -> argument types; every entry point returns int status unless listed in _RESTYPES.
SIGNATURES = {
    "lr_last_error": [],
    "lr_abi_version": [],
    "lr_temporal_probabilities": [_P, _I, _P, _P, _P, _I64, _I64, _I64, _F, _P, _P, _P],
    "lr_temporal_risk": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _D, _P, _P],
    "lr_append": [_P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I, _I64, _I64, _P, _P, _P, _P,
                  _P, _P],
    "lr_append_layers": [_P, _I64, _I64, _I64, _I64, _I, _I64, _P, _P, _P, _P, _P, _P],
    "lr_append_layers_host": [_P, _I64, _I64, _I64, _I64, _I, _I64, _P, _P, _P, _P, _P, _P],
    "lr_compact": [_P, _P, _P, _I64, _I64, _I, _P, _I64, _P, _P, _P, _P],
    "lr_pool": [_P, _I64, _P, _I64, _I64, _I64, _P, _P],
    "lr_merge": [_P, _P, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _I, _P, _P, _P, _P],
    "lr_pack": [_P, _P, _P, _I64, _P, _P, _I64, _I64, _I, _I64, _P, _P, _P],
    "lr_batch_append": [_P, _I64, _P, _P, _I64, _I, _I64, _P, _P, _P, _P],
    "lr_batch_append_host": [_P, _I64, _P, _P, _I64, _I, _I64, _P, _P, _P, _P],
    "lr_pack_layers": [_P, _I64, _P, _I64, _I64, _P, _P, _P],
    "lr_pack_heads": [_P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P],
    "lr_group_mean_queries": [_P, _I64, _I64, _I64, _I64, _I, _P, _P],
    "lr_append_flattened_cache": [_P, _I64, _P, _I64, _I64, _I64, _I, _P, _P, _P, _P],
    "lr_compact_flattened_kv": [_P, _P, _I64, _I64, _I, _P, _I64, _P, _P, _P],
    "lr_decision_risk_scores": [_P, _P, _I, _P, _P, _I64, _I64, _I64, _D, _D, _P, _P],
    "lr_register_host": [_U64, _U64],
    "lr_unregister_host": [_U64],
    "lr_score_workspace_bytes": [_I64, _I64, _I64, _I64],
    "lr_score_segments": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _F, _D, _P, _SZ,
                          _P, _P, _I, _P],
    "lr_debug_segment_logits": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P],
    "lr_select_workspace_bytes": [_I64, _I64, _I64],
    "lr_select_refine": [_P, _P, _I64, _P, _P, _I64, _I64, _P, _SZ, _P, _P, _P, _P, _P, _P, _P,
                         _P],
    "lr_select_refine_sets": [_P, _P, _I64, _P, _P, _I64, _I64, _P, _SZ, _P, _P, _P, _P, _P, _P,
                              _P],
    "lr_pool_select_refine_sets": [_P, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _P, _SZ, _P,
                                   _P, _P, _P, _P, _P, _P],
    "lr_select_refine_queue": [_P, _I64, _I64, _I64, _P, _SZ, _P, _P, _P, _P, _P, _P],
    "lr_compact_heads": [_P, _I64, _P, _P, _P, _I64, _I, _I64, _I64, _P, _P, _P, _P],
    "lr_compact_heads_layout": [_P, _I64, _P, _P, _P, _I64, _I, _I64, _I64, _P, _P, _P, _I64, _P,
                                _P, _P],
    "lr_reinsert_plan": [_P, _I64, _P, _I64, _P, _P, _P, _P],
    "lr_reinsert_plan_layout": [_P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _P, _P],
    "lr_reinsert_group": [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P],
    "lr_reinsert_resident": [_P, _I64, _P, _I64, _I64, _I64, _I, _I64, _P, _P, _P, _P],
    "lr_reinsert_recalled": [_P, _I64, _P, _I64, _I, _I64, _P, _P, _P, _P],
    "lr_queue_index": [_P, _P, _I64, _P, _P, _P, _I64, _P, _P],
    "lr_queue_evict_plan": [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P],
    "lr_history_append": [_P, _I64, _I64, _I64, _I, _I64, _I64, _P, _I64, _P, _P],
    "lr_staging_alloc": [_SZ, _P],
    "lr_staging_free": [_P],
    "lr_copy_words": [_P, _P, _I64, _P],
    "lr_stream_copy": [_P, _P, _I64, _P],
    "lr_packed_attention_workspace_bytes": [_I64, _I64, _I64, _I64, _I64],
    "lr_packed_attention": [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64,
                            _I, _I64, _F, _P, _P, _SZ, _P],
    "lr_packed_attention_pending_workspace_bytes": [_I64, _I64, _I64, _I64],
    "lr_packed_attention_pending": [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _I64,
                                    _I64, _I, _I64, _F, _P, _P, _P, _P, _SZ, _P],
    "lr_packed_attention_scratch_bytes": [],
    "lr_packed_attention_noalloc": [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _I64,
                                    _I64, _I64, _I, _I64, _F, _P, _P],
    "lr_head_logits": [_P, _I64, _P, _P, _I64, _I64, _I, _P, _P],
    "lr_margin_stats_workspace_bytes": [_I64, _I64],
    "lr_margin_stats": [_P, _I64, _I64, _P, _P, _P, _P, _P, _SZ, _P],
    "lr_row_sum_workspace_bytes": [_I64, _I64, _I64],
    "lr_hidden_gradient": [_P, _P, _P, _I64, _P, _I64, _I64, _I, _P, _P, _P, _SZ, _P],
    "lr_pre_gradient": [_P, _P, _I64, _I64, _I, _P, _P, _P, _SZ, _P],
    "lr_pre_gradient_layers_workspace_bytes": [_I64, _I64, _I64],
    "lr_pre_gradient_layers": [_P, _I64, _I64, _I64, _I, _P, _SZ, _P],
}
_RESTYPES = {"lr_last_error": ctypes.c_char_p, "lr_score_workspace_bytes": ctypes.c_size_t,
             "lr_select_workspace_bytes": ctypes.c_size_t,
             "lr_packed_attention_workspace_bytes": ctypes.c_size_t,
             "lr_packed_attention_scratch_bytes": ctypes.c_size_t,
             "lr_packed_attention_pending_workspace_bytes": ctypes.c_size_t,
             "lr_row_sum_workspace_bytes": ctypes.c_size_t,
             "lr_margin_stats_workspace_bytes": ctypes.c_size_t,
             "lr_pre_gradient_layers_workspace_bytes": ctypes.c_size_t}

_library = None


class LazyRecallLibraryError(RuntimeError):
    """Raised when the native library is missing or an entry point fails."""


def load() -> ctypes.CDLL:
    """Open the library once and declare every exported entry point."""
    global _library
    if _library is not None:
        return _library
    if not LIBRARY_PATH.exists():
        raise LazyRecallLibraryError(
            f"{LIBRARY_PATH.name} is not built; run `python -m code_for_iclr27_amd.build` "
            "(there is no CPU fallback for the LazyRecall HIP ops)")
    library = ctypes.CDLL(os.fspath(LIBRARY_PATH))
    for name, argtypes in SIGNATURES.items():
        function = getattr(library, name)
        function.argtypes = argtypes
        function.restype = _RESTYPES.get(name, ctypes.c_int)
    _library = library
    return library


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def last_error() -> str:
    message = load().lr_last_error()
    return message.decode() if message else ""


def call(name: str, *args) -> None:
    """Invoke an entry point and raise RuntimeError with the library's message on failure."""
    status = getattr(load(), name)(*args)
    if status != LR_OK:
        raise LazyRecallLibraryError(last_error() or f"{name} failed with status {status}")


def ptr(tensor) -> int | None:
    """Device address of a tensor (None for an empty tensor, which the ABI accepts as NULL)."""
    if tensor is None or tensor.numel() == 0:
        return None
    return tensor.data_ptr()


def stream_of(tensor) -> int:
    """Raw hipStream_t of the current torch stream on the tensor's device."""
    return torch.cuda.current_stream(tensor.device).cuda_stream


DTYPE_CODES = {
    torch.float32: LR_DTYPE_F32,
    torch.float64: LR_DTYPE_F64,
    torch.float16: LR_DTYPE_F16,
    torch.bfloat16: LR_DTYPE_BF16,
}
