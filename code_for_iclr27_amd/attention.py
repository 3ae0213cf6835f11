"""Attention over the packed ragged KV layout, the drop-in for ``packed_attention`` of
src/lazy_recall/attention.py:15-35 (and its use by batch_attention.py:92-97).

The reference hands the packed per-(request, KV head) segments to flash_attn's
``flash_attn_varlen_func`` (causal, softmax scale dim^-0.5, one KV head per segment, G query
heads). Here the same call runs the HIP kernel ``packed_attention_kernel`` of
liblazyrecall_hip.so through ``lr_packed_attention``: split-key flash decoding with QK^T on
MFMA, P*V on the VALU, f32 accumulation and the output rounded to the input dtype. There is no
CPU path and no flash_attn dependency; CPU tensors are rejected.

Forward only: the reference's audit step differentiates through this call with flash_attn's
deterministic backward (attention.py:25-33); that backward is not part of this library, so a
call that would need it raises.
"""

from __future__ import annotations

import torch

from . import _lib


def flash_attn_deterministic_status():
    """attention.py:10-11. No deterministic backward has run through this module."""
    return None


_native_module = None


def _native():
    """The C++ host module with lr_packed_attention bound (once): a decode step calls this once
    per layer, and its checks, allocations and launch run in C++ on torch's current stream."""
    global _native_module
    if _native_module is None:
        import ctypes
        from .scoring import _planner
        planner = _planner()
        library = _lib.load()
        address = lambda name: ctypes.cast(getattr(library, name), ctypes.c_void_p).value
        planner.bind_attention(address("lr_packed_attention"),
                               address("lr_packed_attention_workspace_bytes"),
                               address("lr_packed_attention_pending"),
                               address("lr_packed_attention_pending_workspace_bytes"))
        _native_module = planner
    return _native_module


def packed_attention(queries, keys, values, metadata, length, kv_heads, pending=None):
    """attention.py:15-35 -> [batch, length, query_heads * dim] in the queries' dtype.

    ``queries`` [batch, query_heads, length, dim] (any strides with dim contiguous), ``keys`` and
    ``values`` hold the packed rows (reshaped to [-1, dim]), ``metadata`` carries
    ``cu_seqlens_k`` (int32 [batch*kv_heads + 1] on the device), ``max_seqlen_k`` (host int) and
    ``decoding_cu_seqlens_q`` ([batch*kv_heads + 1]; every segment has ``length`` queries).
    The checks (flash_attn's messages), the output and workspace allocation and the launch of
    ``lr_packed_attention`` run in the C++ host module (csrc/host_plan.cpp attention_launch).

    ``pending`` (decode only, ``length`` 1): ``(new_keys, new_values)``, each
    ``[batch, kv_heads, 1, dim]``, the step's own tokens not yet appended. Each segment then
    attends over its cached rows and its pending row, which sits where the append would put it
    (after the cached rows), so the result equals the call on the appended cache bit for bit;
    ``metadata`` describes the cache without them. The step's appends can then wait for one
    ``_C.append_layers`` launch after every layer's attention.
    """
    if torch.is_grad_enabled() and queries.requires_grad:
        raise RuntimeError("packed_attention: the deterministic attention backward is not "
                           "implemented on the HIP path (forward only)")
    new_keys, new_values = (None, None) if pending is None else pending
    return (_native_module or _native()).packed_attention(
        queries, keys, values, metadata.cu_seqlens_k, metadata.decoding_cu_seqlens_q.numel(),
        int(metadata.max_seqlen_k), int(length), int(kv_heads), new_keys, new_values)
