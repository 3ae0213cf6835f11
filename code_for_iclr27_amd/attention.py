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


def _check(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def packed_attention(queries, keys, values, metadata, length, kv_heads):
    """attention.py:15-35 -> [batch, length, query_heads * dim] in the queries' dtype.

    ``queries`` [batch, query_heads, length, dim] (any strides with dim contiguous), ``keys`` and
    ``values`` hold the packed rows (reshaped to [-1, dim]), ``metadata`` carries
    ``cu_seqlens_k`` (int32 [batch*kv_heads + 1] on the device), ``max_seqlen_k`` (host int) and
    ``decoding_cu_seqlens_q`` ([batch*kv_heads + 1]; every segment has ``length`` queries).
    """
    batch, query_heads, query_length, dimension = queries.shape
    length, kv_heads = int(length), int(kv_heads)
    _check(query_length == length, "Query length differs from the queries tensor")
    _check(kv_heads > 0 and query_heads % kv_heads == 0,
           "Number of heads in key/value must divide number of heads in query")
    groups = query_heads // kv_heads
    if torch.is_grad_enabled() and queries.requires_grad:
        raise RuntimeError("packed_attention: the deterministic attention backward is not "
                           "implemented on the HIP path (forward only)")
    _check(queries.dtype in (torch.float16, torch.bfloat16),
           "FlashAttention only supports fp16 and bf16 data type")
    _check(keys.dtype == queries.dtype and values.dtype == queries.dtype,
           "query and key must have the same dtype")
    for tensor in (queries, keys, values):
        _check(tensor.is_cuda, "Expected contiguous CUDA tensor")
        _check(tensor.device == queries.device, "CUDA devices differ")
    _check(dimension in (64, 128, 256), "Head dimension must be 64, 128 or 256")
    _check(queries.stride(-1) == 1, "Input tensor must have contiguous last dimension")
    keys = keys.reshape(-1, dimension)
    values = values.reshape(-1, dimension)
    _check(keys.is_contiguous() and values.is_contiguous(), "Expected contiguous CUDA tensor")
    _check(keys.shape == values.shape, "Keys and values differ in shape")
    cumulative = metadata.cu_seqlens_k
    segments = batch * kv_heads
    _check(cumulative.is_cuda and cumulative.dtype == torch.int32 and cumulative.is_contiguous()
           and cumulative.numel() == segments + 1, "cu_seqlens_k must have shape (batch_size + 1)")
    _check(cumulative.device == queries.device, "CUDA devices differ")
    decoding = metadata.decoding_cu_seqlens_q
    _check(decoding.numel() == segments + 1, "cu_seqlens_q must have shape (batch_size + 1)")
    max_keys = int(metadata.max_seqlen_k)
    _check(max_keys >= 0, "Invalid max_seqlen_k")
    scale = dimension ** -0.5
    device = queries.device
    with torch.cuda.device(device):
        out = torch.empty((batch, length, query_heads, dimension), dtype=queries.dtype,
                          device=device)
        stream = _lib.stream_of(queries)
        size = _lib.load().lr_packed_attention_workspace_bytes(segments, groups, length,
                                                               max_keys, dimension)
        workspace = torch.empty(size, dtype=torch.uint8, device=device) if size else None
        _lib.call("lr_packed_attention", queries.data_ptr(), queries.stride(0), queries.stride(1),
                  queries.stride(2), _lib.ptr(keys), _lib.ptr(values), keys.shape[0],
                  cumulative.data_ptr(), batch, kv_heads, groups, length, dimension,
                  _lib.DTYPE_CODES[queries.dtype], max_keys, float(scale), out.data_ptr(),
                  None if workspace is None else workspace.data_ptr(),
                  0 if workspace is None else workspace.numel(), stream)
    return out.view(batch, length, query_heads * dimension)
