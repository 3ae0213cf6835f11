"""Drop-in for the reference module ``lazy_recall._legacy_C`` (csrc/cache_legacy.cu:304-308).

Three functions with the reference's argument order, checks and messages
(csrc/cache_legacy.cu:137-302), launching liblazyrecall_hip.so on the current stream.
"""

from __future__ import annotations

import torch

from . import _lib
from ._C import _check, _elem_bytes


def _check_flat_matrix(tensor: torch.Tensor, name: str) -> None:
    # csrc/cache_legacy.cu:137-141
    _check(tensor.is_cuda, f"{name} must be CUDA")
    _check(tensor.is_contiguous(), f"{name} must be contiguous")
    _check(tensor.dim() == 2, f"{name} must be rank two")


def append_flattened_cache(cache, states, head_lens, cu_head_lens):
    """csrc/cache_legacy.cu:145-197: insert each head's [N, D] states at the end of its
    segment of the flat [rows, D] cache -> [rows + B*H*N, D]."""
    _check_flat_matrix(cache, "cache")
    _check(states.is_cuda and states.is_contiguous(), "states must be contiguous CUDA")
    _check(states.dim() == 4, "states must have shape [B,H,N,D]")
    _check(cache.dtype == states.dtype, "cache and states must share dtype")
    _check(head_lens.dtype == torch.int32, "head_lens must be int32")
    _check(cu_head_lens.dtype == torch.int32, "cu_head_lens must be int32")
    _check(head_lens.is_cuda and cu_head_lens.is_cuda, "length metadata must be CUDA")
    _check(head_lens.is_contiguous() and cu_head_lens.is_contiguous(),
           "length metadata must be contiguous")
    _check(cache.device == states.device and cache.device == head_lens.device
           and cache.device == cu_head_lens.device, "append inputs must share one CUDA device")
    _check(cache.size(1) == states.size(3), "head_dim mismatch")
    total_heads = states.size(0) * states.size(1)
    new_length, head_dim = states.size(2), cache.size(1)
    _check(head_lens.numel() == total_heads, "head count mismatch")
    _check(cu_head_lens.numel() == total_heads + 1, "cumulative length count mismatch")
    elem = _elem_bytes(cache, "append_flattened_cache")
    with torch.cuda.device(cache.device):
        output = torch.empty((cache.size(0) + total_heads * new_length, head_dim),
                             dtype=cache.dtype, device=cache.device)
        _lib.call("lr_append_flattened_cache", _lib.ptr(cache), cache.size(0), _lib.ptr(states),
                  total_heads, new_length, head_dim, elem, _lib.ptr(head_lens),
                  _lib.ptr(cu_head_lens), _lib.ptr(output), _lib.stream_of(cache))
    return output


def compact_flattened_kv(keys, values, keep_indices):
    """csrc/cache_legacy.cu:199-242: gather ``keep_indices`` rows of K and V."""
    _check_flat_matrix(keys, "keys")
    _check_flat_matrix(values, "values")
    _check(keys.shape == values.shape, "K/V shape mismatch")
    _check(keys.dtype == values.dtype, "K/V dtype mismatch")
    _check(keep_indices.is_cuda and keep_indices.is_contiguous(),
           "keep_indices must be contiguous CUDA")
    _check(keep_indices.dtype == torch.int64, "keep_indices must be int64")
    _check(keep_indices.dim() == 1, "keep_indices must be rank one")
    _check(keys.device == values.device and keys.device == keep_indices.device,
           "compaction inputs must share one CUDA device")
    elem = _elem_bytes(keys, "compact_flattened_kv")
    rows, head_dim = keep_indices.numel(), keys.size(1)
    with torch.cuda.device(keys.device):
        output_keys = torch.empty((rows, head_dim), dtype=keys.dtype, device=keys.device)
        output_values = torch.empty((rows, head_dim), dtype=values.dtype, device=keys.device)
        if rows == 0:
            return [output_keys, output_values]
        _lib.call("lr_compact_flattened_kv", keys.data_ptr(), values.data_ptr(), keys.size(0),
                  head_dim, elem, keep_indices.data_ptr(), rows, output_keys.data_ptr(),
                  output_values.data_ptr(), _lib.stream_of(keys))
    return [output_keys, output_values]


def decision_risk_scores(probabilities, values, head_outputs, gradients, base_margin,
                         denominator_epsilon):
    """csrc/cache_legacy.cu:244-302: frozen local-LOO Bernoulli decision KL per candidate."""
    _check_flat_matrix(probabilities, "probabilities")
    _check_flat_matrix(values, "values")
    _check_flat_matrix(head_outputs, "head_outputs")
    _check_flat_matrix(gradients, "gradients")
    _check(probabilities.dtype == torch.float32, "probabilities must be float32")
    _check(head_outputs.dtype == torch.float32, "head_outputs must be float32")
    _check(gradients.dtype == torch.float32, "gradients must be float32")
    _check(probabilities.size(0) == head_outputs.size(0), "mapped-query-head mismatch")
    _check(head_outputs.shape == gradients.shape, "head output/gradient mismatch")
    _check(probabilities.size(1) == values.size(0), "candidate count mismatch")
    _check(values.size(1) == head_outputs.size(1), "head_dim mismatch")
    _check(probabilities.device == values.device and probabilities.device == head_outputs.device
           and probabilities.device == gradients.device,
           "score inputs must share one CUDA device")
    _check(0.0 < denominator_epsilon < 1.0, "denominator_epsilon must be in (0,1)")
    _elem_bytes(values, "decision_risk_scores")
    groups, candidates = probabilities.shape
    head_dim = values.size(1)
    with torch.cuda.device(values.device):
        scores = torch.empty((candidates,), dtype=torch.float32, device=values.device)
        if candidates == 0:
            return scores
        _lib.call("lr_decision_risk_scores", probabilities.data_ptr(), values.data_ptr(),
                  _lib.DTYPE_CODES[values.dtype], head_outputs.data_ptr(), gradients.data_ptr(),
                  groups, candidates, head_dim, float(base_margin), float(denominator_epsilon),
                  scores.data_ptr(), _lib.stream_of(values))
    return scores
