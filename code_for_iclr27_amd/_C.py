"""Drop-in for the reference module ``lazy_recall._C`` (csrc/bindings.cpp:20-29).

Same eight functions, argument order, return arity, validation and error type (RuntimeError)
as the reference's pybind launchers in csrc/scoring.cu:205-329, csrc/recall.cu:49-111 and
csrc/batch_append.cu:36-94. Each function validates its tensors, allocates outputs with torch
on the input's device and launches the HIP kernels of liblazyrecall_hip.so on the current
stream. There is no CPU path: CPU tensors are rejected exactly as the reference rejects them.
"""

from __future__ import annotations

from typing import List

import numpy as np
import torch

from . import _lib

_FLOATING = (torch.float32, torch.float64, torch.float16, torch.bfloat16)


def _check(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _check_cuda(tensor: torch.Tensor, reference: torch.Tensor) -> None:
    # csrc/scoring.cu:10-13
    _check(tensor.is_cuda and tensor.is_contiguous(), "Expected contiguous CUDA tensor")
    _check(tensor.device == reference.device, "CUDA devices differ")


def _elem_bytes(tensor: torch.Tensor, op: str) -> int:
    if tensor.dtype not in _FLOATING:
        raise RuntimeError(f'"{op}" not implemented for \'{tensor.dtype}\'')
    return tensor.element_size()


def temporal_probabilities(logits, projected_values, query_positions, key_positions, scale):
    """csrc/scoring.cu:205-233 -> [probabilities f32 [W,G,T], output_projection f32 [W,G]]."""
    for tensor in (logits, projected_values, query_positions, key_positions):
        _check_cuda(tensor, logits)
    _check(logits.dim() == 3, "logits must be [window, groups, positions]")
    _check(logits.dtype in (torch.float32, torch.float16, torch.bfloat16),
           "Only FP32/FP16/BF16 scores are supported")
    window, groups, length = logits.shape
    _check(window > 0 and groups > 0 and length > 0, "Empty attention dimensions")
    _check(projected_values.dtype == torch.float32 and projected_values.dim() == 2
           and projected_values.size(0) == groups and projected_values.size(1) == length,
           "Invalid projected values")
    _check(query_positions.dtype == torch.int64 and query_positions.numel() == window,
           "Invalid query positions")
    _check(key_positions.dtype == torch.float32 and key_positions.numel() == length,
           "Invalid key positions")
    with torch.cuda.device(logits.device):
        probabilities = torch.empty(logits.shape, dtype=torch.float32, device=logits.device)
        output = torch.empty((window, groups), dtype=torch.float32, device=logits.device)
        _lib.call("lr_temporal_probabilities", logits.data_ptr(), _lib.DTYPE_CODES[logits.dtype],
                  projected_values.data_ptr(), query_positions.data_ptr(), key_positions.data_ptr(),
                  window, groups, length, float(scale), probabilities.data_ptr(), output.data_ptr(),
                  _lib.stream_of(logits))
    return [probabilities, output]


def temporal_risk(probabilities, output_projection, projected_values, margin, first, last, epsilon):
    """csrc/scoring.cu:235-255 -> scores f32 [last - first]."""
    for tensor in (probabilities, output_projection, projected_values, margin):
        _check_cuda(tensor, probabilities)
        _check(tensor.dtype == torch.float32, "Risk inputs must be float32")
    _check(probabilities.dim() == 3, "Invalid probability dimensions")
    window, groups, length = probabilities.shape
    first, last = int(first), int(last)
    _check(window > 0 and groups > 0 and first >= 0 and last > first and last <= length
           and epsilon > 0, "Invalid risk interval")
    _check(margin.numel() == 1 and output_projection.numel() == window * groups
           and projected_values.numel() == groups * length, "Risk shapes differ")
    with torch.cuda.device(probabilities.device):
        result = torch.empty((last - first,), dtype=torch.float32, device=probabilities.device)
        _lib.call("lr_temporal_risk", probabilities.data_ptr(), output_projection.data_ptr(),
                  projected_values.data_ptr(), margin.data_ptr(), window, groups, length, first,
                  last, float(epsilon), result.data_ptr(), _lib.stream_of(probabilities))
    return result


_native_module = None


def _native():
    """The C++ host module with lr_append / lr_compact bound (once): the per-layer decode-time
    ops run their checks, allocate their outputs and launch from C++ on torch's current stream."""
    global _native_module
    if _native_module is None:
        import ctypes
        from .scoring import _planner
        planner = _planner()
        library = _lib.load()
        address = lambda name: ctypes.cast(getattr(library, name), ctypes.c_void_p).value
        planner.bind_data_movement(address("lr_append"), address("lr_compact"),
                                   address("lr_append_layers"), address("lr_batch_append"),
                                   address("lr_batch_append_host"),
                                   address("lr_append_layers_host"))
        _native_module = planner
    return _native_module


def append(keys, values, positions, new_keys, new_values, cumulative, logical_start,
           maximum_length):
    """csrc/scoring.cu:264-292 -> [keys, values, positions [N,1], cumulative i32, lengths i32].
    Checks (csrc/scoring.cu:257-283, same order and messages), allocation and launch are made by
    the C++ host module (csrc/host_plan.cpp append_launch); the integers are converted there."""
    return (_native_module or _native()).append(keys, values, positions, new_keys, new_values,
                                                cumulative, logical_start, maximum_length)


def append_layers(keys, values, positions, new_keys, new_values, cumulative, logical_starts,
                  maximum_length):
    """One decode step's ``append`` into every layer in one launch (an extra export: the
    reference makes one append call per layer, cache.py:33-52). Each argument except
    ``maximum_length`` is a per-layer list, with ``append``'s meaning. Returns [keys, values,
    positions [rows, 1], cumulative i32 [L, H + 1], lengths i32 [L, H], first row of each layer
    [L + 1]]: every layer's rows packed into one buffer, layer l at rows
    [first[l], first[l + 1])."""
    return list(_native().append_layers(list(keys), list(values), list(positions),
                                        list(new_keys), list(new_values), list(cumulative),
                                        [int(v) for v in logical_starts], int(maximum_length)))


def compact(keys, values, positions, removed):
    """csrc/scoring.cu:294-314 -> [keys, values, positions [N-E,1]]; removed sorted, unique.
    Checks, allocation and launch in the C++ host module (csrc/host_plan.cpp compact_launch)."""
    return (_native_module or _native()).compact(keys, values, positions, removed)


def pool(scores, bounds, maximum_count, width):
    """csrc/scoring.cu:316-329 -> per-segment sliding max of odd ``width``."""
    _check_cuda(scores, scores)
    _check_cuda(bounds, scores)
    _check(scores.dtype == torch.float32 and scores.dim() == 1 and bounds.dtype == torch.int64
           and bounds.dim() == 1 and bounds.numel() >= 2, "Invalid pool layout")
    _check(width > 0 and width % 2 == 1 and maximum_count > 0, "Invalid pool configuration")
    with torch.cuda.device(scores.device):
        output = torch.empty_like(scores)
        _lib.call("lr_pool", _lib.ptr(scores), scores.numel(), bounds.data_ptr(),
                  bounds.numel() - 1, int(maximum_count), int(width), _lib.ptr(output),
                  _lib.stream_of(scores))
    return output


def _check_recall(tensor, reference):
    # csrc/recall.cu:49-52
    _check(tensor.is_cuda and tensor.is_contiguous(), "Expected contiguous CUDA tensor")
    _check(tensor.device == reference.device, "Recall devices differ")


def merge(keys, values, positions, recalled, recalled_positions, mapping):
    """csrc/recall.cu:54-84 -> [keys, values, positions [M,1]] gathered through ``mapping``."""
    for tensor in (keys, values, positions, recalled, recalled_positions, mapping):
        _check_recall(tensor, keys)
    _check(keys.dim() == 2 and keys.size(1) > 0 and keys.shape == values.shape,
           "Invalid K/V shape")
    _check(recalled.dim() == 3 and recalled.size(1) == 2 and recalled.size(2) == keys.size(1),
           "Invalid recalled shape")
    _check(keys.dtype == values.dtype and keys.dtype == recalled.dtype, "K/V dtypes differ")
    _check(positions.dtype == torch.float32 and recalled_positions.dtype == torch.float32
           and positions.numel() == keys.size(0)
           and recalled_positions.numel() == recalled.size(0), "Invalid positions")
    _check(mapping.dim() == 1 and mapping.dtype == torch.int64, "Mapping must be int64")
    elem = _elem_bytes(keys, "recall_merge")
    rows, dimension = mapping.numel(), keys.size(1)
    with torch.cuda.device(keys.device):
        output_keys = torch.empty((rows, dimension), dtype=keys.dtype, device=keys.device)
        output_values = torch.empty_like(output_keys)
        output_positions = torch.empty((rows, 1), dtype=positions.dtype, device=keys.device)
        if rows:
            _lib.call("lr_merge", _lib.ptr(keys), _lib.ptr(values), _lib.ptr(positions),
                      keys.size(0), _lib.ptr(recalled), _lib.ptr(recalled_positions),
                      recalled.size(0), mapping.data_ptr(), rows, dimension, elem,
                      output_keys.data_ptr(), output_values.data_ptr(),
                      output_positions.data_ptr(), _lib.stream_of(keys))
    return [output_keys, output_values, output_positions]


def pack(keys, values, positions, indices, heads, layer, payload, metadata):
    """csrc/recall.cu:86-111: gather evicted rows into ``payload``/``metadata`` in place."""
    for tensor in (keys, values, positions, indices, heads, payload, metadata):
        _check_recall(tensor, keys)
    _check(keys.dim() == 2 and keys.size(1) > 0 and keys.shape == values.shape,
           "Invalid K/V shape")
    _check(keys.dtype == values.dtype and keys.dtype == payload.dtype, "Dtype mismatch")
    _check(indices.dim() == 1 and indices.dtype == torch.int64 and heads.shape == indices.shape
           and heads.dtype == torch.int64, "Invalid gather indices")
    rows, dimension = indices.numel(), keys.size(1)
    _check(payload.dim() == 3 and payload.size(0) == rows and payload.size(1) == 2
           and payload.size(2) == dimension, "Invalid payload buffer")
    _check(positions.numel() == keys.size(0) and positions.dtype == torch.float32,
           "Invalid positions")
    _check(metadata.dim() == 2 and metadata.size(0) == rows and metadata.size(1) == 3
           and metadata.dtype == torch.int64, "Invalid identity buffer")
    if not rows:
        return None
    elem = _elem_bytes(keys, "archive_pack")
    with torch.cuda.device(keys.device):
        _lib.call("lr_pack", keys.data_ptr(), values.data_ptr(), positions.data_ptr(),
                  keys.size(0), indices.data_ptr(), heads.data_ptr(), rows, dimension, elem,
                  int(layer), payload.data_ptr(), metadata.data_ptr(), _lib.stream_of(keys))
    return None


def upload_int64(host: np.ndarray, device: torch.device) -> torch.Tensor:
    """Stage an int64 table in pinned memory and copy it to the device without blocking the
    host (the reference's descriptor copy, csrc/batch_append.cu:81, is synchronous)."""
    staging = torch.empty(host.shape, dtype=torch.int64, pin_memory=True)
    staging.numpy()[...] = host
    return staging.to(device, non_blocking=True)


def batch_append(keys: List[torch.Tensor], values: List[torch.Tensor],
                 positions: List[torch.Tensor], new_keys, new_values,
                 lengths: List[List[int]], logical_positions: List[int]):
    """csrc/batch_append.cu:36-94 -> [keys, values, positions [sum(N_r + H), 1]] packed."""
    _check(new_keys.is_cuda and new_keys.is_contiguous() and new_values.is_contiguous(),
           "Contiguous CUDA states required")
    _check(new_keys.dim() == 4 and new_keys.size(2) == 1 and new_keys.size(3) > 0,
           "Only batched one-token append is supported")
    _check(new_keys.shape == new_values.shape and new_keys.dtype == new_values.dtype
           and new_keys.device == new_values.device, "New K/V mismatch")
    requests, heads, dimension = new_keys.size(0), new_keys.size(1), new_keys.size(3)
    _check(requests > 0 and heads > 0 and len(keys) == requests and len(values) == requests
           and len(positions) == requests and len(lengths) == requests
           and len(logical_positions) == requests, "Request metadata mismatch")
    _elem_bytes(new_keys, "batch_append")
    from .audit import _native_planner
    _native_planner()  # binds the staging entry points
    with torch.cuda.device(new_keys.device):
        # csrc/host_plan.cpp: the reference's descriptor loop (csrc/batch_append.cu:49-80) and
        # its checks, the descriptors in the launch's kernel arguments (up to 64 segments) or
        # in host-coherent staging that the kernel reads in place (the reference's copy,
        # csrc/batch_append.cu:81, blocks the host), allocation, launch
        return list(_native().batch_append(keys, values, positions, new_keys, new_values,
                                           lengths, logical_positions,
                                           _lib.stream_of(new_keys)))
