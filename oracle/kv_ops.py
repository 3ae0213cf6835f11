"""Data-movement oracle (numpy; test infrastructure only).

Every function restates one reference operation on host arrays. K/V arrays may be any numpy
dtype (bf16 tensors are passed as uint16 bit patterns) because the operations only move rows.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def compact(keys, values, positions, removed):
    """csrc/scoring.cu:164-188 (and the CPU branch cache.py:162-167): drop the sorted, unique
    row indices ``removed`` from K, V and the position column."""
    removed = np.asarray(removed, dtype=np.int64)
    keep = np.ones(keys.shape[0], dtype=bool)
    keep[removed] = False
    return keys[keep], values[keep], np.asarray(positions).reshape(-1)[keep].reshape(-1, 1)


def compact_by_gather_rule(keys, values, positions, removed):
    """The reference kernel's own gather rule, written out (csrc/scoring.cu:172-187): output
    row r reads input row r + #{i : removed[i] - i <= r}."""
    removed = np.asarray(removed, dtype=np.int64)
    rows = keys.shape[0] - removed.size
    shifted = removed - np.arange(removed.size)
    source = np.arange(rows) + np.searchsorted(shifted, np.arange(rows), side="right")
    pos = np.asarray(positions).reshape(-1)
    return keys[source], values[source], pos[source].reshape(-1, 1)


def append(keys, values, positions, new_keys, new_values, cumulative, logical_start, maximum_length):
    """csrc/scoring.cu:130-162,264-292: head h's rows move to cumulative[h] + h*A, followed by
    the A new rows of new_keys[0, h]; new positions are logical_start + i. Rows beyond
    maximum_length + A of a head are not written by the reference and are returned as zeros."""
    cumulative = np.asarray(cumulative, dtype=np.int64)
    positions = np.asarray(positions, dtype=np.float32).reshape(-1)
    _, heads, added, dim = new_keys.shape
    rows = keys.shape[0] + heads * added
    out_k = np.zeros((rows, dim), dtype=keys.dtype)
    out_v = np.zeros((rows, dim), dtype=values.dtype)
    out_p = np.zeros((rows,), dtype=np.float32)
    out_cum = np.zeros(heads + 1, dtype=np.int32)
    out_len = np.zeros(heads, dtype=np.int32)
    covered = maximum_length + added
    for h in range(heads):
        start, length = cumulative[h], cumulative[h + 1] - cumulative[h]
        new_start = start + h * added
        out_cum[h] = new_start
        out_len[h] = length + added
        n_old = min(length, covered)
        out_k[new_start:new_start + n_old] = keys[start:start + n_old]
        out_v[new_start:new_start + n_old] = values[start:start + n_old]
        out_p[new_start:new_start + n_old] = positions[start:start + n_old]
        n_new = max(0, min(length + added, covered) - length)
        out_k[new_start + length:new_start + length + n_new] = new_keys[0, h, :n_new]
        out_v[new_start + length:new_start + length + n_new] = new_values[0, h, :n_new]
        out_p[new_start + length:new_start + length + n_new] = (
            logical_start + np.arange(n_new)).astype(np.float32)
    out_cum[heads] = cumulative[heads] + heads * added
    return out_k, out_v, out_p.reshape(-1, 1), out_cum, out_len


def append_flattened_cache(cache, states, head_lens):
    """_core/cuda_ops.py:38-62 (append_flattened_cache_pytorch): per flat head, its old rows
    then its new [N, D] states."""
    batch, heads, new_length, dim = states.shape
    parts, offset = [], 0
    for flat in range(batch * heads):
        length = int(head_lens[flat])
        if length:
            parts.append(cache[offset:offset + length])
        parts.append(states[flat // heads, flat % heads])
        offset += length
    if not parts:
        return cache[:0]
    return np.concatenate(parts, axis=0).reshape(-1, dim)


def compact_flattened_kv(keys, values, keep_indices):
    """_core/cuda_ops.py:65-76 CPU branch: index_select of kept rows."""
    keep = np.asarray(keep_indices, dtype=np.int64)
    return keys[keep], values[keep]


def merge(keys, values, positions, recalled, recalled_positions, mapping):
    """csrc/recall.cu:7-28 and the CPU branch cache.py:240-245: mapping >= 0 selects an
    existing row, -(i+1) selects recalled row i (K = recalled[i,0], V = recalled[i,1])."""
    mapping = np.asarray(mapping, dtype=np.int64)
    old = keys.shape[0]
    gather = np.where(mapping >= 0, mapping, old - mapping - 1)
    all_k = np.concatenate((keys, recalled[:, 0]))
    all_v = np.concatenate((values, recalled[:, 1]))
    all_p = np.concatenate((np.asarray(positions, dtype=np.float32).reshape(-1),
                            np.asarray(recalled_positions, dtype=np.float32).reshape(-1)))
    return all_k[gather], all_v[gather], all_p[gather].reshape(-1, 1)


def pack(keys, values, positions, indices, heads, layer):
    """csrc/recall.cu:30-47: payload[r] = (K[idx], V[idx]); metadata[r] = (layer, head,
    int64(position)) with C truncation of the float position."""
    indices = np.asarray(indices, dtype=np.int64)
    payload = np.stack((keys[indices], values[indices]), axis=1)
    pos = np.asarray(positions, dtype=np.float32).reshape(-1)[indices]
    metadata = np.stack((np.full(indices.shape, layer, dtype=np.int64),
                         np.asarray(heads, dtype=np.int64),
                         np.trunc(pos).astype(np.int64)), axis=1)
    return payload, metadata


def batch_append(keys: Sequence, values: Sequence, positions: Sequence, new_keys, new_values,
                 lengths: Sequence[Sequence[int]], logical_positions: Sequence[int]):
    """csrc/batch_append.cu:8-94 (equivalently batch_attention.py:30-38 per request): one packed
    buffer ordered (request, head), each head's old rows followed by its one new row."""
    parts_k, parts_v, parts_p = [], [], []
    for r, head_lengths in enumerate(lengths):
        pos = np.asarray(positions[r], dtype=np.float32).reshape(-1)
        offset = 0
        for h, length in enumerate(head_lengths):
            parts_k.append(keys[r][offset:offset + length])
            parts_v.append(values[r][offset:offset + length])
            parts_p.append(pos[offset:offset + length])
            parts_k.append(new_keys[r, h, 0][None])
            parts_v.append(new_values[r, h, 0][None])
            parts_p.append(np.asarray([logical_positions[r]], dtype=np.float32))
            offset += length
    return (np.concatenate(parts_k), np.concatenate(parts_v),
            np.concatenate(parts_p).reshape(-1, 1))


def pool(scores, bounds, width):
    """csrc/scoring.cu:190-203: per segment [bounds[s], bounds[s+1]) sliding max of odd
    width; neighbours outside the segment do not exist and NaN neighbours are ignored (fmaxf)."""
    scores = np.asarray(scores, dtype=np.float32)
    out = np.empty_like(scores)
    half = width // 2
    for s in range(len(bounds) - 1):
        begin, end = int(bounds[s]), int(bounds[s + 1])
        seg = scores[begin:end]
        n = seg.size
        padded = np.full(n + 2 * half, -np.inf, dtype=np.float32)
        padded[half:half + n] = seg
        windows = np.lib.stride_tricks.sliding_window_view(padded, width)
        out[begin:end] = np.fmax.reduce(windows, axis=1, initial=-np.inf) if n else seg
    return out


def merge_plan(old_positions, head_lengths, recalled_metadata) -> Tuple[np.ndarray, List[int]]:
    """recall/planning.py:34-52: per head, stable argsort of existing + recalled positions ->
    source mapping (>= 0 existing row, -(i+1) recalled row i) and new head lengths."""
    old_positions = np.asarray(old_positions, dtype=np.int64).reshape(-1)
    meta = np.asarray(recalled_metadata, dtype=np.int64).reshape(-1, 3)
    if sum(head_lengths) != len(old_positions):
        raise ValueError("Position lengths do not match metadata")
    mapping, lengths, start = [], [], 0
    for head, length in enumerate(head_lengths):
        existing = old_positions[start:start + length]
        chosen = np.flatnonzero(meta[:, 1] == head)
        combined = np.concatenate((existing, meta[chosen, 2]))
        if len(np.unique(combined)) != len(combined):
            raise ValueError("Cannot merge duplicate physical KV identities")
        sources = np.concatenate((np.arange(start, start + length), -chosen - 1))
        mapping.extend(sources[np.argsort(combined, kind="stable")])
        lengths.append(len(combined))
        start += length
    return np.asarray(mapping, dtype=np.int64), lengths
