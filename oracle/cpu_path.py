"""The reference's CPU math path (LAZY_RECALL_BUILD_CUDA=0), restated with torch-CPU ops.

Test infrastructure and the timed CPU baseline of bench.py — never a product path.

  temporal_head_scores_cpu   src/lazy_recall/scoring.py:61-149 (temporal_head_scores_reference)
  pool_cpu                   src/lazy_recall/scoring.py:336-353 (F.max_pool1d per segment)
  refine_cpu                 src/lazy_recall/selection.py:52-88 (CPU torch.topk)
  compact_cpu                src/lazy_recall/cache.py:162-167 (keep mask + index_select)
  audit_step_cpu             score -> pool -> select -> compact for a whole synthetic cache

The operations are the reference's own torch calls (the CPU path *is* these library
routines), which is why this file reads like the reference function by function.
"""

from __future__ import annotations

import math
from typing import List

import numpy as np
import torch
import torch.nn.functional as F

from .selection import Selection, refine_arrays


def _risk_from_margin_drop(base_margin: torch.Tensor, margin_drop: torch.Tensor) -> torch.Tensor:
    margin = base_margin.to(dtype=torch.float64)
    compared = margin - margin_drop.to(torch.float64)
    probability = torch.sigmoid(margin)
    return (probability * (margin - compared) - F.softplus(margin)
            + F.softplus(compared)).clamp_min(0.0)


def temporal_head_scores_cpu(queries, query_positions, keys, key_positions, values,
                             candidate_start, candidate_end, margin_gradient, base_margin,
                             denominator_epsilon, query_chunk_size):
    """scoring.py:75-149 on CPU tensors: queries [W, G, d] bf16, keys/values [T, d] bf16."""
    gradient = margin_gradient.float()
    all_value_gradient = torch.matmul(gradient, values.float().transpose(0, 1))
    value_gradient = all_value_gradient[:, candidate_start:candidate_end]
    count = candidate_end - candidate_start
    minimum = torch.full((count,), torch.inf, dtype=torch.float32)
    maximum = torch.full_like(minimum, -torch.inf)
    key_transpose = keys.transpose(0, 1)
    for start in range(0, queries.shape[0], query_chunk_size):
        end = min(start + query_chunk_size, queries.shape[0])
        logits = torch.matmul(queries[start:end].to(keys.dtype), key_transpose) / math.sqrt(keys.shape[-1])
        causal = key_positions.reshape(1, 1, -1) <= query_positions[start:end].reshape(-1, 1, 1)
        logits = logits.masked_fill(~causal, -torch.inf)
        probabilities = F.softmax(logits.float(), dim=-1)
        output_gradient = torch.matmul(probabilities.transpose(0, 1),
                                       all_value_gradient.unsqueeze(-1)).squeeze(-1).transpose(0, 1)
        candidate = probabilities[:, :, candidate_start:candidate_end]
        ratio = candidate / (1.0 - candidate).clamp_min(denominator_epsilon)
        drop = (ratio * (value_gradient.reshape(1, *value_gradient.shape)
                         - output_gradient.unsqueeze(-1))).sum(dim=1)
        minimum = torch.minimum(minimum, drop.amin(dim=0))
        maximum = torch.maximum(maximum, drop.amax(dim=0))
    return torch.maximum(_risk_from_margin_drop(base_margin, minimum),
                         _risk_from_margin_drop(base_margin, maximum)).to(torch.float32)


def pool_cpu(scores: torch.Tensor, cumulative_ends: List[int], kernel_size: int = 7) -> torch.Tensor:
    parts, start = [], 0
    for end in cumulative_ends:
        parts.append(F.max_pool1d(scores[start:end].reshape(1, 1, -1), kernel_size=kernel_size,
                                  stride=1, padding=kernel_size // 2).reshape(-1))
        start = end
    return torch.cat(parts, dim=0)


def refine_cpu(raw: torch.Tensor, pooled: torch.Tensor, ends, position_starts, count) -> Selection:
    return refine_arrays(raw.numpy(), pooled.numpy(), ends, position_starts, count, tie="torch")


def compact_cpu(keys, values, positions, absolute_removed):
    keep = torch.ones(positions.shape[0], dtype=torch.bool)
    keep[torch.as_tensor(absolute_removed, dtype=torch.long)] = False
    keep_indices = torch.nonzero(keep, as_tuple=False).reshape(-1)
    return (keys.index_select(0, keep_indices), values.index_select(0, keep_indices),
            positions.index_select(0, keep_indices))


def audit_step_cpu(layers, query_positions, margin, count, protect_recent=32, pool_kernel=7,
                   epsilon=1e-6, query_chunk_size=250):
    """One audit step over CPU layer states (dicts with keys, values, positions [rows],
    head_lens, queries [Hq, W, d], gradient [Hq, d]): score every head, pool, refine, compact.
    Returns (scores, pooled, selection, compacted layers)."""
    scores, ends, segments, starts = [], [], [], []
    running = 0
    for layer_index, layer in enumerate(layers):
        head_lens = layer["head_lens"]
        hq = layer["queries"].shape[0]
        groups = hq // len(head_lens)
        bounds = np.concatenate(([0], np.cumsum(head_lens)))
        for head, length in enumerate(head_lens):
            first, last = 0, max(0, int(length) - protect_recent)
            if last <= first:
                continue
            rows = slice(int(bounds[head]), int(bounds[head + 1]))
            mapped = layer["queries"][head * groups:(head + 1) * groups].permute(1, 0, 2)
            part = temporal_head_scores_cpu(
                mapped, query_positions, layer["keys"][rows], layer["positions"][rows],
                layer["values"][rows], first, last,
                layer["gradient"][head * groups:(head + 1) * groups], margin, epsilon,
                query_chunk_size)
            scores.append(part)
            running += last - first
            ends.append(running)
            segments.append((layer_index, head))
            starts.append(first)
    raw = torch.cat(scores)
    if not torch.isfinite(raw).all():
        raise RuntimeError("LazyRecall produced non-finite scores; refusing to construct a deletion queue")
    pooled = pool_cpu(raw, ends, pool_kernel)
    selection = refine_cpu(raw, pooled, ends, starts, count)
    removals = selection.groups(segments)
    compacted = []
    for layer_index, layer in enumerate(layers):
        bounds = np.concatenate(([0], np.cumsum(layer["head_lens"])))
        absolute = [int(bounds[h]) + int(p) for (l, h), ps in removals.items() if l == layer_index
                    for p in ps]
        compacted.append(compact_cpu(layer["keys"], layer["values"], layer["positions"], absolute))
    return raw, pooled, selection, compacted
