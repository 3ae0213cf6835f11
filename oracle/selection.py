"""Selection oracle (numpy / CPU torch; test infrastructure only).

Restates refine_arrays and transplant (src/lazy_recall/selection.py:42-88) and the controller's
evict-prefix position remap (src/lazy_recall/controller.py:57-70).

Two tie rules are provided for the two bottom-k steps:
  "canonical"  ties broken by ascending index (a stable sort of (value, index)) — the rule the
               HIP selection implements;
  "torch"      CPU torch.topk(largest=False, sorted=True), the routine the reference calls on
               its CPU path; its order inside a group of equal values is unspecified.
Both agree whenever the k-th value is not tied across the cut.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Selection:
    values: np.ndarray       # f32 [count], ascending raw scores
    segments: np.ndarray     # i64 [count], segment id of each slot
    positions: np.ndarray    # i64 [count], refined position (position_start + local)
    changed: int             # refined picks not among the raw picks
    changed_heads: int       # segments with at least one changed pick
    quotas: np.ndarray       # i64 [segments]

    def groups(self, coordinates):
        """selection.py:29-39: per (layer, head) the sorted refined positions."""
        grouped = {}
        for s in np.unique(self.segments):
            layer, head = coordinates[int(s)]
            grouped[(int(layer), int(head))] = np.sort(self.positions[self.segments == s])
        return grouped


def bottom_k(values: np.ndarray, k: int, tie: str = "canonical"):
    """k smallest (indices, values), ascending, ties by the chosen rule."""
    values = np.asarray(values, dtype=np.float32)
    if tie == "torch":
        import torch

        result = torch.topk(torch.from_numpy(values.copy()), k, largest=False, sorted=True)
        return result.indices.numpy().astype(np.int64), result.values.numpy()
    order = np.lexsort((np.arange(values.size), values))[:k]
    return order.astype(np.int64), values[order]


def transplant(segment_ids, local_positions):
    """selection.py:42-49: each head's refined selections, in order, fill that head's slots in
    the order the slots appear."""
    order = np.argsort(segment_ids, kind="stable")
    result = np.empty(len(segment_ids), dtype=np.int64)
    result[order] = local_positions
    return result


def refine_arrays(raw, pooled, ends, position_starts, count, tie: str = "canonical") -> Selection:
    """selection.py:52-88: global bottom-`count` on raw scores fixes each segment's quota; each
    segment then takes its bottom-quota on pooled scores; results are transplanted into the
    global slots."""
    raw = np.asarray(raw, dtype=np.float32)
    pooled = np.asarray(pooled, dtype=np.float32)
    ends = np.asarray(ends, dtype=np.int64)
    starts = np.concatenate(([0], ends[:-1]))
    position_starts = np.asarray(position_starts, dtype=np.int64)
    count = min(max(0, int(count)), raw.size)
    if not count:
        empty = np.empty(0, dtype=np.int64)
        return Selection(np.empty(0, np.float32), empty, empty, 0, 0, np.zeros(len(ends), np.int64))
    indices, values = bottom_k(raw, count, tie)
    segment_ids = np.searchsorted(ends, indices, side="right")
    quotas = np.bincount(segment_ids, minlength=len(ends))
    selected_local, selected_segments = [], []
    for s, (start, end, quota) in enumerate(zip(starts, ends, quotas)):
        if quota:
            local, _ = bottom_k(pooled[start:end], int(quota), tie)
            selected_local.append(local)
            selected_segments.extend([s] * int(quota))
    selected_local = np.concatenate(selected_local)
    selected_segments = np.asarray(selected_segments, dtype=np.int64)
    positions = transplant(segment_ids, selected_local + position_starts[selected_segments])
    refined_global = selected_local + starts[selected_segments]
    changed = ~np.isin(refined_global, indices, assume_unique=True)
    changed_heads = np.unique(selected_segments[changed]).size
    return Selection(values, segment_ids.astype(np.int64), positions, int(changed.sum()),
                     int(changed_heads), quotas.astype(np.int64))


def evict_prefix_remap(positions, removed_at_audit):
    """controller.py:63-66: positions selected at audit time shift down by the number of
    earlier removals of the same head."""
    removed = np.asarray(removed_at_audit, dtype=np.int64)
    positions = np.asarray(positions, dtype=np.int64)
    return positions - np.searchsorted(removed, positions), np.union1d(removed, positions)
