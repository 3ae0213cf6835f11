"""Host-side recall merge planning (src/lazy_recall/recall/planning.py:34-52).

``merge_plan`` returns the same mapping and head lengths as the reference: per KV head, the
existing rows followed by that head's recalled rows, stably ordered by absolute position;
mapping >= 0 selects existing row i, -(i+1) selects recalled row i. The reference loops over
heads with one argsort each; this version orders every head at once with a single lexsort.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def merge_plan(old_positions, head_lengths: Sequence[int],
               recalled_metadata) -> Tuple[np.ndarray, List[int]]:
    old_positions = np.asarray(old_positions, dtype=np.int64).reshape(-1)
    meta = np.asarray(recalled_metadata, dtype=np.int64).reshape(-1, 3)
    lengths = np.asarray(head_lengths, dtype=np.int64)
    if int(lengths.sum()) != len(old_positions):
        raise ValueError("Position lengths do not match metadata")
    heads = lengths.size
    head_of_old = np.repeat(np.arange(heads, dtype=np.int64), lengths)
    head_of_new = meta[:, 1]
    if head_of_new.size and (head_of_new.min() < 0 or head_of_new.max() >= heads):
        # rows of heads outside this layer's head range are ignored, as in the reference loop
        keep = (head_of_new >= 0) & (head_of_new < heads)
        chosen = np.flatnonzero(keep)
    else:
        chosen = np.arange(len(meta))
    head = np.concatenate((head_of_old, head_of_new[chosen]))
    position = np.concatenate((old_positions, meta[chosen, 2]))
    source = np.concatenate((np.arange(len(old_positions), dtype=np.int64), -chosen - 1))
    tiebreak = np.arange(head.size)  # existing rows first, then recalled rows, in input order
    order = np.lexsort((tiebreak, position, head))
    sorted_head, sorted_position = head[order], position[order]
    duplicate = (sorted_head[1:] == sorted_head[:-1]) & (sorted_position[1:] == sorted_position[:-1])
    if duplicate.any():
        raise ValueError("Cannot merge duplicate physical KV identities")
    new_lengths = np.bincount(head, minlength=heads)
    return source[order], new_lengths.tolist()
