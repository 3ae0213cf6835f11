"""Query-history oracle (test infrastructure only): the reference's QueryHistory
(src/lazy_recall/history.py:11-63) restated on numpy arrays, one bounded deque per layer plus
one of positions, and ``layer`` as the concatenation of a layer's deque along the query axis.
"""

from __future__ import annotations

from collections import deque

import numpy as np


class QueryHistory:
    def __init__(self, num_layers: int, window_size: int) -> None:
        """history.py:12-19"""
        if int(window_size) <= 0:
            raise ValueError("temporal window must be positive")
        self.window_size = int(window_size)
        self.queries = [deque(maxlen=self.window_size) for _ in range(int(num_layers))]
        self.positions = deque(maxlen=self.window_size)

    def append(self, queries, absolute_position: int) -> None:
        """history.py:21-38 (queries: one [1, Hq, 1, d] array per layer)."""
        if len(queries) != len(self.queries):
            raise RuntimeError("Query-history layer count mismatch")
        position = int(absolute_position)
        if self.positions and position <= self.positions[-1]:
            raise RuntimeError("Query positions must be strictly increasing")
        self.positions.append(position)
        for layer_index, query in enumerate(queries):
            if query.shape[0] != 1 or query.shape[2] != 1:
                raise RuntimeError(f"Expected one decode query at layer {layer_index}")
            self.queries[layer_index].append(np.array(query))

    def layer(self, layer_index: int):
        """history.py:51-63: ([1, Hq, n, d], positions [n] int64)."""
        history = self.queries[layer_index]
        if not history:
            raise RuntimeError(f"No query history for layer {layer_index}")
        return np.concatenate(list(history), axis=2), np.asarray(list(self.positions), np.int64)
