"""Device-resident query history: the reference's QueryHistory (src/lazy_recall/history.py:11-78)
with the same constructor, methods, checks and messages, kept in one doubled ring on the GPU.

The reference holds a deque of per-step [1, Hq, 1, d] tensors per layer and builds each layer's
window with ``torch.cat`` (plus a blocking ``torch.tensor`` of the positions) at every audit
(history.py:51-63). Here every append is one launch (``lr_history_append``) that writes all
layers' queries into a [layers, Hq, 2W, d] ring, and ``layer`` returns a strided view of the ring
and of its [2W] position array: no copy, no host-to-device transfer, and the fused scorer reads
the window where it lies (its query-head stride is 2W rows).

Views alias the ring: an append after ``layer``/``audit_window`` overwrites the oldest row the
view shows (stream-ordered on the appending stream). A caller that keeps a window across appends
clones it; the audit step consumes it before the next append, as the reference's audit does.
"""

from __future__ import annotations

import ctypes
from collections import deque
from typing import Deque, List, Sequence, Tuple

import torch

from . import _lib

_RING_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


class QueryHistory:
    def __init__(self, num_layers: int, window_size: int) -> None:
        self.window_size = int(window_size)
        if self.window_size <= 0:
            raise ValueError("temporal window must be positive")
        self.num_layers = int(num_layers)
        self._positions: Deque[int] = deque(maxlen=self.window_size)
        self._appended = 0
        self._ring = None            # [layers, Hq, 2W, d]
        self._ring_positions = None  # [2W] int64

    def _allocate(self, query: torch.Tensor) -> None:
        if not query.is_cuda:
            raise RuntimeError("QueryHistory keeps its ring on the GPU; queries must be CUDA tensors")
        if query.dtype not in _RING_DTYPES:
            raise RuntimeError(f"Query history holds bf16, f16 or f32 queries, got {query.dtype}")
        heads, dim = query.shape[1], query.shape[3]
        self._ring = torch.empty((self.num_layers, heads, 2 * self.window_size, dim),
                                 dtype=query.dtype, device=query.device)
        self._ring_positions = torch.empty((2 * self.window_size,), dtype=torch.int64,
                                           device=query.device)

    def append(self, queries: Sequence[torch.Tensor], absolute_position: int) -> None:
        """history.py:21-38. Everything is checked before anything is written."""
        if len(queries) != self.num_layers:
            raise RuntimeError("Query-history layer count mismatch")
        position = int(absolute_position)
        if self._positions and position <= self._positions[-1]:
            raise RuntimeError("Query positions must be strictly increasing")
        for layer_index, query in enumerate(queries):
            if query.dim() != 4 or query.shape[0] != 1 or query.shape[2] != 1:
                raise RuntimeError(
                    f"Expected one decode query at layer {layer_index}, got "
                    f"{tuple(query.shape)}"
                )
        if self._ring is None:
            self._allocate(queries[0])
        ring = self._ring
        expected = (1, ring.shape[1], 1, ring.shape[3])
        sources = []
        for query in queries:
            if (tuple(query.shape) != expected or query.dtype != ring.dtype
                    or query.device != ring.device):
                raise RuntimeError("Query-history layer shape mismatch")
            sources.append(query.detach().contiguous())
        slot = self._appended % self.window_size
        pointers = (ctypes.c_void_p * len(sources))(*[q.data_ptr() for q in sources])
        with torch.cuda.device(ring.device):
            _lib.call("lr_history_append", pointers, len(sources), ring.shape[1], ring.shape[3],
                      ring.element_size(), self.window_size, slot, ring.data_ptr(), position,
                      self._ring_positions.data_ptr(), _lib.stream_of(ring))
        self._positions.append(position)
        self._appended += 1

    def capture_model(self, model, absolute_position: int) -> None:
        """history.py:40-49"""
        queries = []
        for layer_index, layer in enumerate(model.model.layers):
            query = getattr(layer.self_attn, "_last_query_states", None)
            if query is None:
                raise RuntimeError(
                    f"Layer {layer_index} did not expose _last_query_states"
                )
            queries.append(query.detach())
        self.append(queries, absolute_position)

    def _window(self) -> Tuple[int, int]:
        count = len(self._positions)
        start = self._appended % self.window_size if self._appended >= self.window_size else 0
        return start, count

    def layer(self, layer_index: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """history.py:51-63: (queries [1, Hq, n, d], positions [n] int64), oldest first, as
        views of the ring."""
        if not self._positions or not 0 <= layer_index < self.num_layers:
            raise RuntimeError(f"No query history for layer {layer_index}")
        start, count = self._window()
        queries = self._ring[layer_index, :, start:start + count].unsqueeze(0)
        return queries, self._ring_positions[start:start + count]

    def audit_window(self) -> Tuple[List[torch.Tensor], torch.Tensor]:
        """Every layer's window as the fused scorer takes it ([Hq, n, d] views with a query-head
        stride of 2W rows) and the shared positions [n] int64."""
        if not self._positions:
            raise RuntimeError("No query history for layer 0")
        start, count = self._window()
        return ([self._ring[l, :, start:start + count] for l in range(self.num_layers)],
                self._ring_positions[start:start + count])

    @property
    def size(self) -> int:
        return len(self._positions)

    @property
    def positions(self) -> Tuple[int, ...]:
        return tuple(self._positions)

    @property
    def retained_bytes(self) -> int:
        """The bytes of the queries the window holds (history.py:73-78)."""
        if self._ring is None:
            return 0
        per_query = self._ring.shape[1] * self._ring.shape[3] * self._ring.element_size()
        return self.num_layers * len(self._positions) * per_query

    @property
    def allocated_bytes(self) -> int:
        """Device bytes of the ring and its positions (twice the full window)."""
        if self._ring is None:
            return 0
        return (self._ring.numel() * self._ring.element_size()
                + self._ring_positions.numel() * self._ring_positions.element_size())
