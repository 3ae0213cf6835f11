"""Allocation-preserving selection on the GPU (src/lazy_recall/selection.py).

``ArrayReferences`` keeps the reference's queue type and API (selection.py:8-39).
``select_refine`` runs refine_arrays + transplant (selection.py:42-88) entirely on the device
(``lr_select_refine``) and returns device tensors without synchronising; ``refine_arrays``
wraps it with the reference's signature and host return values.

Tie rule: where equal scores straddle a bottom-k cut, the lower index is taken (the order of
a stable sort by (score, index)). The reference defers to torch.topk, whose choice inside such
a tie group is unspecified; outside tie groups the two agree exactly.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from typing import Optional, Sequence as Seq

import numpy as np
import torch

from . import _C, _lib


@dataclass(order=True)
class KVReference:
    """_core/scoring.py:214-219: one queued slot. Instances order by score, then layer, head and
    position (dataclass field order), as the reference's."""
    score: float
    layer: int
    head: int
    position: int


class ArrayReferences(Sequence):
    """The deletion-queue type of selection.py:8-39: three parallel columns in queue order (raw
    score, score-segment id, position within the head) and the (layer, head) of every segment.
    An integer index gives a ``KVReference``; a slice gives another queue over the same
    segments."""

    def __init__(self, scores, segments, positions, coordinates):
        self.scores = np.asarray(scores)
        self.segments = np.asarray(segments, dtype=np.int64)
        self.positions = np.asarray(positions, dtype=np.int64)
        self.coordinates = np.asarray(coordinates, dtype=np.int64).reshape(-1, 2)
        if not len(self.scores) == len(self.segments) == len(self.positions):
            raise ValueError("Queue column lengths differ")

    def __len__(self):
        return len(self.positions)

    def __getitem__(self, index):
        if isinstance(index, slice):
            return ArrayReferences(self.scores[index], self.segments[index],
                                   self.positions[index], self.coordinates)
        layer, head = (int(v) for v in self.coordinates[self.segments[index]])
        return KVReference(float(self.scores[index]), layer, head, int(self.positions[index]))

    def groups(self):
        """The queued positions of each (layer, head), ascending, keyed in segment order. One
        sort by (segment, position) covers every head; each head is then one run of it."""
        if not len(self):
            return {}
        order = np.lexsort((self.positions, self.segments))
        segments, positions = self.segments[order], self.positions[order]
        firsts = np.flatnonzero(np.concatenate(([True], segments[1:] != segments[:-1])))
        lasts = np.append(firsts[1:], len(segments))
        coordinates = self.coordinates[segments[firsts]]
        return {(int(layer), int(head)): positions[first:last]
                for (layer, head), first, last in zip(coordinates, firsts, lasts)}


@dataclass
class DeviceSelection:
    """Result of lr_select_refine, resident on the device. When the queue half ran on a side
    stream, ``queue_ready`` is the event that ends it: ``wait_queue()`` orders the current
    stream after it (``references()`` does so itself)."""
    values: Optional[torch.Tensor]   # f32 [count] ascending raw scores (None: queue not ordered)
    segments: Optional[torch.Tensor]  # i64 [count]
    positions: Optional[torch.Tensor]  # i64 [count] transplanted refined positions
    quotas: torch.Tensor             # i64 [S] picks per segment
    offsets: torch.Tensor            # i64 [S + 1] exclusive prefix of quotas
    removed_positions: torch.Tensor  # i64 [count] per-segment ascending positions
    changed: torch.Tensor            # i64 [S] refined picks absent from the raw picks
    coordinates: Seq  # (layer, head) per segment: list of pairs or an int array [S, 2]
    queue_ready: Optional[torch.cuda.Event] = None

    def wait_queue(self) -> None:
        if self.queue_ready is not None:
            torch.cuda.current_stream(self.quotas.device).wait_event(self.queue_ready)
            self.queue_ready = None

    def references(self) -> ArrayReferences:
        if self.values is None:
            raise RuntimeError("the queue order was not computed (select_refine(queue=False))")
        self.wait_queue()
        return ArrayReferences(self.values.cpu().numpy(), self.segments.cpu().numpy(),
                               self.positions.cpu().numpy(), self.coordinates)

    def change_counts(self):
        changed = self.changed.cpu().numpy()
        return int(changed.sum()), int(np.count_nonzero(changed))


class SelectWorkspace:
    """Grow-only device workspace reused across calls. A queue half still running on a side
    stream is waited for (by the current stream) before the buffer is handed out again."""

    def __init__(self):
        self.buffer = None
        self.pending: Optional[torch.cuda.Event] = None

    def get(self, nbytes: int, device) -> torch.Tensor:
        if self.pending is not None:
            torch.cuda.current_stream(device).wait_event(self.pending)
            self.pending = None
        if self.buffer is None or self.buffer.numel() < nbytes or self.buffer.device != device:
            self.buffer = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=device)
        return self.buffer


_workspace = SelectWorkspace()


def select_refine(raw: torch.Tensor, pooled: torch.Tensor, cumulative_ends: Seq[int],
                  position_starts: Seq[int], coordinates, count: int,
                  ends_device: torch.Tensor | None = None,
                  starts_device: torch.Tensor | None = None,
                  workspace: SelectWorkspace | None = None,
                  quotas_out: torch.Tensor | None = None,
                  queue: bool = True,
                  queue_stream: torch.cuda.Stream | None = None) -> DeviceSelection | None:
    """Launch the device selection; returns None when nothing is selected. ``ends_device`` /
    ``starts_device`` may be passed pre-uploaded (i64 device tensors), and then
    ``cumulative_ends`` / ``position_starts`` may be None; ``quotas_out`` (i64
    device [segments]) receives the quotas when given. With ``queue_stream`` the queue order
    (values, segments, positions) is computed there, after the removal sets, concurrently with
    whatever the caller enqueues next on the current stream; the workspace must not be reused
    before ``queue_ready`` (``wait_queue()``). With ``queue=False`` only the removal sets
    (quotas, offsets, removed_positions, changed) are computed: they are all that removing
    every selected slot needs (controller.py:154 groups the removed references per head)."""
    total = raw.numel()
    segments = len(cumulative_ends) if cumulative_ends is not None else ends_device.numel()
    count = min(max(0, int(count)), total)
    if not count:
        return None
    if not (raw.is_cuda and pooled.is_cuda and raw.is_contiguous() and pooled.is_contiguous()
            and raw.dtype == torch.float32 and pooled.dtype == torch.float32
            and pooled.numel() == total):
        raise RuntimeError("Allocation and refinement layouts differ")
    device = raw.device
    if ends_device is None or starts_device is None:
        table = _C.upload_int64(np.stack((np.asarray(cumulative_ends, np.int64),
                                          np.asarray(position_starts, np.int64))), device)
        ends_device, starts_device = table[0], table[1]
    workspace = workspace or _workspace
    nbytes = _lib.load().lr_select_workspace_bytes(total, segments, count)
    buffer = workspace.get(nbytes, device)
    out = torch.empty((3 * count + 2 * segments + 1,), dtype=torch.int64, device=device)
    values = torch.empty((count,), dtype=torch.float32, device=device)
    seg_ids, positions, removed = out[:count], out[count:2 * count], out[2 * count:3 * count]
    quotas = out[3 * count:3 * count + segments] if quotas_out is None else quotas_out
    offsets_changed = torch.empty((2 * segments + 1,), dtype=torch.int64, device=device)
    offsets, changed = offsets_changed[:segments + 1], offsets_changed[segments + 1:]
    if not queue:
        _lib.call("lr_select_refine_sets", raw.data_ptr(), pooled.data_ptr(), total,
                  ends_device.data_ptr(), starts_device.data_ptr(), segments, count,
                  buffer.data_ptr(), buffer.numel(), quotas.data_ptr(), offsets.data_ptr(),
                  removed.data_ptr(), changed.data_ptr(), None, None, _lib.stream_of(raw))
        return DeviceSelection(None, None, None, quotas, offsets, removed, changed, coordinates)
    if queue_stream is None:
        _lib.call("lr_select_refine", raw.data_ptr(), pooled.data_ptr(), total,
                  ends_device.data_ptr(), starts_device.data_ptr(), segments, count,
                  buffer.data_ptr(), buffer.numel(), values.data_ptr(), seg_ids.data_ptr(),
                  positions.data_ptr(), quotas.data_ptr(), offsets.data_ptr(), removed.data_ptr(),
                  changed.data_ptr(), _lib.stream_of(raw))
        return DeviceSelection(values, seg_ids, positions, quotas, offsets, removed, changed,
                               coordinates)
    current = torch.cuda.current_stream(device)
    _lib.call("lr_select_refine_sets", raw.data_ptr(), pooled.data_ptr(), total,
              ends_device.data_ptr(), starts_device.data_ptr(), segments, count,
              buffer.data_ptr(), buffer.numel(), quotas.data_ptr(), offsets.data_ptr(),
              removed.data_ptr(), changed.data_ptr(), None, None, current.cuda_stream)
    sets_done = torch.cuda.Event()
    sets_done.record(current)
    queue_stream.wait_event(sets_done)
    _lib.call("lr_select_refine_queue", starts_device.data_ptr(), total, segments, count,
              buffer.data_ptr(), buffer.numel(), quotas.data_ptr(), offsets.data_ptr(),
              values.data_ptr(), seg_ids.data_ptr(), positions.data_ptr(),
              queue_stream.cuda_stream)
    queue_ready = torch.cuda.Event()
    queue_ready.record(queue_stream)
    # memory the side stream uses stays reserved until that stream's work is done
    for tensor in (buffer, values, out, offsets_changed, quotas, starts_device):
        tensor.record_stream(queue_stream)
    workspace.pending = queue_ready
    return DeviceSelection(values, seg_ids, positions, quotas, offsets, removed, changed,
                           coordinates, queue_ready)


def refine_arrays(allocation, refinement, count):
    """selection.py:52-88 signature: (ArrayReferences, changed, changed_heads)."""
    if (allocation.segments != refinement.segments
            or allocation.cumulative_ends != refinement.cumulative_ends):
        raise ValueError("Allocation and refinement layouts differ")
    coordinates = [(segment.layer, segment.head) for segment in allocation.segments]
    if len(set(coordinates)) != len(coordinates):
        raise ValueError("Each physical head must have exactly one score segment")
    ends = np.asarray(allocation.cumulative_ends, dtype=np.int64)
    starts = np.concatenate(([0], ends[:-1]))
    if ends[-1] != allocation.scores.numel() or any(
            end - start != segment.count for start, end, segment in zip(starts, ends, allocation.segments)):
        raise ValueError("Invalid segment bounds")
    result = select_refine(allocation.scores.contiguous(), refinement.scores.contiguous(),
                           allocation.cumulative_ends,
                           [segment.position_start for segment in allocation.segments],
                           coordinates, count)
    if result is None:
        return ArrayReferences([], [], [], coordinates), 0, 0
    changed, changed_heads = result.change_counts()
    return result.references(), changed, changed_heads
