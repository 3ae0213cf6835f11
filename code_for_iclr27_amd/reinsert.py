"""Reinsertion of recalled KV rows into every layer at once: LazyRecallCache.insert_payload
(src/lazy_recall/cache.py:201-253) for all layers, with merge_plan (recall/planning.py:34-52)
and _C.merge (csrc/recall.cu:7-28) done on the device.

The reference, per layer: copies the layer's positions to the host, runs merge_plan (a stable
argsort per head), uploads the mapping and the recalled positions, and gathers both sources
with one merge launch; the payload was copied into HBM beforehand. Here:
  * the host (the C++ host module, one pass) checks the identities and counts the recalled
    rows of each (layer, head) from the metadata it already holds, which fixes the new layout;
    nothing is read back from the device;
  * one pinned block (the slot table and the recalled positions grouped by head) and then the
    payload are copied in on a side stream of default priority;
  * on the caller's stream, as soon as the metadata has landed: a plan (group and sort each
    head's recalled rows, find their rows in the merged head, flag duplicate identities), then
    the resident rows of every layer move to their new rows (a resident row's new row is its
    old one plus the recalled positions below it, so this needs only the plan, not the
    payload) while the payload is still in flight; then, once the payload has landed, the
    recalled rows go into the gaps.
The merged heads are ordered by position exactly as merge_plan orders them; the resident
positions of each head must ascend, which the cache maintains (append, compaction and merge
all keep it).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .audit import DeviceLayout, PackedLayers
from .scoring import LayerState, _planner

_FLAG_DUPLICATE, _FLAG_IDENTITY, _FLAG_HEAD_LIMIT = 1, 4, 8


@dataclass
class ReinsertOutcome:
    layers: PackedLayers          # merged layers: views into one packed K, V and positions buffer
    head_lens: List[List[int]]
    recalled_rows: torch.Tensor   # i64 [M] (device): row of each recalled entry in its merged head
    inserted: int
    # Recorded on the side stream after the copy of a caller-owned pinned host payload: the
    # payload buffer is read until it completes, so the caller must not refill or free it
    # before (payload_copied.synchronize(), or a stream wait on it). None when nothing of the
    # caller's is read after run() returns (a device payload, or an unpinned one, which run()
    # stages through pinned memory of its own).
    payload_copied: Optional[torch.cuda.Event] = None

    @property
    def layout(self) -> DeviceLayout:
        """The merged layers' metadata on the device (head_lens, cu_seqlens_k, max_seqlen_k)."""
        return self.layers.layout


class Reinserter:
    """Reusable reinsertion runner: keeps a side stream and a host-coherent flag word per
    device."""

    def __init__(self):
        self.streams = {}
        self.flags = {}
        self.counts = {}

    def _side_stream(self, device) -> torch.cuda.Stream:
        stream = self.streams.get(device)
        if stream is None:
            stream = self.streams[device] = torch.cuda.Stream(device)
        return stream

    def _host_flag(self, device) -> int:
        address = self.flags.get(device)
        if address is None:
            pointer = ctypes.c_void_p()
            _lib.call("lr_staging_alloc", 8, ctypes.byref(pointer))
            address = self.flags[device] = pointer.value
        return address

    def _host_counts(self, device, slots) -> int:
        """Host-coherent words for the recalled rows of every slot (device-grouped path)."""
        address, size = self.counts.get(device, (None, 0))
        if size < slots:
            if address is not None:
                _lib.call("lr_staging_free", address)
            pointer = ctypes.c_void_p()
            _lib.call("lr_staging_alloc", 8 * slots, ctypes.byref(pointer))
            address, size = pointer.value, slots
            self.counts[device] = (address, size)
        return address

    def __del__(self):
        # at interpreter exit the module globals may already be gone; the process releases
        # its pinned memory then anyway
        library = getattr(_lib, "_library", None) if _lib is not None else None
        if library is None:
            return
        for address in getattr(self, "flags", {}).values():
            library.lr_staging_free(address)
        for address, _ in getattr(self, "counts", {}).values():
            library.lr_staging_free(address)

    def run(self, layers: Sequence[LayerState], payload: torch.Tensor, metadata) -> ReinsertOutcome:
        """Inserts payload rows [M, 2, d] (K at [i, 0], V at [i, 1]; pinned host memory or
        device memory) with identities metadata [M, 3] = (layer, head, position) into
        ``layers`` (a list of LayerState or a PackedLayers). Returns the merged layers; raises
        before returning, as the reference does, if an identity is already resident or
        repeated. The merges are enqueued on the current stream. A pinned host payload is still
        being read when run() returns: ``outcome.payload_copied`` marks the end of its copy.

        ``metadata`` on the host (a numpy array or an unpinned tensor) is checked and grouped
        by head in C++ before the launches. An int64 tensor in device memory, or in pinned host
        memory (copied in on the side stream ahead of the payload), is grouped on the device
        instead (lr_reinsert_group): the host never walks the identities, and reads each
        head's count back after the plan, with the flags."""
        if isinstance(metadata, torch.Tensor) and (metadata.is_cuda or metadata.is_pinned()):
            return self._run_device_grouped(layers, payload, metadata)
        metadata = np.ascontiguousarray(np.asarray(metadata, dtype=np.int64).reshape(-1, 3))
        count = len(metadata)
        if tuple(payload.shape[:2]) != (count, 2):
            raise ValueError("Recall payload/identity shape mismatch")
        packed = isinstance(layers, PackedLayers)
        if packed:
            tensors = ([layers.keys], [layers.values], [layers.positions])
            lengths, packed_offsets = layers.kept, layers.offsets
        else:
            tensors = ([l.keys for l in layers], [l.values for l in layers],
                       [l.positions for l in layers])
            lengths, packed_offsets = [list(l.head_lens) for l in layers], []
        try:
            block, new_lens, offsets, out_rows, max_length = _planner().reinsert_prepare(
                *tensors, lengths, packed_offsets, torch.from_numpy(metadata))
        except RuntimeError as error:
            if "Invalid recall identity" in str(error) or "Too many recalled rows" in str(error):
                raise ValueError(str(error)) from None
            raise
        keys0 = tensors[0][0]
        dim, dtype, device = keys0.shape[1], keys0.dtype, keys0.device
        if payload.dtype != dtype or tuple(payload.shape[2:]) != (dim,):
            raise RuntimeError("Recalled payload must match the cache dtype and head dim")
        slots = len(lengths) * len(lengths[0])

        current = torch.cuda.current_stream(device)
        side = self._side_stream(device)
        stream = current.cuda_stream
        out_keys = torch.empty((out_rows, dim), dtype=dtype, device=device)
        out_values = torch.empty_like(out_keys)
        out_positions = torch.empty((out_rows,), dtype=torch.float32, device=device)
        recalled_rows = torch.empty((count,), dtype=torch.int64, device=device)
        workspace = torch.empty((3 * max(count, 1),), dtype=torch.int64, device=device)
        flag = torch.zeros((1,), dtype=torch.int64, device=device)

        # copies in, on the side stream (nothing there waits for the caller's earlier work):
        # the table and metadata block (small) first, then a host payload
        on_device = payload.is_cuda
        if on_device:
            payload_device = payload.contiguous()  # the caller's stream, like its producer
        with torch.cuda.stream(side):
            block_device = block.to(device, non_blocking=True)
            planned_in = torch.cuda.Event()
            planned_in.record(side)
            if not on_device:
                source = payload if payload.is_pinned() else payload.pin_memory()
                payload_device = source.to(device, non_blocking=True)
                payload_ready = torch.cuda.Event()
                payload_ready.record(side)
        # memory allocated for the side stream's copies stays reserved until the current
        # stream's reads of it are done
        block_device.record_stream(current)
        if not on_device:
            payload_device.record_stream(current)

        current.wait_event(planned_in)
        host_flag = self._host_flag(device)
        table = block_device.data_ptr()
        heads = len(lengths[0])
        layout = torch.empty((slots + len(lengths) * (heads + 1),), dtype=torch.int32,
                             device=device)
        _lib.call("lr_reinsert_plan_layout", table, slots,
                  table + 8 * slots * _lib.LR_REINSERT_WORDS if count else None, count,
                  workspace.data_ptr(), _lib.ptr(recalled_rows), flag.data_ptr(), heads,
                  layout.data_ptr(), layout.data_ptr() + 4 * slots, stream)
        _lib.call("lr_copy_words", flag.data_ptr(), host_flag, 1, stream)
        planned = torch.cuda.Event()
        planned.record(current)
        _lib.call("lr_reinsert_resident", table, slots, workspace.data_ptr(), count, max_length,
                  dim, keys0.element_size(), out_rows, out_keys.data_ptr(),
                  out_values.data_ptr(), out_positions.data_ptr(), stream)
        if not on_device:
            current.wait_event(payload_ready)
        _lib.call("lr_reinsert_recalled", workspace.data_ptr(), count, _lib.ptr(payload_device),
                  dim, keys0.element_size(), out_rows, out_keys.data_ptr(),
                  out_values.data_ptr(), out_positions.data_ptr(), stream)
        planned.synchronize()  # the plan only; the merges may still run
        word = ctypes.c_int64.from_address(host_flag).value
        if word & _FLAG_DUPLICATE:
            raise ValueError("Cannot merge duplicate physical KV identities")
        if word & _FLAG_HEAD_LIMIT:
            raise ValueError("Too many recalled rows for one head")
        merged = PackedLayers(out_keys, out_values, out_positions, new_lens, offsets,
                              layers.sources if packed else list(layers),
                              DeviceLayout(layout, new_lens))
        caller_buffer = not on_device and source is payload
        return ReinsertOutcome(merged, new_lens, recalled_rows, count,
                               payload_ready if caller_buffer else None)


    def _run_device_grouped(self, layers, payload, metadata) -> ReinsertOutcome:
        """run() for identities in device (or pinned host) memory: the table goes up through
        the host module's staging ring, the grouping (count, prefix, scatter), the plan, the
        resident rows and the recalled rows run on the current stream, and the host builds its
        layout from the counts once the plan is done."""
        if metadata.dtype != torch.int64 or metadata.dim() != 2 or metadata.shape[1] != 3:
            raise ValueError("Recall metadata must be an int64 [count, 3] array")
        count = int(metadata.shape[0])
        if tuple(payload.shape[:2]) != (count, 2):
            raise ValueError("Recall payload/identity shape mismatch")
        packed = isinstance(layers, PackedLayers)
        if packed:
            tensors = ([layers.keys], [layers.values], [layers.positions])
            lengths, packed_offsets = layers.kept, layers.offsets
        else:
            tensors = ([l.keys for l in layers], [l.values for l in layers],
                       [l.positions for l in layers])
            lengths, packed_offsets = [list(l.head_lens) for l in layers], []
        keys0 = tensors[0][0]
        dim, dtype, device = keys0.shape[1], keys0.dtype, keys0.device
        if payload.dtype != dtype or tuple(payload.shape[2:]) != (dim,):
            raise RuntimeError("Recalled payload must match the cache dtype and head dim")
        heads = len(lengths[0])
        slots = len(lengths) * heads
        current = torch.cuda.current_stream(device)

        # copies in, on the side stream: host metadata first (small), then a host payload
        side = self._side_stream(device)
        on_device = payload.is_cuda
        if on_device:
            payload_device = payload.contiguous()
        meta_device = metadata.contiguous() if metadata.is_cuda else None
        meta_ready = payload_ready = None
        source = None
        if meta_device is None or not on_device:
            with torch.cuda.stream(side):
                if meta_device is None:
                    meta_device = metadata.to(device, non_blocking=True)
                    meta_ready = torch.cuda.Event()
                    meta_ready.record(side)
                if not on_device:
                    source = payload if payload.is_pinned() else payload.pin_memory()
                    payload_device = source.to(device, non_blocking=True)
                    payload_ready = torch.cuda.Event()
                    payload_ready.record(side)
            if meta_ready is not None:
                meta_device.record_stream(current)
            if payload_ready is not None:
                payload_device.record_stream(current)

        # the table upload, the waits for the copies, the grouping, the plan and both merges are
        # enqueued by the host module (csrc/host_plan.cpp reinsert_device_launch), which waits
        # for the plan only
        (out_keys, out_values, out_positions, layout, recalled_rows, new_lens, offsets,
         word) = _reinsert_module().reinsert_device(
            *tensors, lengths, packed_offsets, payload_device, meta_device,
            meta_ready.cuda_event if meta_ready is not None else 0,
            payload_ready.cuda_event if payload_ready is not None else 0,
            self._host_flag(device), self._host_counts(device, slots), current.cuda_stream)
        if word & _FLAG_IDENTITY:
            raise ValueError("Invalid recall identity")
        if word & _FLAG_DUPLICATE:
            raise ValueError("Cannot merge duplicate physical KV identities")
        if word & _FLAG_HEAD_LIMIT:
            raise ValueError("Too many recalled rows for one head")
        merged = PackedLayers(out_keys, out_values, out_positions, new_lens, offsets,
                              layers.sources if packed else list(layers),
                              DeviceLayout(layout, new_lens))
        caller_buffer = source is not None and source is payload
        return ReinsertOutcome(merged, new_lens, recalled_rows, count,
                               payload_ready if caller_buffer else None)


_module = None


def _reinsert_module():
    """The C++ host module with the reinsertion entry points bound (once)."""
    global _module
    if _module is None:
        from .audit import _native_planner
        planner = _native_planner()
        library = _lib.load()
        address = lambda name: ctypes.cast(getattr(library, name), ctypes.c_void_p).value
        planner.bind_reinsert(address("lr_reinsert_group"), address("lr_reinsert_plan_layout"),
                              address("lr_reinsert_resident"), address("lr_reinsert_recalled"))
        _module = planner
    return _module


_default = Reinserter()


def reinsert(layers, payload, metadata) -> ReinsertOutcome:
    """Module-level convenience over one shared Reinserter."""
    return _default.run(layers, payload, metadata)
