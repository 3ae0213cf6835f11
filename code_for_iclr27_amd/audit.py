"""One LazyRecall audit step on the GPU: score -> Pool7 -> select -> compact.

Mirrors LazyController.run_audit (src/lazy_recall/controller.py:140-159) for the KV work it
drives: compute_score_table (scoring.py:198-308), pool_score_table (scoring.py:322-353),
allocation_preserving_references / refine_arrays (scoring.py:356-361, selection.py:52-88) and
the immediate removal LazyRecallCache.remove_positions (cache.py:92-180) of every layer.

The reference runs these as a Python loop of ~4 launches per (layer, head), per-segment
torch.topk calls with device->host copies, host list -> tensor copies per layer and one
compaction launch per layer. Here the host builds one int64 metadata block (segment table,
pool bounds, segment ends, head table), uploads it once (a host-coherent staging buffer read by
a copy kernel on the step's stream), and enqueues:
3 scoring kernels, 1 pool kernel, the selection kernels and 1 compaction kernel covering all
layers. The only synchronisation is a wait for the per-segment quotas, which the host needs to
describe the new ragged layout (as the reference's metadata rebuild does): the selection stores
them into host-coherent memory, with an event right after the selection, before the compaction
is enqueued, so the host builds the layout (and enqueues the caller's next work) while the
compaction runs. The
eviction-queue order (a per-segment sort and a merge of all segments' picks) is only needed
for a non-empty lazy queue; on request it runs on a side stream while the compaction, which
needs only the removal sets, runs on the current stream.
"""

from __future__ import annotations

import math
import time
from collections import abc
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _C, _lib
from .scoring import LayerState, ScoreSegment, ScoreTable, SegmentPlan, _planner, plan_segments
from .selection import ArrayReferences, DeviceSelection, SelectWorkspace, select_refine

_bound = False


def _native_planner():
    """The C++ host module, with the library entry points it launches bound once."""
    global _bound
    planner = _planner()
    if not _bound:
        import ctypes

        library = _lib.load()
        address = lambda name: ctypes.cast(getattr(library, name), ctypes.c_void_p).value
        planner.bind_library(address("lr_score_workspace_bytes"), address("lr_score_segments"),
                             address("lr_pool"), address("lr_select_workspace_bytes"),
                             address("lr_pool_select_refine_sets"),
                             address("lr_select_refine_queue"),
                             address("lr_queue_index"), address("lr_queue_evict_plan"),
                             address("lr_compact_heads_layout"), address("lr_last_error"),
                             address("lr_staging_alloc"), address("lr_staging_free"),
                             address("lr_copy_words"))
        _bound = True
    return planner


def pool_score_table(table: ScoreTable, kernel_size: int = 7) -> ScoreTable:
    """scoring.py:322-335 (GPU branch) with this package's ``_C.pool``."""
    if kernel_size <= 0 or kernel_size % 2 == 0:
        raise ValueError("pool kernel must be a positive odd integer")
    started = time.perf_counter()
    bounds = torch.tensor([0] + list(table.cumulative_ends), dtype=torch.int64,
                          device=table.scores.device)
    scores = _C.pool(table.scores.contiguous(), bounds,
                     max(segment.count for segment in table.segments), kernel_size)
    return ScoreTable(scores, list(table.segments), list(table.cumulative_ends),
                      table.score_ms + (time.perf_counter() - started) * 1000.0)


class DeviceLayout:
    """The metadata the reference rebuilds with host-to-device copies after every layout change
    (metadata.head_lens, metadata.cu_seqlens_k and metadata.max_seqlen_k; cache.py:171-178 after
    a compaction, cache.py:246 after a reinsertion), here written on the device by the launch
    that changed the layout. ``block`` is one i32 tensor: the new length of every (layer, head)
    slot, then each layer's cumulative lengths (0, then the running sum).

    ``head_lens[l]`` (i32 [H]) and ``cu_seqlens_k[l]`` (i32 [H + 1]) are device views, ready for
    ``_C.append``'s ``cumulative`` argument; ``max_seqlen_k[l]`` is a host int, from the lengths
    the host already knows. The views are valid in stream order after the launch."""

    def __init__(self, block: torch.Tensor, kept: Sequence[Sequence[int]]):
        layers, heads = len(kept), len(kept[0])
        self.block = block
        self.head_lens = block[:layers * heads].view(layers, heads)
        self.cu_seqlens_k = block[layers * heads:].view(layers, heads + 1)
        self.max_seqlen_k = [max(lengths, default=0) for lengths in kept]

    def layer(self, index: int):
        """(head_lens i32 [H], cu_seqlens_k i32 [H + 1], max_seqlen_k) of one layer."""
        return self.head_lens[index], self.cu_seqlens_k[index], self.max_seqlen_k[index]


class PackedLayers(abc.Sequence):
    """The compacted layers of an audit: every layer's rows live in one packed K, V and
    positions buffer (layer-major, heads in order). Layer i's LayerState, with views into those
    buffers, is created when first indexed. ``layout`` (a DeviceLayout, or None) holds the
    layers' metadata on the device when the launch that made them wrote it."""

    def __init__(self, keys, values, positions, kept: List[List[int]], offsets: List[int],
                 sources: Sequence[LayerState], layout: Optional[DeviceLayout] = None):
        self.keys, self.values, self.positions = keys, values, positions
        self.kept = kept                                   # [L][H] rows kept per head
        self.offsets = offsets                             # [L + 1] first row of each layer
        self.sources = sources
        self.layout = layout
        self._cache = {}

    def __len__(self) -> int:
        return len(self.sources)

    def __getitem__(self, index):
        if isinstance(index, slice):
            return [self[i] for i in range(*index.indices(len(self)))]
        if index < 0:
            index += len(self)
        if not 0 <= index < len(self):
            raise IndexError(index)
        layer = self._cache.get(index)
        if layer is None:
            start, end = self.offsets[index], self.offsets[index + 1]
            source = self.sources[index]
            layer = LayerState(self.keys[start:end], self.values[start:end],
                               self.positions[start:end], list(self.kept[index]),
                               source.prompt_lens, source.queries, source.gradient)
            self._cache[index] = layer
        return layer


def _archive_hook(transport, keys, count):
    """The C++ launcher's archive hook for a RecallTransport (None without one): packs a fused
    layout change's removed rows into a free archive slot, on the current stream, before the
    compaction is enqueued. The batch of ``count`` rows is checked against the staging
    capacity here, before any launch (record_evicted's check, transport.py:139-141)."""
    if transport is None:
        return None
    if keys.dim() != 2 or keys.shape[1] != transport.dimension or keys.element_size() != 2:
        raise RuntimeError("Recall configuration does not match the cache")
    if count > transport.capacity:
        transport.counters["archive_overflows"] += 1
        raise RuntimeError("Eviction batch exceeds configured archive staging capacity")

    def hook(head_table, slots, heads_per_layer, quotas, offsets, positions, count, max_rows):
        transport.record_evicted_heads(head_table, slots, heads_per_layer, quotas, offsets,
                                       positions, count, max_rows)
    return hook


def _removed_now(layers, count, immediate):
    """Rows an audit step removes at once (an upper bound when fewer candidates exist)."""
    if count <= 0:
        return 0
    return count if immediate < 0 or immediate >= count else immediate


class EvictionQueue:
    """The deletion queue an audit leaves behind, kept on the device: controller.py:148-158
    removes the first ``immediate`` selected slots and keeps ``references[immediate:]`` as
    ``self.queue``; evict_prefix (controller.py:57-70) later removes its next batches, each
    position shifted down by the earlier removals of its head below it.

    ``len(queue)`` counts the slots still queued, ``references()`` copies them to the host as
    the reference's ``ArrayReferences``, and ``evict_prefix(layers, count)`` removes the next
    ``count`` of them from ``layers`` as they are now (the audit's compacted layers, with any
    tokens appended since): one plan launch and one compaction of every layer
    (lr_queue_evict_plan, lr_compact_heads), then a wait for the plan only. The queue is tied to
    the cache it was selected from; after a recall splice the reference starts a new one
    (controller.py:113-114)."""

    def __init__(self, values, order, rank, quotas, offsets, removed, coordinates, slot_segment,
                 consumed, sync):
        """Enqueues, on the current stream, a copy of the queue's segment ids to pinned host
        memory: each batch's per-segment counts (and so the new layout) are then counted on
        the host, and evict_prefix never waits for the device."""
        self.count = int(values.numel())
        self.values = values                     # f32 [count], queue order
        self.segments = order[:self.count]       # i64 [count]
        self.positions = order[self.count:]      # i64 [count], audit-time positions
        self.rank = rank                         # i32: queue slot of each position-sorted pick
        self.quotas, self.offsets, self.removed = quotas, offsets, removed
        self.coordinates = coordinates           # (layer, head) of every segment
        self.slot_segment = slot_segment         # segment (or -1) of every (layer, head) slot
        self.consumed = int(consumed)            # queue slots already removed (a prefix)
        self._sync = sync
        self._segments_host = torch.empty((self.count,), dtype=torch.int64, pin_memory=True)
        self._segments_host.copy_(self.segments, non_blocking=True)
        self._host_ready = torch.cuda.Event()
        self._host_ready.record()

    def __len__(self) -> int:
        return self.count - self.consumed

    def references(self) -> ArrayReferences:
        """The slots still queued, in queue order (controller.queue)."""
        start = self.consumed
        return ArrayReferences(self.values[start:].cpu().numpy(),
                               self.segments[start:].cpu().numpy(),
                               self.positions[start:].cpu().numpy(), self.coordinates)

    def evict_prefix(self, layers: Sequence[LayerState], count: int, transport=None):
        """controller.py:57-70 for the device queue: removes the next ``count`` queued slots
        and returns the new layers (a PackedLayers; ``.kept`` holds the head lengths, ``.layout``
        the device metadata). With a ``transport`` (a RecallTransport) the removed rows are
        packed for its archive before the compaction, as remove_positions archives them
        (cache.py:110-112)."""
        count = int(count)
        if not count:
            return layers
        if count < 0 or count > len(self):
            raise RuntimeError("Discard queue underflow")
        planner = _native_planner()
        device = (layers.keys if isinstance(layers, PackedLayers) else layers[0].keys).device
        if self._host_ready is not None:  # the audit's copy of the segment ids, once
            self._host_ready.synchronize()
            self._host_ready = None
        if isinstance(layers, PackedLayers):  # the packed buffers, without per-layer views
            tensors = ([layers.keys], [layers.values], [layers.positions])
            lengths, packed_offsets = layers.kept, layers.offsets
        else:
            tensors = ([layer.keys for layer in layers], [layer.values for layer in layers],
                       [layer.positions for layer in layers])
            lengths, packed_offsets = [list(layer.head_lens) for layer in layers], []
        out_keys, out_values, out_positions, kept, offsets, layout = planner.queue_evict_launch(
            *tensors, lengths, self.slot_segment, self.quotas, self.offsets, self.removed,
            self.rank, self._segments_host, self.consumed, self.consumed + count,
            torch.cuda.current_stream(device).cuda_stream, self._sync, packed_offsets,
            _archive_hook(transport, tensors[0][0], count))
        self.consumed += count
        return PackedLayers(out_keys, out_values, out_positions, kept, offsets, layers,
                            DeviceLayout(layout, kept))


@dataclass
class AuditOutcome:
    layers: Sequence[LayerState]      # compacted layers (a PackedLayers: views into one packed
                                      # K/V/pos buffer), or the input layers if none was removed
    head_lens: List[List[int]]
    scores: torch.Tensor              # raw temporal scores [S]
    pooled: torch.Tensor              # Pool7 scores [S]
    selection: Optional[DeviceSelection]
    plan: SegmentPlan
    removed: int
    queue: Optional[EvictionQueue] = None  # the lazy queue (run(..., immediate=k), k < count)

    @property
    def layout(self) -> Optional[DeviceLayout]:
        """The compacted layers' metadata on the device (None when no compaction ran: the
        caller's metadata then still holds)."""
        return getattr(self.layers, "layout", None)

    @property
    def segments(self) -> List[ScoreSegment]:
        return self.plan.segments

    @property
    def cumulative_ends(self) -> List[int]:
        return self.plan.cumulative_ends


class _Workspace:
    def __init__(self):
        self.buffers = {}

    def get(self, name: str, nbytes: int, device) -> torch.Tensor:
        buffer = self.buffers.get(name)
        if buffer is None or buffer.numel() < nbytes or buffer.device != device:
            buffer = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=device)
            self.buffers[name] = buffer
        return buffer


class AuditStep:
    """Reusable audit-step runner (keeps its scratch buffers between calls)."""

    def __init__(self):
        self.workspace = _Workspace()
        self.select_workspace = SelectWorkspace()
        self.queue_streams = {}
        self.syncs = {}

    def _queue_stream(self, device) -> torch.cuda.Stream:
        """Side stream (default priority) for the eviction-queue order; the compaction, which
        needs only the removal sets, runs meanwhile on the current stream."""
        stream = self.queue_streams.get(device)
        if stream is None:
            stream = torch.cuda.Stream(device)
            self.queue_streams[device] = stream
        return stream

    def run(self, layers: Sequence[LayerState], query_positions: torch.Tensor,
            margin: torch.Tensor, count: int, protect_recent: int = 32, pool_kernel: int = 7,
            denominator_epsilon: float = 1e-6, check_finite: bool = True,
            queue_order: bool = False, timer=None, native: bool = True,
            immediate: Optional[int] = None, transport=None) -> AuditOutcome:
        """Scores and selects ``count`` slots (controller.run_audit, controller.py:140-159).

        ``immediate`` None (or >= count) removes every selected slot now; the lazy queue
        ``references[immediate:]`` is then empty and the removal sets are all the step needs,
        so the queue order (``outcome.selection.values/segments/positions``) is computed only
        with ``queue_order=True``, on the step's stream between the selection and the
        compaction (``native=False``: on a side stream beside the compaction).
        ``0 <= immediate < count`` is the lazy form: the queue order is computed, its first
        ``immediate`` slots are removed (with 0 the layers are returned as they are) and the rest
        stay queued on the device as ``outcome.queue`` (an EvictionQueue) for evict_prefix.
        ``timer`` (optional) gets ``timer.mark(name)`` calls between the launches of each
        stage, on the current stream, for per-stage event timing. The launches are made by the
        C++ host module; ``native=False`` makes the same launches from Python (a cross-check).
        ``transport`` (a RecallTransport, native launches only): the rows the step removes are
        packed for its archive before the compaction, as remove_positions archives them
        (cache.py:110-112); the queued slots follow with each evict_prefix batch given it.
        """
        if pool_kernel <= 0 or pool_kernel % 2 == 0:
            raise ValueError("pool kernel must be a positive odd integer")
        immediate = -1 if immediate is None else int(immediate)
        if immediate < -1:
            raise ValueError("immediate must be non-negative")
        if not native:
            if transport is not None:
                raise ValueError("archiving an audit's removals needs the native launcher")
            return self._run_python(layers, query_positions, margin, count, protect_recent,
                                    pool_kernel, denominator_epsilon, check_finite, queue_order,
                                    timer, immediate)
        return self._run_native(layers, query_positions, margin, count, protect_recent,
                                pool_kernel, denominator_epsilon, check_finite, timer,
                                queue_order, immediate, transport)

    def _run_python(self, layers, query_positions, margin, count, protect_recent, pool_kernel,
                    denominator_epsilon, check_finite, queue_order, timer, immediate=-1):
        """The same step launched from Python (plan_segments, ctypes calls)."""
        mark = timer.mark if timer is not None else (lambda name: None)
        plan = plan_segments(layers, protect_prompt=True, protect_recent=protect_recent,
                             pinned=True)
        device = layers[0].keys.device
        stream = torch.cuda.current_stream(device).cuda_stream
        segments = plan.segment_count
        heads = plan.head_slots
        dim = plan.dim
        elem = 2

        # --- one int64 metadata block (pinned), uploaded once ------------------------------
        device_block = plan.block.to(device, non_blocking=True)
        base = device_block.data_ptr()
        table_ptr = base + 8 * plan.parts["table"][0]
        bounds_ptr = base + 8 * plan.parts["bounds"][0]
        heads_ptr = base + 8 * plan.parts["heads"][0]
        ends_d = plan.part("ends", device_block)
        starts_d = plan.part("starts", device_block)
        max_length = plan.max_head_length
        # quotas and the non-finite score count come back in one small copy at the end
        info = torch.zeros((segments + 1,), dtype=torch.int64, device=device)
        nonfinite = info[segments:].view(torch.int32)[:1]

        # --- scores ------------------------------------------------------------------------
        total = plan.total
        score_bytes = _lib.load().lr_score_workspace_bytes(
            segments, plan.groups, plan.window, segments * plan.groups * plan.max_length)
        score_ws = self.workspace.get("score", score_bytes, device)
        scores = torch.empty((2 * total,), dtype=torch.float32, device=device)
        raw, pooled = scores[:total], scores[total:]
        margin = margin.to(device=device, dtype=torch.float32).reshape(1)
        stage_names = ("projected_values", "row_stats", "column_scores")
        stage_masks = (1, 2, 4) if timer is not None else (7,)
        mark("start")
        for index, stages in enumerate(stage_masks):
            _lib.call("lr_score_segments", table_ptr, segments, plan.groups,
                      plan.window, dim, plan.max_length, plan.max_candidates, plan.query_stride,
                      query_positions.data_ptr(), margin.data_ptr(), float(1.0 / math.sqrt(dim)),
                      float(denominator_epsilon), score_ws.data_ptr(), score_bytes,
                      raw.data_ptr(), nonfinite.data_ptr(), stages, stream)
            mark(stage_names[index] if timer is not None else "score")

        # --- Pool7 -------------------------------------------------------------------------
        _lib.call("lr_pool", raw.data_ptr(), total, bounds_ptr, segments,
                  plan.max_candidates, pool_kernel, pooled.data_ptr(), stream)
        mark("pool")

        # --- selection ---------------------------------------------------------------------
        count = min(max(0, int(count)), total)
        if immediate > count:
            raise RuntimeError("Not enough unprotected candidates to enforce the budget")
        lazy = count > 0 and 0 <= immediate < count
        selection = select_refine(raw, pooled, None, None, plan.segment_info[:2].T, count,
                                  ends_device=ends_d, starts_device=starts_d,
                                  workspace=self.select_workspace, quotas_out=info[:segments],
                                  queue=queue_order or lazy,
                                  queue_stream=self._queue_stream(device) if queue_order and not lazy else None)
        if lazy:
            return self._finish_lazy(plan, info, raw, pooled, selection, count, immediate, layers,
                                     heads_ptr, max_length, check_finite, stream, mark)
        mark("select")

        # --- compaction of every layer -----------------------------------------------------
        out_rows = plan.rows_total - count
        out_keys = torch.empty((out_rows, dim), dtype=layers[0].keys.dtype, device=device)
        out_values = torch.empty_like(out_keys)
        out_positions = torch.empty((out_rows,), dtype=torch.float32, device=device)
        if selection is not None:
            _lib.call("lr_compact_heads", heads_ptr, heads, selection.quotas.data_ptr(),
                      selection.offsets.data_ptr(), selection.removed_positions.data_ptr(), dim,
                      elem, max_length, out_rows, out_keys.data_ptr(), out_values.data_ptr(),
                      out_positions.data_ptr(), stream)
            mark("compact")
        else:
            out_keys.copy_(torch.cat([layer.keys for layer in layers]))
            out_values.copy_(torch.cat([layer.values for layer in layers]))
            out_positions.copy_(torch.cat([layer.positions.reshape(-1) for layer in layers]))
        if selection is not None and selection.queue_ready is not None:
            selection.wait_queue()  # join the queue order back before the step ends
            mark("queue_join")
        return self._finish(plan, info, raw, pooled, selection, count, out_keys, out_values,
                            out_positions, layers, check_finite)

    def _finish_lazy(self, plan, info, raw, pooled, selection, count, immediate, layers,
                     heads_ptr, max_length, check_finite, stream, mark):
        """The Python path's lazy form: the queue index and the plan of the queue's first
        ``immediate`` slots, their compaction, then one copy of the batch quotas."""
        device = raw.device
        segments = plan.segment_count
        rank = torch.empty((count,), dtype=torch.int32, device=device)
        _lib.call("lr_queue_index", selection.segments.data_ptr(), selection.positions.data_ptr(),
                  count, selection.quotas.data_ptr(), selection.offsets.data_ptr(),
                  selection.removed_positions.data_ptr(), segments, rank.data_ptr(), stream)
        batch = torch.zeros((count + segments,), dtype=torch.int64, device=device)
        if immediate:
            _lib.call("lr_queue_evict_plan", selection.quotas.data_ptr(),
                      selection.offsets.data_ptr(), selection.removed_positions.data_ptr(),
                      rank.data_ptr(), segments, 0, immediate, batch[count:].data_ptr(),
                      batch.data_ptr(), None, stream)
        mark("select")
        out_rows = plan.rows_total - immediate
        out_keys = out_values = out_positions = None
        if immediate:
            out_keys = torch.empty((out_rows, plan.dim), dtype=layers[0].keys.dtype, device=device)
            out_values = torch.empty_like(out_keys)
            out_positions = torch.empty((out_rows,), dtype=torch.float32, device=device)
            _lib.call("lr_compact_heads", heads_ptr, plan.head_slots, batch[count:].data_ptr(),
                      selection.offsets.data_ptr(), batch.data_ptr(), plan.dim, 2, max_length,
                      out_rows, out_keys.data_ptr(), out_values.data_ptr(),
                      out_positions.data_ptr(), stream)
            mark("compact")
        host_info = info.cpu().numpy()
        if check_finite and int(host_info[segments:].view(np.int32)[0]):
            raise RuntimeError("LazyRecall produced non-finite scores; refusing to construct a deletion queue")
        quotas = batch[count:].cpu().numpy()
        segment_index, lengths = plan.head_info
        removed_per_slot = np.where(segment_index >= 0, quotas[np.maximum(segment_index, 0)], 0)
        kept = (lengths - removed_per_slot).reshape(-1, plan.heads)
        new_lens = kept.tolist()
        if immediate:
            offsets = np.concatenate(([0], np.cumsum(kept.sum(axis=1)))).tolist()
            new_layers = PackedLayers(out_keys, out_values, out_positions, new_lens, offsets, layers)
        else:
            new_layers = list(layers)
        order = torch.cat((selection.segments, selection.positions))
        queue = EvictionQueue(selection.values, order, rank, selection.quotas, selection.offsets,
                              selection.removed_positions, plan.segment_info[:2].T,
                              [int(v) for v in segment_index], immediate, self._sync_for(device))
        return AuditOutcome(new_layers, new_lens, raw, pooled, selection, plan, immediate, queue)

    def _sync_for(self, device):
        sync = self.syncs.get(device)
        if sync is None:
            sync = self.syncs[device] = _native_planner().StepSync()
        return sync

    @staticmethod
    def _finish(plan, info, raw, pooled, selection, count, out_keys, out_values, out_positions,
                layers, check_finite):
        """The Python path's end: one copy of the quotas (which waits for the whole step), then
        the new ragged layout (host metadata, views into the packed buffers)."""
        segments = plan.segment_count
        host_info = info.cpu().numpy()  # the step's only synchronisation
        quotas = host_info[:segments]
        bad = int(host_info[segments:].view(np.int32)[0])
        if check_finite and bad:
            raise RuntimeError("LazyRecall produced non-finite scores; refusing to construct a deletion queue")
        segment_index, lengths = plan.head_info
        removed_per_slot = np.where(segment_index >= 0, quotas[np.maximum(segment_index, 0)], 0)
        kept = (lengths - removed_per_slot).reshape(-1, plan.heads)
        offsets = np.concatenate(([0], np.cumsum(kept.sum(axis=1)))).tolist()
        new_lens = kept.tolist()
        new_layers = PackedLayers(out_keys, out_values, out_positions, new_lens, offsets, layers)
        return AuditOutcome(new_layers, new_lens, raw, pooled, selection, plan, count)

    def _run_native(self, layers, query_positions, margin, count, protect_recent, pool_kernel,
                    denominator_epsilon, check_finite, timer=None, queue_order=False,
                    immediate=-1, transport=None):
        """The step with planning and every launch done by the C++ host module
        (csrc/host_plan.cpp audit_launch): no Python between the launches. With
        ``queue_order`` the queue half of the selection follows the removal sets on the same
        stream, before the compaction: on a side stream its small launches waited for the
        compaction's workgroups to free the CUs, which cost more than running them first."""
        if len(layers) == 0:
            raise RuntimeError("No layers to score")
        planner = _native_planner()
        device = layers[0].keys.device
        sync = self._sync_for(device)
        margin = margin.to(device=device, dtype=torch.float32).reshape(1)
        mark = None if timer is None else timer.mark
        (block, meta, segment_info, head_info, scores, info, quotas, offsets, removed, changed,
         out_keys, out_values, out_positions, device_block, select_ws,
         queue_state, layout) = planner.audit_launch(
            [layer.keys for layer in layers], [layer.values for layer in layers],
            [layer.positions for layer in layers], [layer.queries for layer in layers],
            [layer.gradient for layer in layers], [list(layer.head_lens) for layer in layers],
            [None if layer.prompt_lens is None else list(layer.prompt_lens) for layer in layers],
            int(protect_recent), query_positions, margin, int(count), int(immediate),
            int(pool_kernel), float(denominator_epsilon),
            torch.cuda.current_stream(device).cuda_stream, mark, sync,
            _archive_hook(transport, layers[0].keys, _removed_now(layers, count, immediate)),
            bool(queue_order))
        plan = SegmentPlan(block, meta, segment_info, head_info, len(layers[0].head_lens))
        total = plan.total
        count = min(max(0, int(count)), total)
        selection = None
        if queue_state is not None and len(queue_state) == 3:  # the lazy form
            values, order, rank = queue_state
            selection = DeviceSelection(values, order[:count], order[count:], quotas, offsets,
                                        removed, changed, plan.segment_info[:2].T)
            kept, offsets_out = sync.wait(check_finite)
            if immediate:
                new_layers = PackedLayers(out_keys, out_values, out_positions, kept, offsets_out,
                                          layers, DeviceLayout(layout, kept))
            else:
                new_layers = list(layers)
            queue = EvictionQueue(values, order, rank, quotas, offsets, removed,
                                  plan.segment_info[:2].T, [int(v) for v in plan.head_info[0]],
                                  immediate, sync)
            return AuditOutcome(new_layers, [list(lengths) for lengths in kept], scores[:total],
                                scores[total:], selection, plan, immediate, queue)
        if count:
            selection = DeviceSelection(None, None, None, quotas, offsets, removed, changed,
                                        plan.segment_info[:2].T)
            if queue_state is not None:  # the queue order, computed before the compaction
                values, order = queue_state
                selection.values = values
                selection.segments, selection.positions = order[:count], order[count:]
        # waits for the selection only; the compaction may still run (outputs in stream order)
        kept, offsets = sync.wait(check_finite)
        new_layers = PackedLayers(out_keys, out_values, out_positions, kept, offsets, layers,
                                  None if layout is None else DeviceLayout(layout, kept))
        return AuditOutcome(new_layers, [list(lengths) for lengths in kept], scores[:total],
                            scores[total:], selection, plan, count)
