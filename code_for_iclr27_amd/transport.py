"""The recall transport: eviction batches out to the host archive, search results back to HBM
(the drop-in for RecallTransport, src/lazy_recall/recall/transport.py:46-361, and its CPU worker,
recall/cpu_worker.py:136-182).

What a caller sees is the reference's: the constructor arguments, record_evicted / step /
ready_result / release_result / retire_finished / remove_admitted / wait_pending / finish /
close, the per-slot state names ("free", "copying", "worker"; "free", "copying_query",
"worker", "copying_result", "retiring"), the counter keys and the stats.

How it works is this package's own:
  * the native ring (liblazyrecall_recall.so, csrc/recall_ring.cpp) owns the slot states, two
    default-priority copy streams (one per direction) with their events, the exact-MIPS archive
    (csrc/archive.cpp) and one worker thread. The worker takes archive batches, searches and
    removals in submission order, waits for each job's copy event itself, calls the archive and
    enqueues the results' copy into device staging. Nothing here polls or forwards messages: a
    method only reads states, and the worker moves them;
  * an eviction batch is one pinned upload of a (layer, head, row) descriptor list with the
    layers' pointer table and one packing launch for every layer (lr_pack_layers); a search's
    queries are one launch averaging every layer's group queries (lr_group_mean_queries);
  * the buffers are torch's: pinned host staging (``host``), device staging, allocated once.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np
import torch

from . import _lib

LIBRARY_PATH = Path(__file__).resolve().parent / "liblazyrecall_recall.so"

_P, _I64, _I, _D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
_IP = ctypes.POINTER(ctypes.c_int)
SIGNATURES = {
    "lrr_last_error": ([], ctypes.c_char_p),
    "lrr_create": ([_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I] + [_P] * 10, _P),
    "lrr_destroy": ([_P], None),
    "lrr_acquire_archive": ([_P, _D, _IP, _IP], _I),
    "lrr_abandon_archive": ([_P, _I], _I),
    "lrr_commit_archive": ([_P, _I, _I64, _P], _I),
    "lrr_acquire_query": ([_P, _IP], _I),
    "lrr_abandon_query": ([_P, _I], _I),
    "lrr_commit_query": ([_P, _I, _I64, _P], _I),
    "lrr_result_ready": ([_P, _I], _I),
    "lrr_release_result": ([_P, _I, _P], _I),
    "lrr_drop_result": ([_P, _I], _I),
    "lrr_retire": ([_P], _I),
    "lrr_remove": ([_P, _P, _I64], _I),
    "lrr_wait_pending": ([_P, _D], _I),
    "lrr_flush": ([_P, _D], _I),
    "lrr_archive_state": ([_P, _I], _I),
    "lrr_query_state": ([_P, _I], _I),
    "lrr_query_step": ([_P, _I], _I64),
    "lrr_result_count": ([_P, _I], _I64),
    "lrr_counters": ([_P, _P], _I),
    "lrr_worker_alive": ([_P], _I),
    "lrr_check": ([_P], _I),
}
ARCHIVE_STATES = ("free", "filling", "copying", "worker")
QUERY_STATES = ("free", "filling", "copying_query", "worker", "copying_result", "retiring")
RESULT_STATE = 4
# the counter keys the ring's worker keeps, in lrr_counters order
WORKER_COUNTERS = ("indexed_vectors", "capacity_drops", "searches_completed", "retrieved_vectors",
                   "h2d_bytes", "cpu_peak_rss_kib")
_TIMEOUT = 3
_library = None


def load() -> ctypes.CDLL:
    """liblazyrecall_recall.so, opened once after torch (one HIP runtime per process)."""
    global _library
    if _library is None:
        if not LIBRARY_PATH.exists():
            raise _lib.LazyRecallLibraryError(
                f"{LIBRARY_PATH.name} is not built; run `python -m code_for_iclr27_amd.build`")
        library = ctypes.CDLL(os.fspath(LIBRARY_PATH))
        for name, (argtypes, restype) in SIGNATURES.items():
            function = getattr(library, name)
            function.argtypes, function.restype = argtypes, restype
        _library = library
    return _library


def _check(status: int) -> None:
    if status == 0:
        return
    message = load().lrr_last_error().decode()
    if status == _TIMEOUT:
        raise TimeoutError(message)
    raise RuntimeError(message)


class _WorkerView:
    """The ring's worker thread as seen from Python (``is_alive``)."""

    name = "LazyRecall-CPU-archive"

    def __init__(self, transport):
        self._transport = transport

    def is_alive(self) -> bool:
        ring = self._transport._ring
        return bool(ring) and bool(load().lrr_worker_alive(ring))


class RecallTransport:
    def __init__(self, layers, heads, query_heads, dimension, search_interval=32, topk=4,
                 archive_buffers=16, cpu_threads=2, evict_interval=8,
                 archive_capacity_per_head=32768, timeout_seconds=60.0):
        if (query_heads % heads or min(layers, heads, dimension, search_interval, topk,
                                        archive_buffers, cpu_threads) <= 0):
            raise ValueError("Invalid recall configuration")
        self.layers, self.heads, self.dimension = int(layers), int(heads), int(dimension)
        self.groups = query_heads // heads
        self.search_interval, self.topk = int(search_interval), int(topk)
        self.capacity = max(evict_interval, topk) * layers * heads
        self.result_capacity = topk * layers * heads
        self.timeout = float(timeout_seconds)
        self.closed = False
        self._ring = None
        self.counters = dict.fromkeys(
            ("archived_vectors", "archive_batches", "indexed_vectors", "submitted_queries",
             "searches_completed", "skipped_busy_queries", "retrieved_vectors", "spliced_vectors",
             "splices", "d2h_bytes", "h2d_bytes", "archive_overflows", "cpu_peak_rss_kib",
             "query_age_tokens_max", "archive_backpressure", "capacity_drops",
             "superseded_results"), 0)
        self.config = dict(layers=layers, heads=heads, dimension=dimension, topk=topk,
                           cpu_threads=cpu_threads,
                           archive_capacity_per_head=archive_capacity_per_head)
        L, H, d, B = self.layers, self.heads, self.dimension, int(archive_buffers)
        shapes = dict(archive_kv=((B, self.capacity, 2, d), torch.int16),
                      archive_meta=((B, self.capacity, 3), torch.int64),
                      queries=((2, L, H, d), torch.float32),
                      result_kv=((2, self.result_capacity, 2, d), torch.int16),
                      result_meta=((2, self.result_capacity, 3), torch.int64))
        self.host = {name: torch.empty(shape, dtype=dtype, pin_memory=True)
                     for name, (shape, dtype) in shapes.items()}
        device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        self.archive_gpu = torch.empty(shapes["archive_kv"][0], dtype=torch.bfloat16, device=device)
        self.archive_meta_gpu = torch.empty(shapes["archive_meta"][0], dtype=torch.int64, device=device)
        self.query_gpu = torch.empty(shapes["queries"][0], dtype=torch.float32, device=device)
        self.result_gpu = torch.empty(shapes["result_kv"][0], dtype=torch.bfloat16, device=device)
        self.result_meta_gpu = torch.empty(shapes["result_meta"][0], dtype=torch.int64, device=device)
        ring = load().lrr_create(
            L, H, d, self.topk, B, self.capacity, self.result_capacity,
            int(archive_capacity_per_head), int(cpu_threads), device.index,
            *(self.host[name].data_ptr() for name in shapes),
            *(t.data_ptr() for t in (self.archive_gpu, self.archive_meta_gpu, self.query_gpu,
                                     self.result_gpu, self.result_meta_gpu)))
        if not ring:
            raise ValueError(load().lrr_last_error().decode())
        self._ring = ring
        self.thread = _WorkerView(self)
        self.worker_info = dict(kind="ready", thread=_WorkerView.name, pid=os.getpid(),
                                archive="exact-MIPS (host C++)")

    # ---- states --------------------------------------------------------------------------
    @property
    def archive_states(self):
        library = load()
        return [ARCHIVE_STATES[library.lrr_archive_state(self._ring, s)]
                for s in range(self.host["archive_kv"].shape[0])]

    @property
    def query_states(self):
        library = load()
        return [QUERY_STATES[library.lrr_query_state(self._ring, s)] for s in range(2)]

    def pump(self):
        """Reports a worker failure and refreshes the worker's counters (the worker advances
        the slots by itself; there is nothing to forward)."""
        if self.closed:
            return
        library = load()
        if not library.lrr_worker_alive(self._ring):
            raise RuntimeError("CPU recall worker exited unexpectedly")
        _check(library.lrr_check(self._ring))
        values = (ctypes.c_int64 * len(WORKER_COUNTERS))()
        _check(library.lrr_counters(self._ring, values))
        for key, value in zip(WORKER_COUNTERS, values):
            self.counters[key] = int(value)

    # ---- eviction batches ----------------------------------------------------------------
    @staticmethod
    def _batch(removals):
        """(layer, head, position) of every distinct removed slot, in (layer, head, position)
        order: the order the reference packs and archives them (transport.py:141-167)."""
        keys = sorted(removals)
        parts = [np.asarray(removals[key], dtype=np.int64).reshape(-1) for key in keys]
        sizes = np.fromiter((len(p) for p in parts), dtype=np.int64, count=len(parts))
        if not sizes.sum():
            return np.empty((0, 3), np.int64)
        coordinates = np.asarray(keys, dtype=np.int64).reshape(-1, 2)
        segment = np.repeat(np.arange(len(keys), dtype=np.int64), sizes)
        positions = np.concatenate(parts)
        order = np.lexsort((positions, segment))
        segment, positions = segment[order], positions[order]
        keep = np.ones(len(positions), dtype=bool)
        keep[1:] = (segment[1:] != segment[:-1]) | (positions[1:] != positions[:-1])
        segment, positions = segment[keep], positions[keep]
        return np.column_stack((coordinates[segment, 0], coordinates[segment, 1], positions))

    @torch.no_grad()
    def record_evicted(self, cache, removals):
        """transport.py:129-177: pack the evicted rows of every layer into a free archive slot,
        copy them out and archive them (the latter two by the ring, in the background)."""
        self.pump()
        batch = self._batch(removals)
        count = len(batch)
        if count == 0:
            return
        if count > self.capacity:
            self.counters["archive_overflows"] += 1
            raise RuntimeError("Eviction batch exceeds configured archive staging capacity")
        library = load()
        slot, waited = ctypes.c_int(-1), ctypes.c_int(0)
        status = library.lrr_acquire_archive(self._ring, self.timeout, ctypes.byref(slot),
                                             ctypes.byref(waited))
        if waited.value:
            self.counters["archive_backpressure"] += 1
        _check(status)
        slot = slot.value
        try:
            self._pack(cache, batch, slot)
            _check(library.lrr_commit_archive(self._ring, slot, count,
                                              torch.cuda.current_stream(self.device).cuda_stream))
        except BaseException:
            library.lrr_abandon_archive(self._ring, slot)
            raise
        self.counters["archived_vectors"] += count
        self.counters["archive_batches"] += 1
        self.counters["d2h_bytes"] += count * (2 * self.dimension * 2 + 3 * 8)

    @torch.no_grad()
    def record_evicted_heads(self, head_table, slots, heads_per_layer, quotas, offsets,
                             positions, count, max_rows):
        """record_evicted for a fused layout change (an audit's removals or an evict_prefix
        batch), whose removal sets are already on the device: the same capacity check, slot,
        pack layout, commit and counters, with the rows packed by lr_pack_heads straight from
        the sets the compaction reads (device addresses; ``count`` rows, at most ``max_rows``
        from one (layer, head)), on the current stream. The reference packs the same rows from
        host removals (transport.py:129-177)."""
        self.pump()
        count = int(count)
        if count == 0:
            return
        if slots != self.layers * self.heads or heads_per_layer != self.heads:
            raise RuntimeError("Recall configuration does not match the cache")
        if count > self.capacity:
            self.counters["archive_overflows"] += 1
            raise RuntimeError("Eviction batch exceeds configured archive staging capacity")
        library = load()
        slot, waited = ctypes.c_int(-1), ctypes.c_int(0)
        status = library.lrr_acquire_archive(self._ring, self.timeout, ctypes.byref(slot),
                                             ctypes.byref(waited))
        if waited.value:
            self.counters["archive_backpressure"] += 1
        _check(status)
        slot = slot.value
        stream = torch.cuda.current_stream(self.device).cuda_stream
        try:
            _lib.call("lr_pack_heads", head_table, slots, heads_per_layer, quotas, offsets,
                      positions, int(max_rows), self.dimension, self.capacity,
                      self.archive_gpu[slot].data_ptr(), self.archive_meta_gpu[slot].data_ptr(),
                      stream)
            _check(library.lrr_commit_archive(self._ring, slot, count, stream))
        except BaseException:
            library.lrr_abandon_archive(self._ring, slot)
            raise
        self.counters["archived_vectors"] += count
        self.counters["archive_batches"] += 1
        self.counters["d2h_bytes"] += count * (2 * self.dimension * 2 + 3 * 8)

    def _pack(self, cache, batch, slot):
        """One upload (layer pointer table + row descriptors) and one lr_pack_layers launch."""
        L, count = self.layers, len(batch)
        block = torch.empty((4 * L + 3 * count,), dtype=torch.int64, pin_memory=True)
        words = block.numpy()
        table = words[:4 * L].reshape(L, 4)
        table[:] = 0
        rows = words[4 * L:].reshape(count, 3)
        rows[:, :2] = batch[:, :2]
        for layer in np.unique(batch[:, 0]).tolist():
            keys, values = cache.key_cache[layer], cache.value_cache[layer]
            positions = cache.position_cache[layer]
            if not (keys.is_cuda and keys.is_contiguous() and values.is_contiguous()
                    and positions.is_contiguous() and keys.dtype in (torch.bfloat16, torch.float16)
                    and values.dtype == keys.dtype and positions.dtype == torch.float32
                    and keys.shape == values.shape and positions.numel() == keys.shape[0]
                    and keys.shape[1] == self.dimension):
                raise RuntimeError("Expected contiguous CUDA tensor")
            if keys.data_ptr() % 16 or values.data_ptr() % 16:
                raise RuntimeError("Cache rows must be aligned to the row granule")
            starts = np.concatenate(([0], np.cumsum(cache.metadata_list[layer].head_lens_cpu)))
            selected = batch[:, 0] == layer
            rows[selected, 2] = starts[batch[selected, 1]] + batch[selected, 2]
            table[layer] = (keys.data_ptr(), values.data_ptr(), positions.data_ptr(), keys.shape[0])
        device_block = block.to(self.device, non_blocking=True)
        _lib.call("lr_pack_layers", device_block.data_ptr(), L,
                  device_block.data_ptr() + 8 * 4 * L, count, self.dimension,
                  self.archive_gpu[slot].data_ptr(), self.archive_meta_gpu[slot].data_ptr(),
                  torch.cuda.current_stream(self.device).cuda_stream)

    # ---- searches ------------------------------------------------------------------------
    @torch.no_grad()
    def step(self, model, cache, step):
        """transport.py:276-301: every search_interval decode steps, the group-mean decode
        queries of every layer go to the archive; the newest results come back to HBM."""
        self.pump()
        self.retire_finished()
        if step % self.search_interval or not self.counters["archived_vectors"]:
            return
        library = load()
        slot = ctypes.c_int(-1)
        _check(library.lrr_acquire_query(self._ring, ctypes.byref(slot)))
        if slot.value < 0:  # both slots busy: drop the older finished result nobody took
            ready = [(library.lrr_query_step(self._ring, s), s) for s in range(2)
                     if library.lrr_result_ready(self._ring, s)]
            if ready:
                _check(library.lrr_drop_result(self._ring, min(ready)[1]))
                self.counters["superseded_results"] += 1
                _check(library.lrr_acquire_query(self._ring, ctypes.byref(slot)))
        if slot.value < 0:
            self.counters["skipped_busy_queries"] += 1
            return
        slot = slot.value
        try:
            self._query_means(model, slot)
            _check(library.lrr_commit_query(self._ring, slot, int(step),
                                            torch.cuda.current_stream(self.device).cuda_stream))
        except BaseException:
            library.lrr_abandon_query(self._ring, slot)
            raise
        self.counters["submitted_queries"] += 1
        self.counters["d2h_bytes"] += self.layers * self.heads * self.dimension * 4

    def _query_means(self, model, slot):
        blocks = model.model.layers
        if len(blocks) != self.layers:
            raise RuntimeError("Model layer count differs from the recall configuration")
        table = torch.empty((self.layers, 2), dtype=torch.int64, pin_memory=True)
        words = table.numpy()
        dtype = None
        for layer, block in enumerate(blocks):
            query = block.self_attn._last_query_states.detach()[0, :, 0]  # [Hq, d]
            if (not query.is_cuda or query.shape != (self.heads * self.groups, self.dimension)
                    or query.stride(1) != 1):
                raise RuntimeError("Historical query-head count changed")
            if dtype is None:
                dtype = query.dtype
            elif query.dtype != dtype:
                raise RuntimeError("Query dtypes differ between layers")
            words[layer] = (query.data_ptr(), query.stride(0))
        _lib.call("lr_group_mean_queries", table.to(self.device, non_blocking=True).data_ptr(),
                  self.layers, self.heads, self.groups, self.dimension, _lib.DTYPE_CODES[dtype],
                  self.query_gpu[slot].data_ptr(), torch.cuda.current_stream(self.device).cuda_stream)

    def ready_result(self):
        """transport.py:263-280: the newest search whose results are in HBM, as (slot, step,
        payload [n, 2, d] bf16, metadata [n, 3] i64 on the device, metadata on the host); older
        finished results are released."""
        self.pump()
        self.retire_finished()
        library = load()
        ready = [(library.lrr_query_step(self._ring, s), s) for s in range(2)
                 if library.lrr_result_ready(self._ring, s)]
        if not ready:
            return None
        step, chosen = max(ready)
        for _, slot in ready:
            if slot != chosen:
                self.release_result(slot)
                self.counters["superseded_results"] += 1
        count = int(library.lrr_result_count(self._ring, chosen))
        return (chosen, int(step), self.result_gpu[chosen, :count],
                self.result_meta_gpu[chosen, :count],
                self.host["result_meta"][chosen, :count].numpy().copy())

    def release_result(self, slot):
        """The consumer's work on the current stream is the slot's last use (transport.py:
        231-235)."""
        _check(load().lrr_release_result(self._ring, int(slot),
                                         torch.cuda.current_stream(self.device).cuda_stream))

    def retire_finished(self):
        if self._ring:
            _check(load().lrr_retire(self._ring))

    def remove_admitted(self, metadata):
        metadata = np.ascontiguousarray(np.asarray(metadata, dtype=np.int64).reshape(-1, 3))
        _check(load().lrr_remove(self._ring, metadata.ctypes.data, len(metadata)))

    def wait_pending(self):
        """Every archive batch archived, every search answered and its results in HBM."""
        _check(load().lrr_wait_pending(self._ring, self.timeout))
        self.pump()

    def finish(self):
        """transport.py:328-343: results nobody took are released, the consumer's stream is
        drained, and every queued job (removals included) has run."""
        self.wait_pending()
        library = load()
        for slot in range(2):
            if library.lrr_query_state(self._ring, slot) == RESULT_STATE:
                self.release_result(slot)
        torch.cuda.current_stream(self.device).synchronize()
        self.retire_finished()
        _check(library.lrr_flush(self._ring, self.timeout))
        self.pump()

    @property
    def stats(self):
        if hasattr(self, "_closed_stats"):
            return dict(self._closed_stats)
        device = (self.archive_gpu, self.archive_meta_gpu, self.query_gpu, self.result_gpu,
                  self.result_meta_gpu)
        return dict(self.counters, worker=self.worker_info,
                    registered_shared_bytes=sum(t.numel() * t.element_size()
                                                for t in self.host.values()),
                    gpu_staging_bytes=sum(t.numel() * t.element_size() for t in device))

    def close(self, abort=False):
        """Stops the worker (after the jobs already queued) and releases the ring; the
        staging buffers go with this object."""
        if self.closed:
            return
        if self._ring:
            if not abort:
                self.pump()
            self._closed_stats = self.stats
            load().lrr_destroy(self._ring)
            self._ring = None
        self.closed = True
        torch.cuda.synchronize(self.device)

    def __del__(self):
        if getattr(self, "_ring", None) and _library is not None:
            _library.lrr_destroy(self._ring)
            self._ring = None
