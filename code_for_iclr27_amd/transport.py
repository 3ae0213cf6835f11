"""The recall transport: evicted KV rows stream to a CPU-owned exact-MIPS archive, periodic
per-(layer, head) queries search it, and the results come back to HBM for reinsertion.

Drop-in for ``RecallTransport`` of src/lazy_recall/recall/transport.py:46-361: same
constructor, methods (record_evicted, pump, ready_result, release_result, retire_finished,
remove_admitted, wait_pending, step, finish, close), slot states, counters and errors. The
layout differs where this pool differs from the reference's:

- staging buffers are pinned host allocations (``pin_memory=True``, hipHostMalloc) instead of
  shared-memory segments pinned with hipHostRegister (refused here for existing memory);
- the archive (code_for_iclr27_amd.archive, host C++) runs on a worker thread of this process
  instead of a spawned process fed through queues: its calls release the GIL, so the decode
  loop keeps running while it adds or searches; commands and replies keep the reference's
  message kinds;
- rows are gathered into the staging slot by the HIP ``pack`` kernel (code_for_iclr27_amd._C)
  and copied device-to-host / host-to-device on a side stream of default priority, ordered by
  events, as the reference does.
"""

from __future__ import annotations

import queue
import resource
import threading
import time
from collections import deque

import numpy as np
import torch

from . import _C
from .archive import ArchiveIndex


def _worker(index, topk, views, commands, replies):
    """cpu_worker.py:136-182 as a thread: the same commands and replies."""
    try:
        while True:
            message = commands.get()
            kind, slot = message["kind"], message.get("slot")
            started = time.perf_counter_ns()
            if kind == "stop":
                return
            if kind == "archive":
                count = message["count"]
                index.add(views["archive_meta"][slot, :count], views["archive_kv"][slot, :count])
                reply = dict(kind="archived", slot=slot, count=count)
            elif kind == "remove":
                index.remove(message["metadata"])
                continue
            elif kind == "search":
                metadata, payload = index.search(views["queries"][slot], topk)
                count = len(metadata)
                views["result_meta"][slot, :count] = metadata
                views["result_kv"][slot, :count] = payload
                reply = dict(kind="searched", slot=slot, count=count, query_step=message["step"])
            elif kind == "flush":
                reply = dict(kind="flushed")
            else:
                raise ValueError(f"Unknown worker command: {kind}")
            reply.update(indexed=index.size, capacity_drops=index.dropped, start_ns=started,
                         end_ns=time.perf_counter_ns(),
                         cpu_peak_rss_kib=resource.getrusage(resource.RUSAGE_SELF).ru_maxrss)
            replies.put(reply)
    except BaseException:  # reported to the owner like the reference's worker errors
        import traceback

        replies.put(dict(kind="error", traceback=traceback.format_exc()))


class RecallTransport:
    def __init__(self, layers, heads, query_heads, dimension, search_interval=32,
                 topk=4, archive_buffers=16, cpu_threads=2, evict_interval=8,
                 archive_capacity_per_head=32768, timeout_seconds=60.0):
        if query_heads % heads or min(layers, heads, dimension, search_interval, topk,
                                      archive_buffers, cpu_threads) <= 0:
            raise ValueError("Invalid recall configuration")
        self.layers, self.heads, self.groups = layers, heads, query_heads // heads
        self.dimension = dimension
        self.search_interval = search_interval
        self.capacity = max(evict_interval, topk) * layers * heads
        self.result_capacity = topk * layers * heads
        self.timeout = timeout_seconds
        self.closed = False
        self.thread = None
        self.copy_stream = torch.cuda.Stream()
        self.archive_states = ["free"] * archive_buffers
        self.query_states = ["free"] * 2
        self.archive_jobs, self.query_jobs, self.events = {}, {}, deque(maxlen=32)
        self.counters = dict(archived_vectors=0, archive_batches=0, indexed_vectors=0,
                             submitted_queries=0, searches_completed=0, skipped_busy_queries=0,
                             retrieved_vectors=0, spliced_vectors=0, splices=0,
                             d2h_bytes=0, h2d_bytes=0, archive_overflows=0,
                             cpu_peak_rss_kib=0, query_age_tokens_max=0,
                             archive_backpressure=0, capacity_drops=0, superseded_results=0)
        specs = dict(archive_kv=((archive_buffers, self.capacity, 2, dimension), torch.int16),
                     archive_meta=((archive_buffers, self.capacity, 3), torch.int64),
                     queries=((2, layers, heads, dimension), torch.float32),
                     result_kv=((2, self.result_capacity, 2, dimension), torch.int16),
                     result_meta=((2, self.result_capacity, 3), torch.int64))
        self.host = {name: torch.empty(shape, dtype=dtype, pin_memory=True)
                     for name, (shape, dtype) in specs.items()}
        views = {name: tensor.numpy() for name, tensor in self.host.items()}
        views["archive_kv"] = views["archive_kv"].view(np.uint16)
        views["result_kv"] = views["result_kv"].view(np.uint16)
        self.views = views
        self.archive_gpu = torch.empty(specs["archive_kv"][0], device="cuda", dtype=torch.bfloat16)
        self.archive_meta_gpu = torch.empty(specs["archive_meta"][0], device="cuda", dtype=torch.int64)
        self.query_gpu = torch.empty(specs["queries"][0], device="cuda", dtype=torch.float32)
        self.result_gpu = torch.empty(specs["result_kv"][0], device="cuda", dtype=torch.bfloat16)
        self.result_meta_gpu = torch.empty(specs["result_meta"][0], device="cuda", dtype=torch.int64)
        self.config = dict(layers=layers, heads=heads, dimension=dimension, topk=topk,
                           cpu_threads=cpu_threads,
                           archive_capacity_per_head=archive_capacity_per_head)
        self.index = ArchiveIndex(layers, heads, dimension, cpu_threads, archive_capacity_per_head)
        self.commands = queue.Queue(maxsize=archive_buffers + 6)
        self.replies = queue.Queue()
        self.thread = threading.Thread(target=_worker, name="LazyRecall-CPU-archive", daemon=True,
                                       args=(self.index, topk, views, self.commands, self.replies))
        self.thread.start()
        self.worker_info = dict(kind="ready", thread=self.thread.name, archive="exact-MIPS C++")

    def _send(self, message):
        try:
            self.commands.put(message, timeout=self.timeout)
        except queue.Full as error:
            raise RuntimeError("Recall command queue backpressure exceeded timeout") from error

    def _copy_out(self, pairs):
        packed = torch.cuda.Event()
        packed.record(torch.cuda.current_stream())
        done = torch.cuda.Event()
        with torch.cuda.stream(self.copy_stream):
            self.copy_stream.wait_event(packed)
            for destination, source in pairs:
                destination.copy_(source, non_blocking=True)
                self.counters["d2h_bytes"] += source.numel() * source.element_size()
            done.record(self.copy_stream)
        return done

    @torch.no_grad()
    def record_evicted(self, cache, removals):
        """transport.py:130-177: gather {(layer, head): positions} into a free staging slot with
        the pack kernel and start its copy to host memory."""
        self.pump()
        count = sum(len(set(positions)) for positions in removals.values())
        if count == 0:
            return
        if count > self.capacity:
            self.counters["archive_overflows"] += 1
            raise RuntimeError("Eviction batch exceeds configured archive staging capacity")
        started = time.perf_counter()
        if "free" not in self.archive_states:
            self.counters["archive_backpressure"] += 1
        while "free" not in self.archive_states:
            if time.perf_counter() - started > self.timeout:
                raise TimeoutError("CPU archive backpressure exceeded timeout")
            self.pump()
            time.sleep(0.001)
        slot = self.archive_states.index("free")
        # Every layer's absolute rows and head ids in one host array, uploaded with one
        # non-blocking copy from pinned memory (the reference uploads two tensors per layer).
        plan = []
        rows_all, heads_all = [], []
        for layer in sorted({layer for layer, _ in removals}):
            bounds = np.concatenate(([0], np.cumsum(cache.metadata_list[layer].head_lens_cpu)))
            start = len(rows_all)
            for (record_layer, head), positions in sorted(removals.items()):
                if record_layer == layer:
                    selected = sorted(set(int(position) for position in positions))
                    rows_all.extend(int(bounds[head]) + position for position in selected)
                    heads_all.extend([head] * len(selected))
            if len(rows_all) > start:
                plan.append((layer, start, len(rows_all)))
        table = torch.tensor([rows_all, heads_all], dtype=torch.int64).pin_memory()
        table = table.to("cuda", non_blocking=True)
        cursor = 0
        for layer, start, end in plan:
            _C.pack(cache.key_cache[layer].contiguous(), cache.value_cache[layer].contiguous(),
                    cache.position_cache[layer].contiguous(), table[0, start:end],
                    table[1, start:end], layer, self.archive_gpu[slot, start:end],
                    self.archive_meta_gpu[slot, start:end])
            cursor = end
        if cursor != count:
            raise AssertionError("Archive packing count mismatch")
        done = self._copy_out([
            (self.host["archive_kv"][slot, :count].view(torch.bfloat16), self.archive_gpu[slot, :count]),
            (self.host["archive_meta"][slot, :count], self.archive_meta_gpu[slot, :count]),
        ])
        self.archive_states[slot] = "copying"
        self.archive_jobs[slot] = dict(event=done, count=count)
        self.counters["archived_vectors"] += count
        self.counters["archive_batches"] += 1

    @torch.no_grad()
    def pump(self):
        """transport.py:180-229: advance every slot whose copy or worker job has finished."""
        if self.closed:
            return
        if not self.thread.is_alive():
            raise RuntimeError("CPU recall worker exited unexpectedly")
        for slot, job in list(self.archive_jobs.items()):
            if self.archive_states[slot] == "copying" and job["event"].query():
                self._send(dict(kind="archive", slot=slot, count=job["count"]))
                self.archive_states[slot] = "worker"
        for slot, job in list(self.query_jobs.items()):
            if self.query_states[slot] == "copying_query" and job["event"].query():
                self._send(dict(kind="search", slot=slot, step=job["step"]))
                self.query_states[slot] = "worker"
        while True:
            try:
                message = self.replies.get_nowait()
            except queue.Empty:
                break
            kind, slot = message["kind"], message.get("slot")
            if kind == "error":
                raise RuntimeError(message["traceback"])
            if kind not in ("archived", "searched", "flushed"):
                raise RuntimeError(f"Unexpected CPU reply: {message}")
            self.events.append(dict(kind=kind, start_ns=message["start_ns"], end_ns=message["end_ns"]))
            self.counters["indexed_vectors"] = message["indexed"]
            self.counters["capacity_drops"] = message.get("capacity_drops", 0)
            self.counters["cpu_peak_rss_kib"] = max(self.counters["cpu_peak_rss_kib"],
                                                    message["cpu_peak_rss_kib"])
            if kind == "flushed":
                self._flushed = True
            elif kind == "archived":
                del self.archive_jobs[slot]
                self.archive_states[slot] = "free"
            else:
                self.counters["searches_completed"] += 1
                self.counters["retrieved_vectors"] += message["count"]
                job = self.query_jobs[slot]
                job.update(count=message["count"], indexed=message["indexed"])
                if not message["count"]:
                    del self.query_jobs[slot]
                    self.query_states[slot] = "free"
                    continue
                count = job["count"]
                done = torch.cuda.Event()
                with torch.cuda.stream(self.copy_stream):
                    self.result_gpu[slot, :count].copy_(
                        self.host["result_kv"][slot, :count].view(torch.bfloat16), non_blocking=True)
                    self.result_meta_gpu[slot, :count].copy_(self.host["result_meta"][slot, :count],
                                                             non_blocking=True)
                    done.record(self.copy_stream)
                self.counters["h2d_bytes"] += count * (2 * self.dimension * 2 + 3 * 8)
                job["event"] = done
                self.query_states[slot] = "copying_result"

    def release_result(self, slot):
        complete = torch.cuda.Event()
        complete.record(torch.cuda.current_stream())
        self.query_jobs[slot]["event"] = complete
        self.query_states[slot] = "retiring"

    def retire_finished(self):
        for slot, job in list(self.query_jobs.items()):
            if self.query_states[slot] == "retiring" and job["event"].query():
                del self.query_jobs[slot]
                self.query_states[slot] = "free"

    def ready_result(self):
        """transport.py:243-258: the newest search result resident in HBM, older ones released:
        (slot, step, payload [n, 2, d] bf16, metadata [n, 3] i64 on the device, metadata host)."""
        self.pump()
        self.retire_finished()
        candidates = [(job["step"], slot) for slot, job in self.query_jobs.items()
                      if self.query_states[slot] == "copying_result" and job["event"].query()]
        if not candidates:
            return None
        _, chosen = max(candidates)
        for _, slot in candidates:
            if slot != chosen:
                self.release_result(slot)
                self.counters["superseded_results"] += 1
        job = self.query_jobs[chosen]
        return (chosen, job["step"], self.result_gpu[chosen, :job["count"]],
                self.result_meta_gpu[chosen, :job["count"]],
                self.views["result_meta"][chosen, :job["count"]].copy())

    def remove_admitted(self, metadata):
        self._send(dict(kind="remove", metadata=np.asarray(metadata, dtype=np.int64).tolist()))

    def wait_pending(self):
        started = time.perf_counter()
        while self.archive_jobs or any(
            self.query_states[slot] in ("copying_query", "worker")
            or (self.query_states[slot] == "copying_result" and not job["event"].query())
            for slot, job in self.query_jobs.items()
        ):
            if time.perf_counter() - started > self.timeout:
                raise TimeoutError("Recall diagnostic wait exceeded timeout")
            self.pump()
            self.retire_finished()
            time.sleep(0.001)

    @torch.no_grad()
    def step(self, model, cache, step):
        """transport.py:277-301: every search_interval steps, submit one query per (layer, KV
        head): the mean over its query group of the last decode query."""
        del cache
        self.pump()
        self.retire_finished()
        if step % self.search_interval or not self.counters["archived_vectors"]:
            return
        if "free" not in self.query_states:
            ready = [(job["step"], slot) for slot, job in self.query_jobs.items()
                     if self.query_states[slot] == "copying_result" and job["event"].query()]
            if ready:
                _, oldest = min(ready)
                del self.query_jobs[oldest]
                self.query_states[oldest] = "free"
                self.counters["superseded_results"] += 1
        if "free" not in self.query_states:
            self.counters["skipped_busy_queries"] += 1
            return
        slot = self.query_states.index("free")
        for layer, block in enumerate(model.model.layers):
            query = block.self_attn._last_query_states.detach()[0, :, 0]
            self.query_gpu[slot, layer].copy_(
                query.view(self.heads, self.groups, self.dimension).float().mean(dim=1))
        done = self._copy_out([(self.host["queries"][slot], self.query_gpu[slot])])
        self.query_jobs[slot] = dict(event=done, step=step)
        self.query_states[slot] = "copying_query"
        self.counters["submitted_queries"] += 1

    def finish(self):
        self.wait_pending()
        for slot in list(self.query_jobs):
            if self.query_states[slot] == "copying_result":
                self.release_result(slot)
        torch.cuda.current_stream().synchronize()
        self.retire_finished()
        self._flushed = False
        self._send(dict(kind="flush"))
        started = time.perf_counter()
        while not self._flushed:
            if time.perf_counter() - started > self.timeout:
                raise TimeoutError("CPU archive flush exceeded timeout")
            self.pump()
            time.sleep(0.001)

    @property
    def stats(self):
        if hasattr(self, "_closed_stats"):
            return dict(self._closed_stats)
        return dict(self.counters, worker=self.worker_info,
                    pinned_host_bytes=sum(t.numel() * t.element_size() for t in self.host.values()),
                    gpu_staging_bytes=sum(t.numel() * t.element_size() for t in
                                          (self.archive_gpu, self.archive_meta_gpu, self.query_gpu,
                                           self.result_gpu, self.result_meta_gpu)))

    def close(self, abort=False):
        if self.closed:
            return
        self._closed_stats = self.stats
        self.closed = True
        if self.thread is not None and self.thread.is_alive():
            try:
                self.commands.put(dict(kind="stop"), timeout=5)
            except queue.Full:
                pass
            if not abort:
                self.thread.join(timeout=self.timeout)
        torch.cuda.synchronize()
        for name in ("archive_gpu", "archive_meta_gpu", "query_gpu", "result_gpu", "result_meta_gpu"):
            if hasattr(self, name):
                delattr(self, name)
