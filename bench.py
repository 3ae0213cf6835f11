#!/usr/bin/env python3
"""Benchmark of the LazyRecall KV-management hot path on one MI355X.

Headline metric: one full audit step on the Llama-3.1-8B cache (cfg1:
32 layers x 8 KV heads x d128, 2250 tokens per head, window 250, G=4): temporal scores of all
567,808 candidates -> Pool7 -> allocation-preserving selection of 64,000 slots -> compaction
of every layer. value = algorithmic bytes of the step / measured step time (GB/s).

The step removes every selected slot at once, so the eviction queue it leaves is empty and its
order is not computed (queue_order_ms_per_step times the step with that order computed too,
over as many steps and warm-up steps as the headline, so that the two compare: a shorter run
carries a larger share of the first step's exposed host work).

Also reported on the same line:
  roofline      the dominant kernel, timed with HIP events on its stream inside the timed loop
                (the only events recorded there)
  stages_us     every stage of the step, from separate steps with events between all stages
  cpu_baseline  the reference's CPU math path (LAZY_RECALL_BUILD_CUDA=0 semantics, restated in
                oracle/cpu_path.py) on a bounded sample of the same workload, host cores
  lazy_window   the controller's steady state at cfg1: an audit that removes 2 of its 250
                selected slots per head at once and queues the rest on the device, then the 31
                evict_prefix batches (8 per head each) that drain the queue
  reinsert      cfg3 recall reinsertion of 512 recalled K/V rows per (layer, head) from pinned
                host memory: end to end (planning, copy and merge overlapped), the host-link
                copy alone (GB/s) and the merge of all 32 layers alone (HBM GB/s)
  ops           the other entry points on their own shapes (append, the legacy flat-cache
                ops, per-layer compact, pack, cfg2 batch_append, packed decode attention on
                cfg1/cfg2 layers, the audit's head logits / hidden gradient / pre-gradient at
                Llama-3.1-8B shapes): device time per call from a held stream, GB/s against the
                HBM peak, host-inclusive step time; and the host recall archive's exact-MIPS
                search (cfg1 shape, 4096 archived rows per head)
  audit_configs the audit step on cfg0 (Llama-3.2-1B), cfg4 (Qwen3.5-style, d256, G6) and cfg3
                (Llama-3.1-8B long budget: 33,792 tokens per head, 1,024 evicted per head)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg1]
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "audit-step KV GB/s (% of HBM peak) + reinsert GB/s, Llama-3.1-8B shape"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--config", default="cfg1")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--cpu-seconds", type=float, default=10.0,
                        help="target CPU work for the bounded CPU-baseline sample")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-reinsert", action="store_true", help="skip the cfg3 reinsertion")
    parser.add_argument("--no-lazy", action="store_true",
                        help="skip the lazy-eviction window (audit + 31 evict_prefix batches)")
    parser.add_argument("--no-ops", action="store_true",
                        help="skip the append / legacy / pack / cfg2 batch-append measurements")
    parser.add_argument("--other-configs", default="cfg0,cfg4,cfg3",
                        help="comma-separated further audit configurations to time ('' for none)")
    parser.add_argument("--event-every", type=int, default=5, metavar="K",
                        help="inside the timed steps, bracket the dominant kernel with events on "
                             "every K-th step (each event costs the GPU a few microseconds)")
    parser.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                        help="first run one plain elementwise copy (negation) of MIB MiB f32, "
                             "the reference dispatch for scaling FETCH_SIZE / WRITE_SIZE counters")
    return parser.parse_args()


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "audit_kernels_cfg1_hbm_traffic.md")


def measured_traffic(kernel, config):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (lines `traffic_bytes_per_launch <config> <kernel> <bytes>`), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                parts = line.split()
                if (len(parts) == 4 and parts[0] == "traffic_bytes_per_launch"
                        and parts[1] == config and parts[2] == kernel):
                    return int(parts[3])
    except OSError:
        pass
    return None


SQ_PROFILE = os.path.join(ROOT, "profiles", "scorer_cfg1_sq_counters.md")
SIMDS, ENGINE_CLOCK_GHZ = 1024, 2.4  # MI355X: 256 CUs x 4 SIMDs, peak engine clock


def measured_valu_cycles(kernel, config):
    """VALU-active cycles (all waves) per launch of `kernel`, from the committed rocprofv3
    SQ_ACTIVE_INST_VALU summary (lines `valu_active_cycles_per_launch <config> <kernel> <n>`),
    or None."""
    try:
        with open(SQ_PROFILE) as f:
            for line in f:
                parts = line.split()
                if (len(parts) == 4 and parts[0] == "valu_active_cycles_per_launch"
                        and parts[1] == config and parts[2] == kernel):
                    return int(parts[3])
    except OSError:
        pass
    return None


class EventTimer:
    """Records a HIP event on the current stream at each mark (events are created up front,
    outside the timed loop). With `only`, marks with other names record nothing: every event
    record costs the GPU a few microseconds between kernels, so the timed steps bracket only
    the dominant kernel."""

    def __init__(self, torch, capacity=16, only=None):
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(capacity)]
        self.marks = []
        self.only = only

    def mark(self, name):
        if self.only is not None and name not in self.only:
            return
        event = self.events[len(self.marks)]
        event.record()
        self.marks.append((name, event))

    def stages(self):
        out = {}
        for (_, a), (name, b) in zip(self.marks, self.marks[1:]):
            out[name] = a.elapsed_time(b) * 1000.0  # us
        return out


def audit_bytes(cfg, rows_total, count, candidates_total, segments):
    """Algorithmic HBM bytes of one audit step (K,V,Q,positions,gradients read once; scores,
    pool and selection tables once; compaction reads and writes each kept row once)."""
    T, d, W, G = cfg.length, cfg.dim, cfg.window, cfg.groups
    heads = cfg.layers * cfg.heads
    score = heads * (2 * T * d * 2 + W * G * d * 2 + T * 4 + W * 8 + G * d * 4) + candidates_total * 4
    select = candidates_total * 4 * 4
    kept = rows_total - count
    compact = 2 * kept * d * 2 * 2 + kept * 4 * 2 + count * 8
    return score + select + compact


def cpu_baseline(torch, layers, qpos, margin, cfg, target_seconds):
    from oracle import cpu_path

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    host = []
    for layer in layers:
        host.append(dict(keys=layer.keys.cpu(), values=layer.values.cpu(),
                         positions=layer.positions.cpu(), head_lens=list(layer.head_lens),
                         queries=layer.queries.cpu(), gradient=layer.gradient.cpu()))
    qpos_c, margin_c = qpos.cpu(), margin.cpu().reshape(())

    def step(n):
        started = time.perf_counter()
        cpu_path.audit_step_cpu(host[:n], qpos_c, margin_c, cfg.evict_per_head * cfg.heads * n,
                                cfg.protect_recent, cfg.pool_kernel, cfg.epsilon)
        return time.perf_counter() - started

    # a one-layer step sizes the sample: the whole audit step over as many layers as make each
    # of the `runs` timed runs about target_seconds / runs; then one warm-up run of that sample
    # and the median of the timed runs
    runs = 5
    per_layer = step(1)
    n = max(1, min(len(host), int(target_seconds / runs / max(per_layer, 1e-3))))
    step(n)
    times = sorted(step(n) for _ in range(runs))
    seconds = times[runs // 2]
    scaled = seconds * len(host) / n
    return n, seconds, scaled, threads, [round(t, 3) for t in times]


def reinsert_bench(torch, seed, reps=5):
    """cfg3: 32 layers x 8 heads x 33,792 resident tokens, 512 recalled tokens per head held in
    pinned host memory with their identities, reinserted at random hole positions.

    end_to_end_ms: host-inclusive time of code_for_iclr27_amd.reinsert with the payload and
    the identities in pinned host memory (as the recall transport stages them): the table on
    the host, the identities and then the payload copied in on a side stream, the grouping and
    plan on the device, the resident-row merge overlapping the payload copy, the recalled-row
    merge; synchronised. end_to_end_host_grouped_ms: the same with the identities as a numpy
    array, grouped on the host in C++ before the launches. h2d: the payload and metadata copy
    alone (host-link GB/s). merge: the reinsertion with payload and identities already in HBM,
    device time from events. merge_per_layer: the reference-shaped drop-in (_C.merge per layer
    with a precomputed merge_plan mapping)."""
    import numpy as np

    from code_for_iclr27_amd import _C, planning, reinsert
    from code_for_iclr27_amd.scoring import LayerState

    L, H, d, T, M = 32, 8, 128, 33792, 512
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed + 3)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 3)
    layers, mappings, meta_rows = [], [], []
    for layer in range(L):
        keys = torch.randn((H * T, d), generator=gen, device=dev).to(torch.bfloat16)
        values = torch.randn((H * T, d), generator=gen, device=dev).to(torch.bfloat16)
        pos_parts, meta = [], []
        for head in range(H):
            holes = rng.choice(T + M, M, replace=False)
            keep = np.ones(T + M, bool)
            keep[holes] = False
            pos_parts.append(np.flatnonzero(keep))
            meta.extend((layer, head, int(p)) for p in holes)
        old = np.concatenate(pos_parts)
        meta = np.asarray(meta, dtype=np.int64)
        mapping, _ = planning.merge_plan(old, [T] * H, meta)
        positions = torch.from_numpy(old.astype(np.float32)).to(dev)
        layers.append(LayerState(keys, values, positions, [T] * H, None, None, None))
        mappings.append(torch.from_numpy(mapping).to(dev))
        meta_rows.append(meta)
    metadata = np.concatenate(meta_rows)
    total = L * H * M
    payload_host = torch.empty((total, 2, d), dtype=torch.bfloat16, pin_memory=True)
    payload_host.copy_(torch.randn((total, 2, d), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16))
    meta_host = torch.from_numpy(metadata).pin_memory()
    payload = torch.empty((total, 2, d), dtype=torch.bfloat16, device=dev)
    meta_dev = torch.empty((total, 3), dtype=torch.int64, device=dev)
    runner = reinsert.Reinserter()
    end_to_end, host_grouped, link, merge, per_layer = [], [], [], [], []
    outcome = None
    for rep in range(reps + 1):
        outcome = None
        torch.cuda.synchronize()
        started = time.perf_counter()
        outcome = runner.run(layers, payload_host, metadata)
        torch.cuda.synchronize()
        host_grouped.append((time.perf_counter() - started) * 1e3)
        outcome = None
        torch.cuda.synchronize()
        started = time.perf_counter()
        outcome = runner.run(layers, payload_host, meta_host)
        torch.cuda.synchronize()
        end_to_end.append((time.perf_counter() - started) * 1e3)
        e0, e1, e2, e3, e4 = (torch.cuda.Event(enable_timing=True) for _ in range(5))
        e0.record()
        payload.copy_(payload_host, non_blocking=True)
        meta_dev.copy_(meta_host, non_blocking=True)
        e1.record()
        torch.cuda.synchronize()
        outcome = None
        e2.record()
        outcome = runner.run(layers, payload, meta_dev)
        e3.record()
        torch.cuda.synchronize()
        recalled_positions = meta_dev[:, 2].to(torch.float32)
        e4.record()
        for layer in range(L):
            state = layers[layer]
            rows = slice(layer * H * M, (layer + 1) * H * M)
            _C.merge(state.keys, state.values, state.positions, payload[rows],
                     recalled_positions[rows], mappings[layer])
        e5 = torch.cuda.Event(enable_timing=True)
        e5.record()
        torch.cuda.synchronize()
        if rep:  # the first repetition warms up
            link.append(e0.elapsed_time(e1))
            merge.append(e2.elapsed_time(e3))
            per_layer.append(e4.elapsed_time(e5))
    end_to_end, host_grouped = end_to_end[1:], host_grouped[1:]
    link_bytes = total * (2 * d * 2 + 3 * 8)
    n_rows, m_rows = L * H * T, total
    merge_bytes = (n_rows + m_rows) * 2 * d * 2 * 2 + n_rows * 4 * 2 + m_rows * (4 + 24)
    per_layer_bytes = L * ((H * T + H * M) * 2 * d * 2 * 2 + (H * T + H * M) * (4 + 4 + 8))
    link_ms, merge_ms = float(np.median(link)), float(np.median(merge))
    e2e_ms, per_layer_ms = float(np.median(end_to_end)), float(np.median(per_layer))
    # spot check: merged positions ascend within every head of a layer
    check = outcome.layers[0].positions.reshape(H, T + M).cpu().numpy()
    assert (np.diff(check, axis=1) > 0).all(), "reinserted positions are not ordered"
    return {
        "workload": "cfg3: 32 layers x 8 KV heads x 33,792 tokens, 512 recalled per (layer, head)",
        "end_to_end_ms": round(e2e_ms, 3),
        "end_to_end_host_grouped_ms": round(float(np.median(host_grouped)), 3),
        "overlap_vs_max_of_h2d_and_merge": round(max(link_ms, merge_ms) / e2e_ms, 3),
        "h2d_GBps": round(link_bytes / (link_ms / 1e3) / 1e9, 2),
        "h2d_ms": round(link_ms, 3),
        "h2d_bytes": link_bytes,
        "merge_GBps": round(merge_bytes / (merge_ms / 1e3) / 1e9, 1),
        "merge_ms": round(merge_ms, 3),
        "merge_hbm_fraction": round(merge_bytes / (merge_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 3),
        "merge_bytes": merge_bytes,
        "merge_per_layer_ms": round(per_layer_ms, 3),
        "merge_per_layer_GBps": round(per_layer_bytes / (per_layer_ms / 1e3) / 1e9, 1),
    }


class HeldStream:
    """Device time of a run of calls without the host's enqueue gaps: a bounded spin kernel
    (torch.cuda._sleep) holds the current stream while the host enqueues the calls and an event
    after each, so consecutive events bracket the calls back to back on the device."""

    def __init__(self, torch):
        self.torch = torch
        cycles = 1 << 22
        a, b = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        torch.cuda.synchronize()
        a.record()
        torch.cuda._sleep(cycles)
        b.record()
        torch.cuda.synchronize()
        self.cycles_per_ms = cycles / max(a.elapsed_time(b), 1e-3)

    def run(self, calls, hold_ms=20.0):
        """Returns (per-call device microseconds, host enqueue milliseconds); the hold is
        lengthened and the run repeated while the enqueue outlasts it."""
        torch = self.torch
        events = [torch.cuda.Event(enable_timing=True) for _ in range(len(calls) + 1)]
        while True:
            torch.cuda.synchronize()
            torch.cuda._sleep(int(self.cycles_per_ms * hold_ms))
            started = time.perf_counter()
            events[0].record()
            for call, event in zip(calls, events[1:]):
                call()
                event.record()
            enqueue_ms = (time.perf_counter() - started) * 1e3
            torch.cuda.synchronize()
            if enqueue_ms < 0.8 * hold_ms or hold_ms > 2000:
                break
            hold_ms *= 4
        return [a.elapsed_time(b) * 1e3 for a, b in zip(events, events[1:])], enqueue_ms


def _op_line(workload, calls, device_us, nbytes, wall_ms):
    """One `ops` entry: median device time per call, bytes per call, HBM roofline fraction."""
    import numpy as np

    us = float(np.median(device_us))
    gbps = nbytes / (us / 1e6) / 1e9
    return {"workload": workload, "calls_per_step": calls, "device_us_per_call": round(us, 2),
            "bytes_per_call": int(nbytes), "GBps": round(gbps, 1),
            "hbm_fraction": round(gbps / HBM_PEAK_GBPS, 4),
            "wall_ms_per_step": round(wall_ms, 3)}


def nbytes_append_layer(rows, heads, dim):
    """Algorithmic bytes of one layer's one-token append: K and V read and written, the
    positions read and written, the new rows read."""
    return (2 * rows * dim * 2 + 2 * (rows + heads) * dim * 2 + rows * 4 + (rows + heads) * 4
            + 2 * heads * dim * 2)


def ops_bench(torch, seed, reps=5):
    """The scope table's data-movement rows outside the audit step, on their own shapes:
    decode-time appends (cfg1 layer, cfg2 static batch), the legacy flat-cache ops, the per-layer
    compaction and the eviction archive pack. Each call's device time comes from a held stream;
    wall_ms_per_step is the host-inclusive time of one decode/audit step's worth of calls."""
    import numpy as np

    from code_for_iclr27_amd import _C, _legacy_C

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 7)
    rng = np.random.default_rng(seed + 7)
    held = HeldStream(torch)
    bf16 = torch.bfloat16
    L, H, d, T, E = 32, 8, 128, 2250, 250  # cfg1 layer shape, 250 evicted per head
    rows = H * T

    def randn(*shape):
        return torch.randn(shape, generator=gen, device=dev).to(bf16)

    def measure(make_calls, per_step):
        calls = make_calls()
        for call in calls[:2]:  # warm the allocator and the library
            call()
        device = []
        for _ in range(reps):
            us, _ = held.run(calls)
            device.extend(us)
        torch.cuda.synchronize()
        walls = []
        for _ in range(reps):
            started = time.perf_counter()
            for call in calls[:per_step]:
                call()
            torch.cuda.synchronize()
            walls.append((time.perf_counter() - started) * 1e3)
        return device, float(np.median(walls))

    out = {}
    # every layer has its own K/V (32 x 18.4 MB, beyond the 256 MB Infinity Cache), as in a
    # decode step, so no call reads rows another call left in the cache
    keys = [randn(rows, d) for _ in range(L)]
    values = [randn(rows, d) for _ in range(L)]
    positions = torch.arange(T, dtype=torch.float32, device=dev).repeat(H)[:, None].contiguous()
    cumulative = torch.arange(0, rows + 1, T, dtype=torch.int32, device=dev)
    new_k, new_v = randn(1, H, 1, d), randn(1, H, 1, d)

    # a10 append: one token per head into every layer (cache.py:33-52)
    device, wall = measure(lambda: [
        (lambda l=l: _C.append(keys[l], values[l], positions, new_k, new_v, cumulative,
                               T, T)) for l in range(L)], L)
    nbytes = nbytes_append_layer(rows, H, d)
    out["append"] = _op_line("cfg1 layer: 8 heads x 2250 rows + 1 token per head, bf16 d128", L,
                             device, nbytes, wall)

    # the same decode step's appends of all 32 layers in one launch (packed outputs)
    device, wall = measure(lambda: [
        (lambda: _C.append_layers(keys, values, [positions] * L, [new_k] * L,
                                  [new_v] * L, [cumulative] * L, [T] * L, T))
        for _ in range(4)], 1)
    out["append_layers"] = _op_line("cfg1 decode step: all 32 layers' appends in one launch", 1,
                                    device, L * nbytes, wall)

    # a11 append_flattened_cache: K and V of every layer (cache_legacy.cu:145-197)
    head_lens = torch.full((H,), T, dtype=torch.int32, device=dev)
    device, wall = measure(lambda: [
        (lambda l=l: _legacy_C.append_flattened_cache((keys if l < L else values)[l % L], new_k,
                                                       head_lens, cumulative))
        for l in range(2 * L)], 2 * L)
    nbytes = rows * d * 2 + (rows + H) * d * 2 + H * d * 2
    out["append_flattened_cache"] = _op_line("cfg1 layer K (or V): 8 heads x 2250 rows + 1 token",
                                             2 * L, device, nbytes, wall)

    # eviction of 250 rows per head, as an audit removes them (sorted absolute rows)
    removed = np.sort(np.concatenate([h * T + rng.choice(T - 32, E, replace=False)
                                      for h in range(H)])).astype(np.int64)
    keep = np.setdiff1d(np.arange(rows), removed)
    removed_d = torch.from_numpy(removed).to(dev)
    keep_d = torch.from_numpy(keep).to(dev)
    kept = keep.size

    # a9 compact, per layer (scoring.cu:294-314)
    device, wall = measure(lambda: [
        (lambda l=l: _C.compact(keys[l], values[l], positions, removed_d))
        for l in range(L)], L)
    nbytes = 2 * kept * d * 2 * 2 + kept * 4 * 2 + removed.size * 8
    out["compact"] = _op_line("cfg1 layer: remove 250 of 2250 rows per head", L, device, nbytes,
                              wall)

    # a12 compact_flattened_kv (cache_legacy.cu:199-242)
    device, wall = measure(lambda: [
        (lambda l=l: _legacy_C.compact_flattened_kv(keys[l], values[l], keep_d))
        for l in range(L)], L)
    nbytes = 2 * kept * d * 2 * 2 + kept * 8
    out["compact_flattened_kv"] = _op_line("cfg1 layer: keep 2000 of 2250 rows per head", L,
                                           device, nbytes, wall)

    # a16 pack: archive the evicted rows of every layer (transport.py:129-177)
    heads_d = torch.from_numpy(removed // T).to(dev)
    payload = torch.empty((removed.size, 2, d), dtype=bf16, device=dev)
    meta = torch.empty((removed.size, 3), dtype=torch.int64, device=dev)
    device, wall = measure(lambda: [
        (lambda l=l: _C.pack(keys[l], values[l], positions, removed_d, heads_d, l,
                             payload, meta)) for l in range(L)], L)
    nbytes = removed.size * (2 * d * 2 * 2 + 4 + 8 + 8 + 3 * 8)
    out["pack"] = _op_line("cfg1 layer: 2000 evicted rows -> [2000, 2, 128] payload", L, device,
                           nbytes, wall)
    del keys, values, positions, payload, meta

    # a14 batch_append, cfg2: 8 requests with per-head lengths U[1500, 2250], one token each
    R = 8
    lengths = [[int(x) for x in rng.integers(1500, 2251, H)] for _ in range(R)]
    totals = [sum(l) for l in lengths]
    req_k = [[randn(n, d) for n in totals] for _ in range(L)]  # every layer its own caches
    req_v = [[randn(n, d) for n in totals] for _ in range(L)]
    req_p = [torch.cat([torch.arange(n, dtype=torch.float32, device=dev) for n in l])[:, None]
             for l in lengths]
    nk, nv = randn(R, H, 1, d), randn(R, H, 1, d)
    logical = [max(l) for l in lengths]
    device, wall = measure(lambda: [
        (lambda l=l: _C.batch_append(req_k[l], req_v[l], req_p, nk, nv, lengths, logical))
        for l in range(L)], L)
    n = sum(totals)
    nbytes = 2 * n * d * 2 + 2 * (n + R * H) * d * 2 + n * 4 + (n + R * H) * 4 + 2 * R * H * d * 2
    out["batch_append"] = _op_line(
        f"cfg2 layer: 8 requests x 8 heads, {n} rows (U[1500,2250] per head) + 1 token each",
        L, device, nbytes, wall)
    del req_k, req_v, req_p

    # packed decode attention (attention.py:15-35, batch_attention.py:92-97): one query token
    # per request and query head (G = 4) over every layer's packed K/V. Each of the 32 layers has
    # its own K/V buffers, as in a decode step, so no layer's rows are cached from the last call.
    from types import SimpleNamespace

    from code_for_iclr27_amd.attention import packed_attention
    for label, requests, head_lengths in (
            ("cfg2 layer: 8 requests x 8 KV heads x G4, U[1500,2250] keys per head", R,
             [h for l in lengths for h in l]),
            ("cfg1 layer: 1 request x 8 KV heads x G4, 2250 keys per head", 1, [T] * H)):
        total = sum(head_lengths)
        layer_k = [randn(total, d) for _ in range(L)]
        layer_v = [randn(total, d) for _ in range(L)]
        queries = randn(requests, H * 4, 1, d)
        meta = SimpleNamespace(
            cu_seqlens_k=torch.tensor([0] + list(np.cumsum(head_lengths)), dtype=torch.int32,
                                      device=dev),
            max_seqlen_k=max(head_lengths),
            decoding_cu_seqlens_q=torch.arange(requests * H + 1, dtype=torch.int32, device=dev))
        device, wall = measure(lambda: [
            (lambda l=l: packed_attention(queries, layer_k[l], layer_v[l], meta, 1, H))
            for l in range(L)], L)
        nbytes = 2 * total * d * 2 + 2 * requests * H * 4 * d * 2 + (requests * H + 1) * 4
        out["packed_attention_" + label[:4]] = _op_line(label, L, device, nbytes, wall)
        del layer_k, layer_v

    # one cfg1 decode step's appends and attention over 32 layers, as the reference runs it
    # (per layer: _C.append, then attention over the appended cache; cache.py:33-52 then
    # attention.py:15-35) and with the appends deferred (per layer: attention with the step's
    # token pending; then one _C.append_layers for every layer)
    step_k = [randn(rows, d) for _ in range(L)]
    step_v = [randn(rows, d) for _ in range(L)]
    step_q = randn(1, H * 4, 1, d)
    step_pos = torch.arange(T, dtype=torch.float32, device=dev).repeat(H)[:, None].contiguous()
    step_cu = torch.arange(0, rows + 1, T, dtype=torch.int32, device=dev)
    decode_q = torch.arange(H + 1, dtype=torch.int32, device=dev)
    cached_meta = SimpleNamespace(cu_seqlens_k=step_cu, max_seqlen_k=T, decoding_cu_seqlens_q=decode_q)

    def eager_step():
        for l in range(L):
            k, v, _, cu, _ = _C.append(step_k[l], step_v[l], step_pos, new_k, new_v, step_cu, T, T)
            packed_attention(step_q, k, v, SimpleNamespace(cu_seqlens_k=cu, max_seqlen_k=T + 1,
                                                           decoding_cu_seqlens_q=decode_q), 1, H)

    def deferred_step():
        for l in range(L):
            packed_attention(step_q, step_k[l], step_v[l], cached_meta, 1, H, pending=(new_k, new_v))
        _C.append_layers(step_k, step_v, [step_pos] * L, [new_k] * L, [new_v] * L, [step_cu] * L,
                         [T] * L, T)

    step_bytes = L * (nbytes_append_layer(rows, H, d) + 2 * (rows + H) * d * 2)
    for name, step_fn in (("decode_step_cfg1_append_then_attend", eager_step),
                          ("decode_step_cfg1_deferred_appends", deferred_step)):
        device, wall = measure(lambda: [step_fn for _ in range(4)], 1)
        out[name] = _op_line("cfg1 decode step, 32 layers: appends of one token per head and "
                             "decode attention (G4)", 1, device, step_bytes, wall)
    del step_k, step_v

    # the audit's margin helpers at the Llama-3.1-8B head (vocab 128,256 x hidden 4096, bf16)
    # and its 32 o_proj matrices [4096, 4096] (_core/scoring.py:34-76, scoring.py:228-237)
    from code_for_iclr27_amd import vjp
    vocab, hidden_size = 128256, 4096
    head = SimpleNamespace(weight=randn(vocab, hidden_size) * 0.02, bias=None)
    model = SimpleNamespace(get_output_embeddings=lambda: head)
    final_hidden = torch.randn((1, hidden_size), generator=gen, device=dev)
    logits = vjp.last_token_logits_float32(model, final_hidden)
    target = int(logits.argmax().item())
    head_bytes = vocab * hidden_size * 2
    for name, call, nbytes in (
            ("head_logits", lambda: vjp.last_token_logits_float32(model, final_hidden),
             head_bytes + vocab * 4 + hidden_size * 4),
            ("hidden_gradient", lambda: vjp.one_vs_rest_hidden_gradient(model, logits, target),
             head_bytes + 3 * vocab * 4 + hidden_size * 4)):
        device, wall = measure(lambda: [call for _ in range(8)], 1)
        out[name] = _op_line(f"Llama-3.1-8B head: {vocab} x {hidden_size} bf16, 1 row", 1,
                             device, nbytes, wall)
    o_weights = [randn(hidden_size, hidden_size) * 0.02 for _ in range(L)]
    posts = [torch.randn(hidden_size, generator=gen, device=dev) for _ in range(L)]
    device, wall = measure(lambda: [
        (lambda l=l: vjp.pre_gradient(posts[l], o_weights[l], 32, 128)) for l in range(L)], L)
    out["pre_gradient"] = _op_line("Llama-3.1-8B layer: post @ o_proj [4096, 4096] bf16", L,
                                   device, hidden_size * hidden_size * 2 + 3 * hidden_size * 4,
                                   wall)
    device, wall = measure(lambda: [
        (lambda: vjp.pre_gradients(posts, o_weights, 32, 128)) for _ in range(4)], 1)
    out["pre_gradients_all_layers"] = _op_line(
        "Llama-3.1-8B: all 32 layers' post @ o_proj in one launch pair", 1, device,
        L * (hidden_size * hidden_size * 2 + 3 * hidden_size * 4) + L * 32, wall)
    del head, logits, o_weights

    # recall archive (cpu_worker.py:17-134, host C++): exact-MIPS search of one query per
    # (layer, KV head) over 4096 archived keys per head, cfg1 shape, on the host's cores
    from code_for_iclr27_amd.archive import ArchiveIndex
    threads = len(os.sched_getaffinity(0))
    rows_per_head = 4096
    archive = ArchiveIndex(L, H, d, threads, 32768)
    bits = torch.randn((L * H * rows_per_head, 2, d), generator=torch.Generator().manual_seed(seed))
    bits = bits.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ids = np.arange(L * H * rows_per_head)
    meta = np.stack([ids // (H * rows_per_head), (ids // rows_per_head) % H, ids % rows_per_head],
                    axis=1).astype(np.int64)
    started = time.perf_counter()
    archive.add(meta, bits)
    add_ms = (time.perf_counter() - started) * 1e3
    queries_host = np.random.default_rng(seed).standard_normal((L * H, d)).astype(np.float32)
    archive.search(queries_host, 4)
    times = []
    for _ in range(reps):
        started = time.perf_counter()
        archive.search(queries_host, 4)
        times.append((time.perf_counter() - started) * 1e3)
    search_ms = float(np.median(times))
    scanned = L * H * rows_per_head * d * 4
    out["archive_search"] = {
        "workload": f"cfg1: 32 layers x 8 KV heads, {rows_per_head} archived rows per head, d128, "
                    "top-4 per head", "threads": threads, "search_ms": round(search_ms, 3),
        "keys_GBps": round(scanned / (search_ms / 1e3) / 1e9, 1),
        "add_ms": round(add_ms, 1), "rows": int(L * H * rows_per_head)}
    del archive, bits

    # recall transport round trip (transport.py:129-307): one eviction batch of 2048 rows
    # (evict_interval 8 x 32 layers x 8 heads) packed, copied out and archived, then one search
    # of 256 group-mean queries, its 1024 results back in HBM
    from code_for_iclr27_amd.transport import RecallTransport
    cache = SimpleNamespace(
        key_cache=[randn(rows, d) for _ in range(L)], value_cache=[randn(rows, d) for _ in range(L)],
        position_cache=[torch.arange(rows, dtype=torch.float32, device=dev)[:, None]] * L,
        metadata_list=[SimpleNamespace(head_lens_cpu=[T] * H)] * L)
    blocks = [SimpleNamespace(self_attn=SimpleNamespace(_last_query_states=randn(1, 4 * H, 1, d)))
              for _ in range(L)]
    model = SimpleNamespace(model=SimpleNamespace(layers=blocks))
    transport = RecallTransport(L, H, 4 * H, d, search_interval=1, topk=4, archive_buffers=4,
                                cpu_threads=threads)
    archive_ms, search_ms = [], []
    for rep in range(reps):
        removals = {(l, h): list(rng.choice(T, 8, replace=False)) for l in range(L) for h in range(H)}
        torch.cuda.synchronize()
        started = time.perf_counter()
        transport.record_evicted(cache, removals)
        transport.wait_pending()
        archive_ms.append((time.perf_counter() - started) * 1e3)
        started = time.perf_counter()
        transport.step(model, cache, rep + 1)
        transport.wait_pending()
        ready = transport.ready_result()
        search_ms.append((time.perf_counter() - started) * 1e3)
        transport.release_result(ready[0])
    transport.finish()
    out["recall_transport"] = {
        "workload": "cfg1: 2048 evicted rows per batch archived; 256 queries, top-4 per head",
        "archive_batch_ms": round(float(np.median(archive_ms)), 3),
        "search_round_trip_ms": round(float(np.median(search_ms)), 3),
        "indexed": transport.counters["indexed_vectors"], "cpu_threads": threads}
    transport.close()
    del cache, blocks, transport

    # query history (history.py:21-38,51-63): one decode step's queries of all 32 layers
    # (Hq 32, d128, bf16) into the device ring, one launch per step
    from code_for_iclr27_amd.history import QueryHistory
    Hq, W = 32, 250
    history = QueryHistory(L, W)
    step_queries = [[randn(1, Hq, 1, d) for _ in range(L)] for _ in range(2)]
    clock = iter(range(1 << 40))
    device, wall = measure(lambda: [
        (lambda i=i: history.append(step_queries[i % 2], next(clock))) for i in range(2 * W)], 1)
    nbytes = 3 * L * Hq * d * 2 + 2 * 8
    out["history_append"] = _op_line("cfg1 decode step: 32 layers x 32 query heads x d128 into "
                                     "the [32, 32, 500, 128] ring", 1, device, nbytes, wall)
    # the audit's window: ring views here, versus the reference's per-layer torch.cat of W
    # [1, Hq, 1, d] tensors plus a torch.tensor of the positions (history.py:51-63)
    from collections import deque
    deques = [deque((randn(1, Hq, 1, d) for _ in range(W)), maxlen=W) for _ in range(L)]
    walls = {}
    for name, gather in (
            ("ring_views", lambda: history.audit_window()),
            ("deque_cat", lambda: ([torch.cat(list(q), dim=2) for q in deques],
                                   torch.tensor(list(range(W)), dtype=torch.long, device=dev)))):
        gather()
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            started = time.perf_counter()
            gather()
            torch.cuda.synchronize()
            times.append((time.perf_counter() - started) * 1e3)
        walls[name] = round(float(np.median(times)), 3)
    out["history_append"]["audit_window_ms"] = walls
    del history, step_queries, deques
    torch.cuda.empty_cache()
    return out


def copy_probe(torch, gib=4, reps=5):
    """What a plain device-to-device copy reaches on this part at a size far beyond the 256 MB
    Infinity Cache, next to the 8 TB/s peak: torch's copy_ (the HIP runtime's copy kernel), and
    the library's calibration copy lr_stream_copy (the nontemporal 16-byte loads and stores of
    the all-layer row kernels), the practical ceiling of the read+write row kernels."""
    import numpy as np

    from code_for_iclr27_amd import _lib

    source = torch.empty((gib << 29,), dtype=torch.bfloat16, device="cuda")
    source.fill_(1.0)
    target = torch.empty_like(source)
    nbytes = 2 * source.numel() * 2
    stream = torch.cuda.current_stream().cuda_stream

    def timed(copy):
        times = []
        for _ in range(reps + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            copy()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        ms = float(np.median(times[1:]))
        return {"ms": round(ms, 3), "GBps": round(nbytes / (ms / 1e3) / 1e9, 1),
                "hbm_fraction": round(nbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4)}

    runtime = timed(lambda: target.copy_(source))
    target.zero_()
    streamed = timed(lambda: _lib.call("lr_stream_copy", source.data_ptr(), target.data_ptr(),
                                       nbytes // 2, stream))
    if not torch.equal(target, source):
        raise RuntimeError("stream copy probe: the copy differs from its source")
    del source, target
    torch.cuda.empty_cache()
    return {"bytes_read_plus_written": nbytes, **runtime, "stream_copy": streamed}


def lazy_window_bench(torch, layers, qpos, margin, cfg, reps=5):
    """The controller's steady state between two audits (controller.py:57-70,122-159) at cfg1:
    an audit selecting 250 slots per (layer, head) that removes 2 per head now and queues the
    rest on the device, then the 31 evict_prefix batches of evict_interval 8 x L x H slots that
    drain the queue (each one plan launch and one compaction of every layer). Host-inclusive
    time of the whole window; the batches' device time from events around them."""
    import numpy as np

    from code_for_iclr27_amd import audit

    slots = cfg.layers * cfg.heads
    immediate, batch, batches = 2 * slots, 8 * slots, 31
    assert immediate + batches * batch == cfg.count
    step = audit.AuditStep()

    def window(events=None):
        outcome = step.run(layers, qpos, margin, cfg.count, cfg.protect_recent, cfg.pool_kernel,
                           cfg.epsilon, immediate=immediate)
        current = outcome.layers
        if events is not None:
            events[0].record()
        for _ in range(batches):
            current = outcome.queue.evict_prefix(current, batch)
        if events is not None:
            events[1].record()
        return current

    window()
    torch.cuda.synchronize()
    walls, evict_us = [], []
    for _ in range(reps):
        events = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        started = time.perf_counter()
        window(events)
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - started) * 1e3)
        evict_us.append(events[0].elapsed_time(events[1]) * 1e3 / batches)
    rows = sum(layer.keys.size(0) for layer in layers)
    d = cfg.dim
    # each batch's compaction reads and writes every kept row (K, V and its position) once
    kept_after = [rows - immediate - (b + 1) * batch for b in range(batches)]
    evict_bytes = sum(2 * k * d * 2 * 2 + k * 4 * 2 + batch * 8 for k in kept_after) / batches
    us = float(np.median(evict_us))
    return {"workload": f"{cfg.name}: audit selecting {cfg.evict_per_head} per head, "
                        f"{immediate // slots} per head removed at once, then {batches} "
                        f"evict_prefix batches of {batch // slots} per head",
            "window_ms": round(float(np.median(walls)), 3),
            "evict_prefix_device_us": round(us, 1),
            "evict_prefix_bytes": int(evict_bytes),
            "evict_prefix_GBps": round(evict_bytes / (us / 1e6) / 1e9, 1),
            "evict_prefix_hbm_fraction": round(evict_bytes / (us / 1e6) / 1e9 / HBM_PEAK_GBPS, 4)}


def audit_config_bench(torch, name, seed, steps=10, warmup=3):
    """A shorter audit-step measurement of another benchmark configuration (cfg0, cfg4, cfg3)."""
    import numpy as np

    from code_for_iclr27_amd import audit, workloads

    cfg = workloads.CONFIGS[name]
    dev = torch.device("cuda:0")
    layers, qpos, margin = workloads.make_audit(cfg, dev, seed=seed, generator_device="cuda")
    step = audit.AuditStep()

    def run(timer=None):
        return step.run(layers, qpos, margin, cfg.count, cfg.protect_recent, cfg.pool_kernel,
                        cfg.epsilon, timer=timer)

    for _ in range(warmup):
        outcome = run()
    torch.cuda.synchronize()
    started = time.perf_counter()
    for _ in range(steps):
        outcome = run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - started) * 1e3 / steps
    timers = [EventTimer(torch) for _ in range(3)]
    for timer in timers:
        run(timer)
    torch.cuda.synchronize()
    stages = {}
    for timer in timers:
        for stage, us in timer.stages().items():
            stages[stage] = stages.get(stage, 0.0) + us / len(timers)
    rows_total = sum(layer.keys.size(0) for layer in layers)
    nbytes = audit_bytes(cfg, rows_total, outcome.removed, int(outcome.scores.numel()),
                         len(outcome.segments))
    line = {"workload": f"{cfg.name}: L{cfg.layers} H{cfg.heads} d{cfg.dim} G{cfg.groups} "
                        f"T{cfg.length} W{cfg.window}, evict {cfg.evict_per_head} per head",
            "ms_per_step": round(ms, 4), "GBps": round(nbytes / (ms / 1e3) / 1e9, 1),
            "hbm_fraction": round(nbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes": nbytes, "evicted": outcome.removed,
            "stages_us": {k: round(v, 1) for k, v in stages.items()}}
    del layers, outcome, step
    torch.cuda.empty_cache()
    return line


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): "
              "this build has no multi-GPU path; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from code_for_iclr27_amd import audit, workloads

    dev = torch.device("cuda:0")
    if args.copy_probe > 0:
        source = torch.ones((args.copy_probe << 18,), dtype=torch.float32, device=dev)
        target = torch.empty_like(source)
        torch.neg(source, out=target)
        torch.cuda.synchronize()
        del source, target
    cfg = workloads.CONFIGS[args.config]
    layers, qpos, margin = workloads.make_audit(cfg, dev, seed=args.seed, generator_device="cuda")
    step = audit.AuditStep()

    def run(timer=None, queue_order=False):
        return step.run(layers, qpos, margin, cfg.count, cfg.protect_recent, cfg.pool_kernel,
                        cfg.epsilon, queue_order=queue_order, timer=timer)

    def average_stages(timers):
        timers = [timer for timer in timers if timer is not None]
        sums = {}
        for timer in timers:
            for name, us in timer.stages().items():
                sums[name] = sums.get(name, 0.0) + us
        return {name: total / len(timers) for name, total in sums.items()}

    def timed(steps, make_timer, queue_order=False, warmup=0):
        """`warmup` untimed steps, then `steps` timed ones between two synchronisations. The
        garbage collector runs before the warm-up steps and is off until the end: a collection
        right before the first timed step leaves the host's caches cold, which made that step's
        host work (0.35-0.55 ms) several times slower than in the following steps."""
        timers = [make_timer(i) for i in range(steps)]
        for timer in timers:  # create the device events before the timed region
            for event in timer.events if timer is not None else ():
                event.record()
        torch.cuda.synchronize()
        gc.collect()
        gc.disable()
        for _ in range(warmup):
            run(None, queue_order)
        torch.cuda.synchronize()
        started = time.perf_counter()
        ends = []
        for timer in timers:
            outcome = run(timer, queue_order)  # returns after the step's device->host copy
            ends.append(time.perf_counter())
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - started
        gc.enable()
        return outcome, timers, elapsed, np.diff([started] + ends) * 1e3

    # stage breakdown (not the timed region): every stage bracketed by events
    _, breakdown, _, _ = timed(max(3, min(args.steps, 10)), lambda i: EventTimer(torch), warmup=3)
    stages = average_stages(breakdown)
    order = list(stages)
    dominant = max(stages, key=stages.get)
    before = "start" if order.index(dominant) == 0 else order[order.index(dominant) - 1]
    # timed region: K steps, events only around the dominant kernel, on every event_every-th
    # step (the kernel's average launch time comes from those steps)
    every = max(1, args.event_every)
    outcome, timers, elapsed, step_ms = timed(
        args.steps, lambda i: EventTimer(torch, only={before, dominant}) if i % every == 0 else None,
        warmup=args.warmup)
    ms_per_step = elapsed * 1e3 / args.steps
    dominant_us = average_stages(timers)[dominant]
    # the same step with the eviction-queue order computed too (it is empty here: every
    # selected slot is removed at once, so the removal sets do not depend on it), timed like
    # the headline (in 20 steps after 3 warm-up ones the first step's exposed host planning
    # added ~40 us a step)
    queue_steps = args.steps
    _, _, queue_elapsed, _ = timed(queue_steps, lambda i: None, True, warmup=args.warmup)
    rows_total = sum(layer.keys.size(0) for layer in layers)
    candidates = int(outcome.scores.numel())
    segments = len(outcome.segments)
    nbytes = audit_bytes(cfg, rows_total, outcome.removed, candidates, segments)
    value = nbytes / (ms_per_step / 1e3) / 1e9

    # dominant kernel roofline, from the timed steps' events
    W, G, d = cfg.window, cfg.groups, cfg.dim
    if dominant in ("column_scores", "row_stats"):
        keys = candidates if dominant == "column_scores" else rows_total
        flops = 2.0 * W * G * d * keys
        achieved = flops / (dominant_us / 1e6) / 1e12
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 1),
                    "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                    "traffic": measured_traffic(dominant, cfg.name), "algorithmic_flops": flops}
        # the kernel's real limit is VALU issue: its VALU-active time per SIMD (counted
        # instructions, committed profile) against this run's measured kernel time
        cycles = measured_valu_cycles(dominant, cfg.name)
        if cycles is not None:
            issue_us = cycles / SIMDS / (ENGINE_CLOCK_GHZ * 1e3)
            roofline["valu"] = {"issue_us_per_simd": round(issue_us, 1),
                                "kernel_us": round(dominant_us, 1),
                                "frac": round(issue_us / dominant_us, 4),
                                "source": "profiles/scorer_cfg1_sq_counters.md"}
    else:
        stage_bytes = {"compact": 2 * (rows_total - outcome.removed) * d * 2 * 2,
                       "projected_values": rows_total * d * 2}.get(dominant, nbytes)
        achieved = stage_bytes / (dominant_us / 1e6) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                    "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBPS, 4),
                    "traffic": measured_traffic(dominant, cfg.name)}

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{cfg.name}: audit step score->pool7->select->compact",
                   "layers": cfg.layers, "kv_heads": cfg.heads, "head_dim": d, "groups": G,
                   "tokens_per_head": cfg.length, "window": W, "evicted": outcome.removed,
                   "candidates": candidates, "batch": 1, "parallelism": "single GPU"},
        "hbm_fraction": round(value / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes": nbytes,
        "stages_us": {k: round(v, 1) for k, v in stages.items()},
        "dominant_kernel_us": round(dominant_us, 1),
        "dominant_kernel_samples": sum(timer is not None for timer in timers),
        "queue_order_ms_per_step": round(queue_elapsed * 1e3 / queue_steps, 4),
        "step_ms_min_median_max": [round(float(np.min(step_ms)), 3), round(float(np.median(step_ms)), 3),
                                   round(float(np.max(step_ms)), 3)],
        "roofline": roofline,
    }

    del outcome
    torch.cuda.empty_cache()
    line["hbm_copy_probe"] = copy_probe(torch)
    if args.config == "cfg1" and not args.no_lazy:
        line["lazy_window"] = lazy_window_bench(torch, layers, qpos, margin, cfg)
        torch.cuda.empty_cache()
    if not args.no_reinsert:
        line["reinsert"] = reinsert_bench(torch, args.seed)
        torch.cuda.empty_cache()
    if not args.no_ops:
        line["ops"] = ops_bench(torch, args.seed)
    others = [name for name in args.other_configs.split(",") if name and name != args.config]
    if others:
        line["audit_configs"] = {name: audit_config_bench(torch, name, args.seed)
                                 for name in others}

    if not args.no_cpu:
        n, seconds, scaled, threads, times = cpu_baseline(torch, layers, qpos, margin, cfg,
                                                          args.cpu_seconds)
        line["cpu_baseline"] = {
            "value": round(nbytes / scaled / 1e9, 4), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"{cfg.name}: full audit step over the first {n} of {cfg.layers} layers "
                       f"({n * cfg.heads} heads), one warm-up run then the median of "
                       f"{len(times)} runs, {seconds:.2f} s on the host, scaled by "
                       f"{cfg.layers}/{n} to {scaled:.2f} s per audit step"),
            "run_seconds": times,
            "cpu_model": _cpu_model(),
        }
    print(json.dumps(line), flush=True)


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it, with its family / model / stepping and the
    logical CPUs this process may use out of those listed."""
    fields, listed = {}, 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, value = line.partition(":")
                key = key.strip()
                if key == "processor":
                    listed += 1
                elif key in ("model name", "cpu family", "model", "stepping", "cpu MHz"):
                    fields.setdefault(key, value.strip())
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    detail = ", ".join(f"{key} {fields[key]}" for key in ("cpu family", "model", "stepping",
                                                          "cpu MHz") if key in fields)
    usable = len(os.sched_getaffinity(0))
    return f"{name} ({detail}; {usable} of {listed} logical CPUs usable)"


if __name__ == "__main__":
    main()
