"""The budget-driven lazy eviction queue on the device (src/lazy_recall/controller.py:57-70,
140-159): an audit that removes only the first `immediate` selected slots and keeps the rest
queued, then evict_prefix batches (with decode appends in between), bit-exact at every step
against the oracle chain: refine_arrays on the GPU's scores, ArrayReferences groups, the
controller's searchsorted(removed_at_audit) remap (oracle.selection.evict_prefix_remap) and
kv_ops.compact / kv_ops.append on a numpy copy of the cache."""

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _C, audit, workloads
from code_for_iclr27_amd.scoring import LayerState
from code_for_iclr27_amd.selection import ArrayReferences
from oracle import kv_ops
from oracle import selection as oselection

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


class OracleCache:
    """A numpy copy of the cache, changed only by the oracle's operations."""

    def __init__(self, layers):
        self.keys = [bits(layer.keys) for layer in layers]
        self.values = [bits(layer.values) for layer in layers]
        self.positions = [layer.positions.cpu().numpy().reshape(-1) for layer in layers]
        self.lens = [list(layer.head_lens) for layer in layers]

    def remove(self, removals):
        """remove_positions (cache.py:92-180): {(layer, head): positions within the head}."""
        for l in range(len(self.keys)):
            starts = np.concatenate(([0], np.cumsum(self.lens[l])))
            rows = [starts[h] + np.asarray(removals[(l, h)], np.int64)
                    for h in range(len(self.lens[l])) if (l, h) in removals]
            if not rows:
                continue
            rows = np.sort(np.concatenate(rows)).astype(np.int64)
            self.keys[l], self.values[l], p = kv_ops.compact(self.keys[l], self.values[l],
                                                             self.positions[l], rows)
            self.positions[l] = p.reshape(-1)
            for h in range(len(self.lens[l])):
                self.lens[l][h] -= len(removals.get((l, h), ()))

    def append(self, l, new_keys, new_values, logical):
        cumulative = np.concatenate(([0], np.cumsum(self.lens[l])))
        k, v, p, _, lengths = kv_ops.append(self.keys[l], self.values[l], self.positions[l],
                                            new_keys, new_values, cumulative, logical,
                                            max(self.lens[l]))
        self.keys[l], self.values[l], self.positions[l] = k, v, p.reshape(-1)
        self.lens[l] = [int(n) for n in lengths]

    def check(self, layers, head_lens):
        assert [list(x) for x in head_lens] == self.lens
        for l, layer in enumerate(layers):
            np.testing.assert_array_equal(bits(layer.keys), self.keys[l])
            np.testing.assert_array_equal(bits(layer.values), self.values[l])
            np.testing.assert_array_equal(layer.positions.cpu().numpy().reshape(-1),
                                          self.positions[l])


def oracle_queue(outcome, count, pool_kernel=7):
    raw = outcome.scores.cpu().numpy()
    ends = np.asarray(outcome.cumulative_ends)
    pooled = kv_ops.pool(raw, np.concatenate(([0], ends)), pool_kernel)
    starts = [s.position_start for s in outcome.segments]
    selection = oselection.refine_arrays(raw, pooled, ends, starts, count)
    coordinates = [(s.layer, s.head) for s in outcome.segments]
    return ArrayReferences(selection.values, selection.segments, selection.positions, coordinates)


def evict_prefix(queue, removed_at_audit, count):
    """controller.py:57-70 on the oracle's host queue (returns removals and the new queue)."""
    removals = {}
    for segment, positions in queue[:count].groups().items():
        removed = removed_at_audit.get(segment, np.empty(0, np.int64))
        removals[segment], removed_at_audit[segment] = oselection.evict_prefix_remap(positions,
                                                                                     removed)
    return removals, queue[count:]


def append_token(device, layers, oracle, step, gen):
    """One decode token per KV head in every layer, GPU (_C.append) and oracle alike."""
    out = []
    for l, layer in enumerate(layers):
        heads = len(layer.head_lens)
        dim = layer.keys.shape[1]
        nk = torch.randn((1, heads, 1, dim), generator=gen).to(torch.bfloat16)
        nv = torch.randn((1, heads, 1, dim), generator=gen).to(torch.bfloat16)
        cumulative = torch.tensor(np.concatenate(([0], np.cumsum(layer.head_lens))),
                                  dtype=torch.int32, device=device)
        logical = 5000 + step
        k, v, p, _, lengths = _C.append(layer.keys, layer.values, layer.positions,
                                        nk.to(device), nv.to(device), cumulative, logical,
                                        max(layer.head_lens))
        oracle.append(l, bits(nk), bits(nv), logical)
        out.append(LayerState(k, v, p.reshape(-1), lengths.cpu().tolist(), layer.prompt_lens,
                              layer.queries, layer.gradient))
    return out


@pytest.mark.parametrize("native", [True, False])
@pytest.mark.parametrize("immediate_fraction", [0.0, 0.3])
def test_lazy_audit_then_evict_prefix_batches(device, native, immediate_fraction):
    head_lengths = [[300, 41, 280, 120], [170, 300, 33, 299], [64, 200, 310, 90]]
    prompts = [[0, 0, 5, 0], [12, 0, 0, 0], [0, 3, 0, 0]]
    layers, qpos = workloads.make_layers(head_lengths, 4, 128, 40, device, seed=21,
                                         prompt_lengths=prompts)
    margin = torch.tensor([2.0], device=device)
    oracle = OracleCache(layers)
    step = audit.AuditStep()
    count = 900
    immediate = int(immediate_fraction * count)
    outcome = step.run(layers, qpos, margin, count, native=native, immediate=immediate)
    queue = oracle_queue(outcome, count)
    got_queue = outcome.selection.references()
    np.testing.assert_array_equal(got_queue.scores, queue.scores)
    np.testing.assert_array_equal(got_queue.segments, queue.segments)
    np.testing.assert_array_equal(got_queue.positions, queue.positions)
    removed_at_audit = {key: np.asarray(v, np.int64) for key, v in queue[:immediate].groups().items()}
    oracle.remove(removed_at_audit)
    queue = queue[immediate:]
    oracle.check(outcome.layers, outcome.head_lens)
    lazy = outcome.queue
    assert lazy is not None and len(lazy) == count - immediate
    remaining = lazy.references()
    np.testing.assert_array_equal(remaining.positions, queue.positions)
    np.testing.assert_array_equal(remaining.segments, queue.segments)

    gen = torch.Generator().manual_seed(5)
    current = list(outcome.layers)
    batches = [37, 1, 250, len(queue) - 288]  # the last one drains the queue
    for index, size in enumerate(batches):
        current = append_token(device, current, oracle, index, gen)
        removals, queue = evict_prefix(queue, removed_at_audit, size)
        oracle.remove(removals)
        current = lazy.evict_prefix(current, size)
        oracle.check(current, current.kept)
        assert len(lazy) == len(queue)
    assert len(lazy) == 0
    with pytest.raises(RuntimeError, match="Discard queue underflow"):
        lazy.evict_prefix(current, 1)
    assert lazy.evict_prefix(current, 0) is current


def test_lazy_audit_refuses_short_selection(device):
    layers, qpos = workloads.make_layers([[100, 90]], 4, 64, 20, device, seed=3)
    margin = torch.tensor([2.0], device=device)
    total = (100 - 32) + (90 - 32)
    with pytest.raises(RuntimeError, match="Not enough unprotected candidates"):
        audit.AuditStep().run(layers, qpos, margin, total + 50, immediate=total + 10)


def test_lazy_window_full_size(device):
    """cfg1 at full size, as the controller's steady state: an audit selecting 250 slots per
    head that removes 2 per head now and queues the rest, then 31 evict_prefix batches of 8 per
    head (evict_interval 8) drain it. Sampled layers bit-exact at the end, every head length
    exact after every batch."""
    cfg = workloads.CONFIGS["cfg1"]
    slots = cfg.layers * cfg.heads
    layers, qpos, margin = workloads.make_audit(cfg, device, seed=17, generator_device="cuda")
    oracle = OracleCache(layers)
    outcome = audit.AuditStep().run(layers, qpos, margin, cfg.count, cfg.protect_recent,
                                    cfg.pool_kernel, cfg.epsilon, immediate=2 * slots)
    queue = oracle_queue(outcome, cfg.count)
    removed_at_audit = {key: np.asarray(v, np.int64)
                        for key, v in queue[:2 * slots].groups().items()}
    queue = queue[2 * slots:]
    lens = [list(l.head_lens) for l in layers]
    for (l, h), positions in removed_at_audit.items():
        lens[l][h] -= len(positions)
    assert [list(x) for x in outcome.head_lens] == lens
    current = outcome.layers
    for batch in range(31):
        removals, queue = evict_prefix(queue, removed_at_audit, 8 * slots)
        for (l, h), positions in removals.items():
            lens[l][h] -= len(positions)
        current = outcome.queue.evict_prefix(current, 8 * slots)
        assert [list(x) for x in current.kept] == lens, batch
    assert len(outcome.queue) == 0 and len(queue) == 0
    # the end state: each head lost exactly its 250 audit-time picks
    oracle.remove({key: np.asarray(v, np.int64) for key, v in removed_at_audit.items()})
    for l in sorted({0, 15, 31}):
        np.testing.assert_array_equal(bits(current[l].keys), oracle.keys[l])
        np.testing.assert_array_equal(bits(current[l].values), oracle.values[l])
        np.testing.assert_array_equal(current[l].positions.cpu().numpy().reshape(-1),
                                      oracle.positions[l])


def staged_rows(oracle, removals):
    """What record_evicted archives for `removals` of the oracle's current cache: (layer, head,
    int64 position) and the K, V rows, in (layer, head, position) order (transport.py:141-167)."""
    meta, payload = [], []
    for l, h in sorted(removals):
        starts = np.concatenate(([0], np.cumsum(oracle.lens[l])))
        for position in sorted(int(p) for p in removals[(l, h)]):
            row = starts[h] + position
            meta.append((l, h, int(oracle.positions[l][row])))
            payload.append(np.stack([oracle.keys[l][row], oracle.values[l][row]]))
    return np.asarray(meta, np.int64).reshape(-1, 3), np.asarray(payload, np.int16)


def check_staged(transport, meta, payload, archived_before):
    """The batch the transport just committed (one archive slot: slot 0), bit-exact."""
    transport.wait_pending()
    n = len(meta)
    assert transport.counters["archived_vectors"] == archived_before + n
    assert transport.counters["indexed_vectors"] == archived_before + n
    np.testing.assert_array_equal(transport.archive_meta_gpu[0][:n].cpu().numpy(), meta)
    np.testing.assert_array_equal(transport.archive_gpu[0][:n].view(torch.int16).cpu().numpy(),
                                  payload)
    return archived_before + n


@pytest.mark.parametrize("immediate", [None, 150])
def test_fused_removals_feed_the_recall_archive(device, immediate):
    """With a RecallTransport attached, the audit's removals (all of them, or the lazy form's
    first `immediate`) and every evict_prefix batch are packed for the archive before their
    compaction, as remove_positions archives its removals first (cache.py:110-112): each
    batch's staged payload and metadata bit-exact against the rows the oracle removes, and the
    worker indexes every one."""
    from code_for_iclr27_amd.transport import RecallTransport

    head_lengths = [[300, 41, 280, 120], [170, 300, 33, 299], [64, 200, 310, 90]]
    layers, qpos = workloads.make_layers(head_lengths, 4, 128, 40, device, seed=21)
    margin = torch.tensor([2.0], device=device)
    transport = RecallTransport(3, 4, 16, 128, topk=2, archive_buffers=1, cpu_threads=2,
                                evict_interval=16, timeout_seconds=30.0)  # 192 rows per batch
    oracle = OracleCache(layers)
    count = 180 if immediate is None else 900
    outcome = audit.AuditStep().run(layers, qpos, margin, count, immediate=immediate,
                                    transport=transport)
    queue = oracle_queue(outcome, count)
    now = count if immediate is None else immediate
    removed_at_audit = {key: np.asarray(v, np.int64) for key, v in queue[:now].groups().items()}
    archived = check_staged(transport, *staged_rows(oracle, removed_at_audit), 0)
    oracle.remove(removed_at_audit)
    oracle.check(outcome.layers, outcome.head_lens)
    if immediate is not None:
        queue = queue[immediate:]
        current = outcome.layers
        for size in (37, 1, 192):
            removals, queue = evict_prefix(queue, removed_at_audit, size)
            expected = staged_rows(oracle, removals)
            current = outcome.queue.evict_prefix(current, size, transport=transport)
            archived = check_staged(transport, *expected, archived)
            oracle.remove(removals)
            oracle.check(current, current.kept)
        with pytest.raises(RuntimeError, match="exceeds configured archive staging capacity"):
            outcome.queue.evict_prefix(current, 193, transport=transport)
        assert transport.counters["archive_overflows"] == 1
        current = outcome.queue.evict_prefix(current, 100)  # a batch without the archive
        assert transport.counters["archived_vectors"] == archived
    transport.close()
