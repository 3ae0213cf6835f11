"""The recall transport (code_for_iclr27_amd.transport.RecallTransport) end to end on the GPU:
evicted rows packed by the HIP pack kernel into a pinned staging slot, copied to the host on
the side stream, archived by the C++ archive on the worker thread; a search every
search_interval steps over per-(layer, head) group-mean queries; results copied back to HBM.
Archived payloads, search results (order included) and metadata are compared bit-exactly with
the oracle archive (oracle/archive.py) fed the same rows and the same host queries; the slot
state machine's counters and states are checked along the way."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from code_for_iclr27_amd.transport import RecallTransport
from oracle import archive as oarchive

pytestmark = pytest.mark.gpu


def make_cache(device, layers, heads, dim, lengths, seed):
    g = torch.Generator().manual_seed(seed)
    cache = SimpleNamespace(key_cache=[], value_cache=[], position_cache=[], metadata_list=[])
    for _ in range(layers):
        rows = sum(lengths)
        cache.key_cache.append(torch.randn((rows, dim), generator=g).bfloat16().to(device))
        cache.value_cache.append(torch.randn((rows, dim), generator=g).bfloat16().to(device))
        positions = torch.cat([torch.arange(n, dtype=torch.float32) * 3 + 7 for n in lengths])
        cache.position_cache.append(positions[:, None].to(device))
        cache.metadata_list.append(SimpleNamespace(head_lens_cpu=list(lengths)))
    return cache


def test_archive_search_and_return(device):
    layers, heads, groups, dim = 2, 2, 4, 128
    lengths = [300, 250]
    cache = make_cache(device, layers, heads, dim, lengths, seed=1)
    transport = RecallTransport(layers, heads, heads * groups, dim, search_interval=4, topk=3,
                                archive_buffers=2, cpu_threads=2, evict_interval=64,
                                timeout_seconds=30.0)
    rng = np.random.default_rng(2)
    removals = {(l, h): list(rng.choice(lengths[h], 40, replace=False))
                for l in range(layers) for h in range(heads)}
    transport.record_evicted(cache, removals)
    transport.wait_pending()
    assert transport.counters["archived_vectors"] == 160
    assert transport.counters["indexed_vectors"] == 160
    assert transport.archive_states == ["free", "free"]

    # the oracle archive fed the same rows (what pack gathers: K, V bits and int64 positions)
    reference = oarchive.ArchiveIndex(layers, heads, dim, 32768)
    metadata, payload = [], []
    for layer in range(layers):
        bounds = np.concatenate(([0], np.cumsum(lengths)))
        k = cache.key_cache[layer].view(torch.int16).cpu().numpy().view(np.uint16)
        v = cache.value_cache[layer].view(torch.int16).cpu().numpy().view(np.uint16)
        p = cache.position_cache[layer].cpu().numpy().reshape(-1)
        for head in range(heads):
            for position in sorted(set(int(x) for x in removals[(layer, head)])):
                row = bounds[head] + position
                metadata.append((layer, head, int(p[row])))
                payload.append(np.stack([k[row], v[row]]))
    reference.add(np.asarray(metadata, np.int64), np.asarray(payload, np.uint16))

    # decode queries: group members near an archived key of their KV head
    g = torch.Generator().manual_seed(3)
    model_layers = []
    for layer in range(layers):
        q = torch.randn((1, heads * groups, 1, dim), generator=g) * 0.1
        for head in range(heads):
            row = np.concatenate(([0], np.cumsum(lengths)))[head] + int(removals[(layer, head)][0])
            q[0, head * groups:(head + 1) * groups, 0] += cache.key_cache[layer][row].float().cpu()
        model_layers.append(SimpleNamespace(self_attn=SimpleNamespace(
            _last_query_states=q.bfloat16().to(device))))
    model = SimpleNamespace(model=SimpleNamespace(layers=model_layers))
    for step in range(1, 4):
        transport.step(model, cache, step)  # not a search step
    assert transport.counters["submitted_queries"] == 0
    transport.step(model, cache, 4)
    assert transport.counters["submitted_queries"] == 1
    transport.wait_pending()
    ready = transport.ready_result()
    assert ready is not None
    slot, step, payload_gpu, meta_gpu, meta_host = ready
    assert step == 4 and transport.counters["searches_completed"] == 1
    queries = transport.host["queries"][slot].numpy().copy()
    expect_meta, expect_payload = reference.search(queries, 3)
    np.testing.assert_array_equal(meta_host, expect_meta)
    np.testing.assert_array_equal(meta_gpu.cpu().numpy(), expect_meta)
    np.testing.assert_array_equal(payload_gpu.view(torch.int16).cpu().numpy().view(np.uint16),
                                  expect_payload)
    assert len(expect_meta) == layers * heads * 3
    transport.release_result(slot)
    torch.cuda.synchronize()
    transport.retire_finished()
    assert transport.query_states == ["free", "free"]

    # admitted rows leave the archive; a flush round-trips through the worker
    transport.remove_admitted(expect_meta[:2])
    transport.finish()
    assert transport.counters["indexed_vectors"] == 158
    stats = transport.stats
    assert stats["d2h_bytes"] > 0 and stats["h2d_bytes"] == len(expect_meta) * (2 * dim * 2 + 24)
    transport.close()
    assert transport.closed and not transport.thread.is_alive()


def test_overflow_and_bad_configuration(device):
    with pytest.raises(ValueError, match="Invalid recall configuration"):
        RecallTransport(2, 3, 8, 64)
    cache = make_cache(device, 1, 1, 64, [100], seed=4)
    transport = RecallTransport(1, 1, 2, 64, topk=2, archive_buffers=1, evict_interval=4)
    with pytest.raises(RuntimeError, match="exceeds configured archive staging capacity"):
        transport.record_evicted(cache, {(0, 0): list(range(5))})
    assert transport.counters["archive_overflows"] == 1
    transport.close()
