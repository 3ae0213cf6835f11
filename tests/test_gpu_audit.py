"""GPU parity of selection (refine_arrays) and of the whole audit step.

Selection is compared bit-exactly with the oracle's canonical-tie refine_arrays on the same
score tables (ties at a cut go to the lower index); on tie-free tables it must also equal the
reference's CPU torch.topk path exactly. The audit step's compacted caches are bit-exact
against the oracle chain (pool -> refine -> per-layer compaction) fed the GPU scores, which
the scorer tests validate separately.
"""

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _lib, audit, scoring, selection, workloads
from oracle import kv_ops
from oracle import selection as oselection

pytestmark = pytest.mark.gpu


def run_select(device, raw, pooled, ends, starts, count):
    coords = [(i // 4, i % 4) for i in range(len(ends))]
    result = selection.select_refine(torch.from_numpy(raw).to(device),
                                     torch.from_numpy(pooled).to(device), list(ends),
                                     list(starts), coords, count)
    torch.cuda.synchronize()
    return result


def compare(result, expect, ends):
    np.testing.assert_array_equal(result.values.cpu().numpy(), expect.values)
    np.testing.assert_array_equal(result.segments.cpu().numpy(), expect.segments)
    np.testing.assert_array_equal(result.positions.cpu().numpy(), expect.positions)
    np.testing.assert_array_equal(result.quotas.cpu().numpy(), expect.quotas)
    offsets = result.offsets.cpu().numpy()
    removed = result.removed_positions.cpu().numpy()
    for s in range(len(ends)):
        got = removed[offsets[s]:offsets[s + 1]]
        np.testing.assert_array_equal(got, np.sort(expect.positions[expect.segments == s]))
    assert result.change_counts() == (expect.changed, expect.changed_heads)


def tables(rng, lengths, ties=False):
    ends = np.cumsum(lengths)
    raw = rng.random(ends[-1]).astype(np.float32) * 1e-3
    if ties:
        raw = np.round(raw * 2000).astype(np.float32) / 2000  # many equal values
    pooled = np.empty_like(raw)
    start = 0
    for end in ends:
        pooled[start:end] = kv_ops.pool(raw[start:end], [0, end - start], 7)
        start = end
    return raw, pooled, ends


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("fraction", [0.001, 0.11, 0.5, 1.0])
def test_select_matches_oracle(device, ties, fraction):
    rng = np.random.default_rng(int(fraction * 1000) + ties)
    lengths = [2218] * 12 + [1, 7, 300, 5000]
    raw, pooled, ends = tables(rng, lengths, ties)
    starts = rng.integers(0, 40, len(lengths))
    count = max(1, int(fraction * raw.size))
    result = run_select(device, raw, pooled, ends, starts, count)
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    compare(result, expect, ends)
    if not ties:
        reference = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="torch")
        # pooled plateaus still tie inside a segment; the raw order must agree exactly
        np.testing.assert_array_equal(result.values.cpu().numpy(), reference.values)
        np.testing.assert_array_equal(result.quotas.cpu().numpy(), reference.quotas)


@pytest.mark.parametrize("fraction", [0.02, 0.3, 0.97])
def test_select_long_segments_across_chunks(device, fraction):
    """Segments longer than one LDS chunk of the per-segment pick (4096 candidates: exactly
    one, one more, several and a ragged last chunk), with many tied values, so the threshold's
    tie group and the pooled tie group both span chunk boundaries: identical to the oracle."""
    rng = np.random.default_rng(int(fraction * 100) + 7)
    lengths = [4096, 4097, 12345, 9000, 33]
    raw, pooled, ends = tables(rng, lengths, ties=True)
    starts = rng.integers(0, 40, len(lengths))
    count = max(1, int(fraction * raw.size))
    result = run_select(device, raw, pooled, ends, starts, count)
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    compare(result, expect, ends)


def test_select_many_segments_and_side_stream(device):
    """More segments than one plan workgroup covers (1024), runs of 0..60 candidates, and the
    queue half on a side stream: identical to the one-stream call and to the oracle."""
    rng = np.random.default_rng(11)
    lengths = rng.integers(1, 60, 1500)
    raw, pooled, ends = tables(rng, lengths, ties=True)
    starts = rng.integers(0, 40, len(lengths))
    count = raw.size // 3
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    coords = [(i // 8, i % 8) for i in range(len(ends))]
    one = run_select(device, raw, pooled, ends, starts, count)
    compare(one, expect, ends)
    side = torch.cuda.Stream(device)
    two = selection.select_refine(torch.from_numpy(raw).to(device),
                                  torch.from_numpy(pooled).to(device), list(ends), list(starts),
                                  coords, count, queue_stream=side)
    two.wait_queue()
    torch.cuda.synchronize()
    compare(two, expect, ends)


def _fused_sets(device, raw_d, bounds_d, starts_d, lengths, count, workspace, width=7):
    """lr_pool_select_refine_sets: pooled table and removal sets."""
    segments, total = len(lengths), raw_d.numel()
    pooled = torch.empty_like(raw_d)
    out = torch.empty((count + 3 * segments + 1,), dtype=torch.int64, device=device)
    removed, quotas = out[:count], out[count:count + segments]
    offsets, changed = out[count + segments:count + 2 * segments + 1], out[count + 2 * segments + 1:]
    _lib.call("lr_pool_select_refine_sets", raw_d.data_ptr(), total, bounds_d.data_ptr(),
              int(max(lengths)), width, pooled.data_ptr(), bounds_d[1:].data_ptr(),
              starts_d.data_ptr(), segments, count, workspace.data_ptr(), workspace.numel(),
              quotas.data_ptr(), offsets.data_ptr(), removed.data_ptr(), changed.data_ptr(), None,
              None, _lib.stream_of(raw_d))
    torch.cuda.synchronize()
    return pooled.cpu().numpy(), quotas.cpu().numpy(), offsets.cpu().numpy(), \
        removed.cpu().numpy(), changed.cpu().numpy()


@pytest.mark.parametrize("ties", [False, True])
def test_pool_select_fused_matches_oracle(device, ties):
    """The fused pool + removal-set entry (its pool launch resets the selection's counters):
    the pooled table equals the oracle's Pool7 bit for bit and the sets equal the oracle's, on
    two calls in a row over one workspace (the second smaller, so stale counts of the first
    would show), against the standalone lr_pool + lr_select_refine_sets as well."""
    rng = np.random.default_rng(5 + ties)
    lengths = [2218] * 9 + [1, 7, 300, 5000, 4097]
    raw, pooled, ends = tables(rng, lengths, ties)
    starts = rng.integers(0, 40, len(lengths))
    raw_d = torch.from_numpy(raw).to(device)
    bounds_d = torch.from_numpy(np.concatenate(([0], ends)).astype(np.int64)).to(device)
    starts_d = torch.from_numpy(starts.astype(np.int64)).to(device)
    first, second = raw.size // 3, max(1, raw.size // 50)
    nbytes = _lib.load().lr_select_workspace_bytes(raw.size, len(lengths), first)
    workspace = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device=device)
    for count in (first, second):
        got_pooled, quotas, offsets, removed, changed = _fused_sets(
            device, raw_d, bounds_d, starts_d, lengths, count, workspace)
        np.testing.assert_array_equal(got_pooled, pooled)
        expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
        np.testing.assert_array_equal(quotas, expect.quotas)
        for s in range(len(lengths)):
            np.testing.assert_array_equal(removed[offsets[s]:offsets[s + 1]],
                                          np.sort(expect.positions[expect.segments == s]))
        separate = selection.select_refine(raw_d, torch.from_numpy(pooled).to(device), list(ends),
                                           list(starts), [(i, 0) for i in range(len(lengths))],
                                           count, queue=False)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(separate.quotas.cpu().numpy(), quotas)
        np.testing.assert_array_equal(separate.offsets.cpu().numpy(), offsets)
        np.testing.assert_array_equal(separate.removed_positions.cpu().numpy(), removed)
        np.testing.assert_array_equal(separate.changed.cpu().numpy(), changed)


@pytest.mark.parametrize("width", [1, 3, 9])
@pytest.mark.parametrize("case", ["one_segment", "count_all", "count_one", "ragged"])
def test_pool_select_fused_edge_cases(device, width, case):
    """The fused entry at pool widths other than 7 and at the edges of the selection: a single
    segment, every candidate selected, a single one, and ragged segments of 1..3000 keys; pooled
    table and sets against the oracle's Pool and refine_arrays."""
    rng = np.random.default_rng(10 * width + ["one_segment", "count_all", "count_one",
                                              "ragged"].index(case))
    lengths = {"one_segment": [3001], "count_all": [17, 400, 5],
               "count_one": [250, 250, 250], "ragged": [1, 2, 3000, 7, 64, 65, 1]}[case]
    ends = np.cumsum(lengths)
    raw = np.round(rng.random(ends[-1]) * 500).astype(np.float32) / 500  # with ties
    pooled = np.empty_like(raw)
    start = 0
    for end in ends:
        pooled[start:end] = kv_ops.pool(raw[start:end], [0, end - start], width)
        start = end
    count = {"one_segment": 777, "count_all": int(ends[-1]), "count_one": 1,
             "ragged": int(ends[-1]) // 3}[case]
    starts = rng.integers(0, 40, len(lengths))
    raw_d = torch.from_numpy(raw).to(device)
    bounds_d = torch.from_numpy(np.concatenate(([0], ends)).astype(np.int64)).to(device)
    starts_d = torch.from_numpy(starts.astype(np.int64)).to(device)
    nbytes = _lib.load().lr_select_workspace_bytes(raw.size, len(lengths), count)
    workspace = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=device)
    got_pooled, quotas, offsets, removed, changed = _fused_sets(
        device, raw_d, bounds_d, starts_d, lengths, count, workspace, width)
    np.testing.assert_array_equal(got_pooled, pooled)
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    np.testing.assert_array_equal(quotas, expect.quotas)
    assert offsets[-1] == count
    for s in range(len(lengths)):
        np.testing.assert_array_equal(removed[offsets[s]:offsets[s + 1]],
                                      np.sort(expect.positions[expect.segments == s]))
    assert int(changed.sum()) == expect.changed


@pytest.mark.parametrize("seed", range(12))
def test_select_random_configurations(device, seed):
    """Seeded random shapes: 1-300 segments of 1-5000 candidates, any count from 1 to all, and a
    tie density from none to heavy, so the threshold's last digit and tie group fall in one,
    several or many segments; removal sets and queue order identical to the oracle."""
    rng = np.random.default_rng(1000 + seed)
    segments = int(rng.integers(1, 301))
    lengths = rng.integers(1, 5001 if segments < 20 else 400, segments)
    ends = np.cumsum(lengths)
    levels = int(rng.choice([0, 3, 50, 5000]))
    raw = rng.random(ends[-1]).astype(np.float32)
    if levels:
        raw = np.floor(raw * levels).astype(np.float32) / levels
    pooled = np.empty_like(raw)
    start = 0
    for end in ends:
        pooled[start:end] = kv_ops.pool(raw[start:end], [0, end - start], 7)
        start = end
    starts = rng.integers(0, 40, segments)
    count = int(rng.integers(1, raw.size + 1))
    result = run_select(device, raw, pooled, ends, starts, count)
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    compare(result, expect, ends)


@pytest.mark.parametrize("crowd", ["lds_network", "global_sort"])
def test_queue_order_crowded_bucket(device, crowd):
    """The queue order cuts the picks into buckets at sampled splitters (every 8th pick here:
    16,384 picks, 2,048 samples). Picks that share one value and sit only between sampled
    positions all land in one bucket: 2,048 of them (sorted by the bucket's LDS network) or
    14,336 (more than a bucket holds in LDS: sorted in global memory). Ties among them go by
    index, across the segment boundary too. Identical to the oracle, every pick selected."""
    rng = np.random.default_rng(31 if crowd == "lds_network" else 37)
    lengths = [5000, 8192, 3192]
    ends = np.cumsum(lengths)
    total = int(ends[-1])
    raw = rng.random(total).astype(np.float32) * 2.0
    at = np.arange(total)
    crowded = (at % 8 == 1) if crowd == "lds_network" else (at % 8 != 0)
    raw[crowded] = 1.0
    pooled = np.empty_like(raw)
    start = 0
    for end in ends:
        pooled[start:end] = kv_ops.pool(raw[start:end], [0, end - start], 7)
        start = end
    starts = [0, 17, 40]
    for count in (total, total - 3000):
        result = run_select(device, raw, pooled, ends, starts, count)
        expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
        compare(result, expect, ends)


def test_select_large_count_radix_path(device):
    """More than 524,288 picks over few segments: the queue order takes the device radix sort
    of the concatenated runs instead of the bucketed merge; identical to the oracle."""
    rng = np.random.default_rng(41)
    lengths = [250_000, 180_000, 5, 220_000]
    raw, pooled, ends = tables(rng, lengths, ties=True)
    starts = [0, 3, 9, 27]
    count = 600_000
    result = run_select(device, raw, pooled, ends, starts, count)
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    compare(result, expect, ends)


def test_select_all_equal_scores(device):
    lengths = [50, 60, 70]
    raw = np.full(180, 0.25, np.float32)
    pooled = raw.copy()
    ends = np.cumsum(lengths)
    for count in (1, 49, 50, 111, 180):
        result = run_select(device, raw, pooled, ends, [0, 3, 5], count)
        expect = oselection.refine_arrays(raw, pooled, ends, [0, 3, 5], count)
        compare(result, expect, ends)


def test_select_nan_and_infinities(device):
    """NaNs of either sign and any payload sort after +inf and among themselves by index (as the
    oracle's numpy sort, and torch.topk, place them); infinities and signed zeros in both tables,
    at every count."""
    rng = np.random.default_rng(23)
    lengths = [40, 1, 57, 30]
    ends = np.cumsum(lengths)
    raw = rng.standard_normal(ends[-1]).astype(np.float32)
    pooled = rng.standard_normal(ends[-1]).astype(np.float32)
    bits = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFFFFFFF, 0x7FA00000], np.uint32)
    specials = np.concatenate((bits.view(np.float32),
                               np.array([np.inf, -np.inf, 0.0, -0.0], np.float32)))
    for table in (raw, pooled):
        at = rng.choice(table.size, 30, replace=False)
        table[at] = specials[rng.integers(0, specials.size, at.size)]
    starts = [0, 5, 9, 11]
    for count in (1, 7, 40, 64, 100, 127, ends[-1]):
        result = run_select(device, raw, pooled, ends, starts, int(count))
        expect = oselection.refine_arrays(raw, pooled, ends, starts, int(count), tie="canonical")
        np.testing.assert_array_equal(result.quotas.cpu().numpy(), expect.quotas)
        np.testing.assert_array_equal(result.segments.cpu().numpy(), expect.segments)
        np.testing.assert_array_equal(result.positions.cpu().numpy(), expect.positions)
        got = result.values.cpu().numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(expect.values))
        finite = ~np.isnan(got)
        np.testing.assert_array_equal(got[finite], expect.values[finite])
        offsets = result.offsets.cpu().numpy()
        removed = result.removed_positions.cpu().numpy()
        for s in range(len(ends)):
            np.testing.assert_array_equal(removed[offsets[s]:offsets[s + 1]],
                                          np.sort(expect.positions[expect.segments == s]))


def test_select_negative_zero_and_signs(device):
    raw = np.asarray([0.0, -0.0, -1.0, 2.0, -0.0, 0.0, 1e-30, -1e-30], np.float32)
    pooled = raw[::-1].copy()
    ends = np.asarray([3, 8])
    for count in range(1, 9):
        result = run_select(device, raw, pooled, ends, [0, 0], count)
        expect = oselection.refine_arrays(raw, pooled, ends, [0, 0], count)
        compare(result, expect, ends)


def test_refine_arrays_signature(device):
    rng = np.random.default_rng(3)
    raw, pooled, ends = tables(rng, [100, 200, 50])
    segs = [scoring.ScoreSegment(0, h, 0, n) for h, n in enumerate([100, 200, 50])]
    allocation = scoring.ScoreTable(torch.from_numpy(raw).to(device), segs, list(ends), 0.0)
    refinement = scoring.ScoreTable(torch.from_numpy(pooled).to(device), segs, list(ends), 0.0)
    refs, changed, heads = selection.refine_arrays(allocation, refinement, 37)
    expect = oselection.refine_arrays(raw, pooled, ends, [0, 0, 0], 37)
    np.testing.assert_array_equal(refs.positions, expect.positions)
    assert (changed, heads) == (expect.changed, expect.changed_heads)
    assert {k: list(v) for k, v in refs.groups().items()} == {
        k: list(v) for k, v in expect.groups([(0, 0), (0, 1), (0, 2)]).items()}


@pytest.mark.parametrize("queue_order", [False, True])
def test_native_and_python_launches_agree(device, queue_order):
    """The C++ host module and the Python launch sequence make the same launches: every output
    of the step is bit-identical (prompt protection and a head without candidates included)."""
    head_lengths = [[400, 380, 35, 410], [390, 10, 400, 402]]
    layers, qpos = workloads.make_layers(head_lengths, 4, 128, 80, device, seed=5,
                                         prompt_lengths=[[3, 0, 40, 7], [0, 0, 12, 390]])
    margin = torch.tensor([2.0], device=device)
    step = audit.AuditStep()
    native = step.run(layers, qpos, margin, 500, queue_order=queue_order)
    python = step.run(layers, qpos, margin, 500, queue_order=queue_order, native=False)
    torch.cuda.synchronize()
    assert native.head_lens == python.head_lens and native.removed == python.removed
    np.testing.assert_array_equal(native.scores.cpu().numpy(), python.scores.cpu().numpy())
    np.testing.assert_array_equal(native.pooled.cpu().numpy(), python.pooled.cpu().numpy())
    for a, b in zip(native.layers, python.layers):
        assert torch.equal(a.keys, b.keys) and torch.equal(a.values, b.values)
        assert torch.equal(a.positions, b.positions)
    for name in ("quotas", "offsets", "removed_positions", "changed"):
        assert torch.equal(getattr(native.selection, name), getattr(python.selection, name))
    if queue_order:
        qa, qb = native.selection.references(), python.selection.references()
        np.testing.assert_array_equal(qa.scores, qb.scores)
        np.testing.assert_array_equal(qa.segments, qb.segments)
        np.testing.assert_array_equal(qa.positions, qb.positions)


@pytest.mark.parametrize("dim,groups,queue_order", [(128, 4, False), (64, 4, False), (128, 4, True)])
def test_audit_step_matches_oracle_chain(device, dim, groups, queue_order):
    head_lengths = [[400, 380, 35, 410], [390, 10, 400, 402], [333, 401, 399, 64]]
    layers, qpos = workloads.make_layers(head_lengths, groups, dim, 80, device, seed=11)
    margin = torch.tensor([2.0], device=device)
    count = 600
    step = audit.AuditStep()
    for _ in range(2):  # the second call reuses the step's workspaces (and side stream)
        outcome = step.run(layers, qpos, margin, count, queue_order=queue_order)
    torch.cuda.synchronize()
    raw = outcome.scores.cpu().numpy()
    ends = np.asarray(outcome.cumulative_ends)
    pooled = kv_ops.pool(raw, np.concatenate(([0], ends)), 7)
    np.testing.assert_array_equal(outcome.pooled.cpu().numpy(), pooled)
    starts = [s.position_start for s in outcome.segments]
    expect = oselection.refine_arrays(raw, pooled, ends, starts, count)
    if queue_order:
        queue = outcome.selection.references()
        np.testing.assert_array_equal(queue.scores, expect.values)
        np.testing.assert_array_equal(queue.segments, expect.segments)
        np.testing.assert_array_equal(queue.positions, expect.positions)
    else:
        assert outcome.selection.values is None
    coords = [(s.layer, s.head) for s in outcome.segments]
    groups_ = expect.groups(coords)
    for layer_index, layer in enumerate(layers):
        bounds = np.concatenate(([0], np.cumsum(layer.head_lens)))
        removed = np.sort(np.concatenate([bounds[h] + groups_.get((layer_index, h), np.zeros(0, np.int64))
                                          for h in range(len(layer.head_lens))])).astype(np.int64)
        ek, ev, ep = kv_ops.compact(layer.keys.view(torch.int16).cpu().numpy(),
                                    layer.values.view(torch.int16).cpu().numpy(),
                                    layer.positions.cpu().numpy(), removed)
        got = outcome.layers[layer_index]
        np.testing.assert_array_equal(got.keys.view(torch.int16).cpu().numpy(), ek)
        np.testing.assert_array_equal(got.values.view(torch.int16).cpu().numpy(), ev)
        np.testing.assert_array_equal(got.positions.cpu().numpy(), ep.reshape(-1))
        expect_lens = [n - len(groups_.get((layer_index, h), [])) for h, n in enumerate(layer.head_lens)]
        assert outcome.head_lens[layer_index] == expect_lens
    assert sum(map(sum, outcome.head_lens)) == sum(map(sum, head_lengths)) - count


def test_pool_score_table_signature(device):
    rng = np.random.default_rng(4)
    raw, _, ends = tables(rng, [30, 1, 90])
    segs = [scoring.ScoreSegment(0, h, 0, n) for h, n in enumerate([30, 1, 90])]
    table = scoring.ScoreTable(torch.from_numpy(raw).to(device), segs, list(ends), 0.0)
    pooled = audit.pool_score_table(table, 7)
    np.testing.assert_array_equal(pooled.scores.cpu().numpy(), kv_ops.pool(raw, np.concatenate(([0], ends)), 7))
