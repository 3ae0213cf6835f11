"""Pins the selection oracle (oracle/selection.py) and the CPU baseline chain (oracle/cpu_path.py)
against checks that do not reuse their code:

- a brute-force restatement with Python's sorted() over (value, index) pairs and explicit loops
  (no lexsort, searchsorted, bincount or argsort), on small random tables with and without ties;
- a known-answer table worked out by hand;
- invariants: quotas sum to count, every segment removes exactly its quota, the removal sets
  are distinct positions, and the torch.topk tie rule equals the canonical one on tie-free data;
- the evict-prefix remap against a direct count;
- audit_step_cpu (the timed CPU baseline) against the oracle chain built from the other modules.
"""

import numpy as np
import pytest
import torch

from oracle import cpu_path, kv_ops, scoring
from oracle import selection as osel


def brute_force(raw, pooled, ends, starts, count):
    """selection.py:52-88 by full sorts and loops."""
    bounds = [0] + [int(e) for e in ends]
    pairs = sorted((float(v), i) for i, v in enumerate(raw))[:count]

    def segment_of(index):
        for s in range(len(ends)):
            if bounds[s] <= index < bounds[s + 1]:
                return s
        raise AssertionError("index outside every segment")

    slot_segments = [segment_of(i) for _, i in pairs]
    quotas = [slot_segments.count(s) for s in range(len(ends))]
    refined = {}
    for s in range(len(ends)):
        local = sorted((float(pooled[bounds[s] + j]), j) for j in range(bounds[s + 1] - bounds[s]))
        refined[s] = [j for _, j in local[:quotas[s]]]
    used = {s: 0 for s in range(len(ends))}
    positions = []
    for s in slot_segments:  # slots of a segment, in slot order, take its refined picks in order
        positions.append(int(starts[s]) + refined[s][used[s]])
        used[s] += 1
    raw_set = {i for _, i in pairs}
    changed = [(s, j) for s in range(len(ends)) for j in refined[s] if bounds[s] + j not in raw_set]
    return (np.asarray([v for v, _ in pairs], np.float32), np.asarray(slot_segments),
            np.asarray(positions), len(changed), len({s for s, _ in changed}), np.asarray(quotas))


def pooled_of(raw, ends, width=7):
    out, start = np.empty_like(raw), 0
    for end in ends:
        out[start:end] = kv_ops.pool(raw[start:end], [0, end - start], width)
        start = end
    return out


@pytest.mark.parametrize("seed", range(12))
def test_refine_arrays_equals_brute_force(seed):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, 9, rng.integers(1, 6))
    ends = np.cumsum(lengths)
    raw = rng.random(ends[-1]).astype(np.float32)
    if seed % 2:
        raw = np.round(raw * 4).astype(np.float32) / 4  # heavy ties
    pooled = pooled_of(raw, ends)
    starts = rng.integers(0, 5, len(lengths))
    for count in range(1, int(ends[-1]) + 1):
        got = osel.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
        values, segments, positions, changed, changed_heads, quotas = brute_force(
            raw, pooled, ends, starts, count)
        np.testing.assert_array_equal(got.values, values)
        np.testing.assert_array_equal(got.segments, segments)
        np.testing.assert_array_equal(got.positions, positions)
        np.testing.assert_array_equal(got.quotas, quotas)
        assert (got.changed, got.changed_heads) == (changed, changed_heads)


def test_refine_arrays_known_answer():
    # two segments: [0.5, 0.1, 0.9] and [0.2, 0.3]; pooled scores chosen by hand
    raw = np.asarray([0.5, 0.1, 0.9, 0.2, 0.3], np.float32)
    pooled = np.asarray([0.4, 0.8, 0.7, 0.6, 0.1], np.float32)
    ends, starts = [3, 5], [10, 20]
    got = osel.refine_arrays(raw, pooled, ends, starts, 3)
    # raw bottom-3: 0.1 (seg 0), 0.2 (seg 1), 0.3 (seg 1) -> quotas [1, 2]
    np.testing.assert_array_equal(got.values, np.asarray([0.1, 0.2, 0.3], np.float32))
    np.testing.assert_array_equal(got.segments, [0, 1, 1])
    np.testing.assert_array_equal(got.quotas, [1, 2])
    # pooled bottom-1 of seg 0 is local 0 (0.4); bottom-2 of seg 1 are local 1 (0.1), 0 (0.6)
    np.testing.assert_array_equal(got.positions, [10, 21, 20])
    # refined seg 0 pick (global 0) is not a raw pick; seg 1 picks {3, 4} equal the raw picks
    assert (got.changed, got.changed_heads) == (1, 1)


@pytest.mark.parametrize("seed", range(4))
def test_selection_invariants_and_torch_rule(seed):
    rng = np.random.default_rng(100 + seed)
    lengths = rng.integers(20, 400, 9)
    ends = np.cumsum(lengths)
    raw = rng.permutation(ends[-1]).astype(np.float32) / ends[-1]  # distinct values
    pooled = pooled_of(raw, ends)
    starts = rng.integers(0, 50, len(lengths))
    count = int(rng.integers(1, ends[-1]))
    canonical = osel.refine_arrays(raw, pooled, ends, starts, count, tie="canonical")
    assert canonical.quotas.sum() == count
    assert np.all(np.diff(canonical.values) >= 0)
    for s in range(len(ends)):
        mine = canonical.positions[canonical.segments == s]
        assert mine.size == canonical.quotas[s] == np.unique(mine).size
    torch_rule = osel.refine_arrays(raw, pooled, ends, starts, count, tie="torch")
    np.testing.assert_array_equal(torch_rule.values, canonical.values)
    np.testing.assert_array_equal(torch_rule.segments, canonical.segments)
    np.testing.assert_array_equal(torch_rule.quotas, canonical.quotas)
    # pooled plateaus tie inside a segment, where torch.topk may take other indices at the cut;
    # both must still take the same multiset of pooled values
    bounds = np.concatenate(([0], ends))
    for s in range(len(ends)):
        pick = lambda sel: np.sort(pooled[bounds[s] + sel.positions[sel.segments == s] - starts[s]])
        np.testing.assert_array_equal(pick(torch_rule), pick(canonical))


def test_evict_prefix_remap_counts_earlier_removals():
    removed = [2, 5, 9]
    queued = [0, 3, 6, 10]
    shifted, union = osel.evict_prefix_remap(queued, removed)
    np.testing.assert_array_equal(shifted, [p - sum(r < p for r in removed) for p in queued])
    np.testing.assert_array_equal(union, sorted(set(removed) | set(queued)))


def test_audit_step_cpu_equals_oracle_chain():
    rng = np.random.default_rng(21)
    heads, groups, dim, window, length = 2, 2, 32, 6, 48
    layers = []
    for _ in range(2):
        rows = heads * length
        layers.append(dict(
            keys=torch.from_numpy((rng.integers(-2, 3, (rows, dim)) * 0.25).astype(np.float32)).to(torch.bfloat16),
            values=torch.randn((rows, dim), generator=torch.Generator().manual_seed(int(rng.integers(1 << 30)))).to(torch.bfloat16),
            positions=torch.arange(length, dtype=torch.float32).repeat(heads),
            head_lens=[length] * heads,
            queries=torch.from_numpy((rng.integers(-2, 3, (heads * groups, window, dim)) * 0.25).astype(np.float32)).to(torch.bfloat16),
            gradient=torch.from_numpy(np.abs(rng.standard_normal((heads * groups, dim))).astype(np.float32))))
    qpos = torch.arange(length - window, length, dtype=torch.int64)
    margin = torch.tensor(2.0)
    count = 20
    raw, pooled, selection, compacted = cpu_path.audit_step_cpu(layers, qpos, margin, count,
                                                                protect_recent=8)
    # the oracle chain: per-head numpy scores -> pool -> refine -> numpy compaction
    scores, ends, coords = [], [], []
    for li, layer in enumerate(layers):
        for h in range(heads):
            rows = slice(h * length, (h + 1) * length)
            q = layer["queries"][h * groups:(h + 1) * groups].permute(1, 0, 2).float().numpy()
            part = scoring.head_scores(q, qpos.numpy(), layer["keys"][rows].float().numpy(),
                                       layer["positions"][rows].numpy(),
                                       layer["values"][rows].float().numpy(), 0, length - 8,
                                       layer["gradient"][h * groups:(h + 1) * groups].numpy(),
                                       np.float32(2.0), 1e-6)
            scores.append(part)
            ends.append(sum(map(len, scores)))
            coords.append((li, h))
    expect_raw = np.concatenate(scores)
    np.testing.assert_allclose(raw.numpy(), expect_raw, rtol=1e-5, atol=1e-12)
    expect_pooled = pooled_of(raw.numpy(), np.asarray(ends))
    np.testing.assert_array_equal(pooled.numpy(), expect_pooled)
    # same tie rule as the CPU path (torch.topk); the tie rules are compared separately above
    expect = osel.refine_arrays(raw.numpy(), expect_pooled, ends, [0] * len(ends), count, tie="torch")
    groups_ = expect.groups(coords)
    for li, layer in enumerate(layers):
        removed = np.sort(np.concatenate(
            [h * length + groups_.get((li, h), np.zeros(0, np.int64)) for h in range(heads)]))
        ek, ev, ep = kv_ops.compact(layer["keys"].view(torch.int16).numpy(),
                                    layer["values"].view(torch.int16).numpy(),
                                    layer["positions"].numpy(), removed.astype(np.int64))
        k, v, p = compacted[li]
        np.testing.assert_array_equal(k.view(torch.int16).numpy(), ek)
        np.testing.assert_array_equal(v.view(torch.int16).numpy(), ev)
        np.testing.assert_array_equal(p.numpy(), ep.reshape(-1))
