"""Host side of the deletion queue (code_for_iclr27_amd.selection.ArrayReferences, the type of
src/lazy_recall/selection.py:8-39): integer indexing gives KVReference elements with the
reference's fields and ordering (_core/scoring.py:214-219), slices stay queues over the same
segments, and groups() equals the oracle's per-head grouping (a loop over np.unique) on queues
built by the oracle selection, whole and for every prefix/suffix split."""

import dataclasses

import numpy as np
import pytest

from code_for_iclr27_amd.selection import ArrayReferences, KVReference
from oracle import selection as osel


def test_queue_elements_are_kv_references():
    queue = ArrayReferences(np.asarray([0.5, 0.25, 0.75], np.float32), [1, 0, 1], [7, 3, 2],
                            [(4, 0), (4, 5)])
    first = queue[0]
    assert isinstance(first, KVReference)
    assert (first.score, first.layer, first.head, first.position) == (0.5, 4, 5, 7)
    assert queue[1].layer == 4 and queue[1].head == 0 and queue[1].position == 3
    assert queue[-1] == KVReference(0.75, 4, 5, 2)
    assert [field.name for field in dataclasses.fields(KVReference)] == \
        ["score", "layer", "head", "position"]
    assert sorted(queue) == [queue[1], queue[0], queue[2]]  # ordered by score first
    assert KVReference(1.0, 0, 0, 3) < KVReference(1.0, 0, 1, 0)  # then layer, head, position
    tail = queue[1:]
    assert isinstance(tail, ArrayReferences) and len(tail) == 2 and tail[0] == queue[1]
    with pytest.raises(ValueError, match="Queue column lengths differ"):
        ArrayReferences([0.0], [0, 1], [0], [(0, 0), (0, 1)])
    assert ArrayReferences([], [], [], []).groups() == {}


@pytest.mark.parametrize("seed", range(6))
def test_groups_match_oracle_grouping(seed):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(5, 60, rng.integers(2, 9))
    ends = np.cumsum(lengths)
    raw = rng.random(ends[-1], dtype=np.float32)
    if seed % 2:
        raw = np.round(raw * 8) / 8  # ties
    pooled = np.maximum(raw, np.roll(raw, 1))
    starts = rng.integers(0, 4, len(lengths))
    count = int(rng.integers(1, ends[-1] + 1))
    selection = osel.refine_arrays(raw, pooled, ends, starts, count)
    coordinates = [(int(s) // 3, int(s) % 3) for s in range(len(lengths))]
    queue = ArrayReferences(selection.values, selection.segments, selection.positions, coordinates)
    for split in sorted({0, 1, count // 2, count - 1, count}):
        for part in (queue[:split], queue[split:]):
            sub = osel.Selection(part.scores, part.segments, part.positions, 0, 0, None)
            expect = sub.groups(coordinates) if len(part) else {}
            got = part.groups()
            assert list(got) == list(expect)
            for key in expect:
                np.testing.assert_array_equal(got[key], expect[key])
