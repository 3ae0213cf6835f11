"""The recall archive (liblazyrecall_archive.so through code_for_iclr27_amd.archive) against the
oracle restatement of cpu_worker.py:17-134, and the oracle pinned by hand-worked answers.

Host code: these run without a GPU. Keys and queries with small integer entries make every inner
product exact in f32 and f64, so search results (order included, ties in insertion order) are
compared exactly; a real-valued case compares the top-k sets where no near-tie straddles them.
"""

import numpy as np
import pytest

from code_for_iclr27_amd import archive as native
from oracle import archive as oracle


def bf16_bits(values):
    return (np.asarray(values, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def payload_for(keys, seed):
    rng = np.random.default_rng(seed)
    values = rng.integers(-3, 4, keys.shape).astype(np.float32)
    return np.stack([bf16_bits(keys), bf16_bits(values)], axis=1)


def test_oracle_known_answers():
    head = oracle.HeadArchive(2, 3)
    keys = np.array([[1, 0], [0, 1], [1, 1], [2, 2]], dtype=np.float32)
    head.add(np.array([10, 11, 12]), payload_for(keys[:3], 0))
    assert head.search(np.array([1.0, 0.0]), 2)[0].tolist() == [10, 12]  # 1 (=12's 1) tie: order
    head.add(np.array([13]), payload_for(keys[3:], 1))  # full: overwrites slot 0 (position 10)
    assert head.dropped == 1 and sorted(head.lookup) == [11, 12, 13]
    head.remove([11])
    assert head.free == [1]
    head.add(np.array([14]), payload_for(keys[:1], 2))  # reuses the freed slot 1
    assert head.lookup[14] == 1 and head.dropped == 1
    assert head.search(np.array([1.0, 1.0]), 5)[0].tolist() == [13, 12, 14]
    with pytest.raises(ValueError, match="Duplicate identities"):
        head.add(np.array([7, 7]), payload_for(keys[:2], 3))


def run_script(index, ops):
    results = []
    for op in ops:
        if op[0] == "add":
            index.add(op[1], op[2])
        elif op[0] == "remove":
            index.remove(op[1])
        else:
            results.append(index.search(op[1], op[2]))
        results.append((index.size, index.dropped))
    return results


def random_ops(seed, layers, heads, dim, steps):
    rng = np.random.default_rng(seed)
    ops = []
    for step in range(steps):
        kind = rng.choice(["add", "add", "remove", "search"])
        if kind == "add":
            n = int(rng.integers(1, 40))
            meta = np.stack([rng.integers(0, layers, n), rng.integers(0, heads, n),
                             rng.integers(0, 60, n)], axis=1).astype(np.int64)
            _, first = np.unique(meta, axis=0, return_index=True)
            meta = meta[np.sort(first)]
            keys = rng.integers(-4, 5, (len(meta), dim)).astype(np.float32)
            ops.append(("add", meta, payload_for(keys, step)))
        elif kind == "remove":
            n = int(rng.integers(1, 10))
            meta = np.stack([rng.integers(0, layers, n), rng.integers(0, heads, n),
                             rng.integers(0, 60, n)], axis=1)
            # unique identities: the reference raises KeyError on a repeated one (it pops the
            # same lookup entry twice), the native archive removes it once
            ops.append(("remove", np.unique(meta, axis=0)))
        else:
            queries = rng.integers(-3, 4, (layers * heads, dim)).astype(np.float32)
            ops.append(("search", queries, int(rng.integers(1, 6))))
    return ops


@pytest.mark.parametrize("seed,capacity", [(0, 8), (1, 16), (2, 1000), (3, 3)])
def test_native_equals_oracle_on_random_operations(seed, capacity):
    layers, heads, dim = 2, 3, 16
    ops = random_ops(seed, layers, heads, dim, 120)
    got = run_script(native.ArchiveIndex(layers, heads, dim, 2, capacity), ops)
    expect = run_script(oracle.ArchiveIndex(layers, heads, dim, capacity), ops)
    assert len(got) == len(expect)
    for g, e in zip(got, expect):
        if isinstance(g[0], np.ndarray):
            np.testing.assert_array_equal(g[0], e[0])
            np.testing.assert_array_equal(g[1], e[1])
        else:
            assert g == e


def test_real_valued_search_sets():
    rng = np.random.default_rng(9)
    layers, heads, dim, rows = 2, 2, 128, 300
    index = native.ArchiveIndex(layers, heads, dim, 4, 4096)
    reference = oracle.ArchiveIndex(layers, heads, dim, 4096)
    keys = rng.standard_normal((rows * layers * heads, dim)).astype(np.float32)
    keys = bf16_bits(keys).astype(np.uint32) << 16
    keys = keys.view(np.float32)
    meta = np.stack([np.repeat(np.arange(layers), heads * rows), np.tile(np.repeat(np.arange(heads), rows), layers),
                     np.tile(np.arange(rows), layers * heads)], axis=1).astype(np.int64)
    payload = payload_for(keys, 4)
    index.add(meta, payload)
    reference.add(meta, payload)
    queries = rng.standard_normal((layers * heads, dim)).astype(np.float32)
    got_meta, got_payload = index.search(queries, 8)
    expect_meta, expect_payload = reference.search(queries, 8)
    np.testing.assert_array_equal(got_meta, expect_meta)
    np.testing.assert_array_equal(got_payload, expect_payload)


def test_errors_like_the_reference():
    index = native.ArchiveIndex(1, 2, 4, 1, 8)
    with pytest.raises(ValueError, match="shape mismatch"):
        index.add(np.zeros((2, 3), np.int64), np.zeros((3, 2, 4), np.uint16))
    with pytest.raises(ValueError, match="Invalid archive identity"):
        index.add(np.array([[0, 2, 5]]), np.zeros((1, 2, 4), np.uint16))
    with pytest.raises(ValueError, match="Duplicate identities"):
        index.add(np.array([[0, 1, 5], [0, 1, 5]]), np.zeros((2, 2, 4), np.uint16))
    assert index.size == 0  # nothing was added by the failed calls
    empty_meta, empty_payload = index.search(np.ones((2, 4), np.float32), 3)
    assert empty_meta.shape == (0, 3) and empty_payload.shape == (0, 2, 4)
