"""Pins the data-movement oracle against independent formulations (CPU only).

compact:        np.delete of the removed rows == the reference kernel's own gather rule
append:         a per-head Python loop == the oracle; new positions are consecutive
legacy append:  torch.cat per head (the reference's own CPU fallback) == the oracle
merge:          merge of disjoint position sets is sorted and a permutation of the union
pool:           torch F.max_pool1d (the reference CPU path) == the oracle
batch_append:   per-request legacy append == the packed oracle
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from hypothesis import given, settings, strategies as st

from oracle import kv_ops


def _rows(rng, n, d, dtype=np.float32):
    return rng.standard_normal((n, d)).astype(dtype)


@settings(max_examples=60, deadline=None)
@given(rows=st.integers(0, 40), dim=st.integers(1, 5), data=st.data())
def test_compact_matches_gather_rule(rows, dim, data):
    rng = np.random.default_rng(rows * 7 + dim)
    drawn = data.draw(st.sets(st.integers(0, max(rows - 1, 0)), max_size=rows)) if rows else set()
    removed = np.sort(np.asarray(sorted(drawn), dtype=np.int64))
    keys, values = _rows(rng, rows, dim), _rows(rng, rows, dim)
    pos = np.arange(rows, dtype=np.float32)
    a = kv_ops.compact(keys, values, pos, removed)
    b = kv_ops.compact_by_gather_rule(keys, values, pos, removed)
    c = (np.delete(keys, removed, 0), np.delete(values, removed, 0), np.delete(pos, removed)[:, None])
    for x, y, z in zip(a, b, c):
        np.testing.assert_array_equal(x, y)
        np.testing.assert_array_equal(x, z)


def test_append_per_head_loop():
    rng = np.random.default_rng(0)
    lens = [3, 0, 5, 2]
    cum = np.concatenate(([0], np.cumsum(lens))).astype(np.int32)
    keys, values = _rows(rng, cum[-1], 4), _rows(rng, cum[-1], 4)
    pos = rng.permutation(cum[-1]).astype(np.float32)
    added = 2
    nk = rng.standard_normal((1, 4, added, 4)).astype(np.float32)
    nv = rng.standard_normal((1, 4, added, 4)).astype(np.float32)
    out_k, out_v, out_p, out_cum, out_len = kv_ops.append(keys, values, pos, nk, nv, cum, 100, max(lens))
    expect_k, expect_p = [], []
    for h, length in enumerate(lens):
        expect_k.append(keys[cum[h]:cum[h + 1]])
        expect_k.append(nk[0, h])
        expect_p.extend(pos[cum[h]:cum[h + 1]])
        expect_p.extend([100, 101])
    np.testing.assert_array_equal(out_k, np.concatenate(expect_k))
    np.testing.assert_array_equal(out_p.reshape(-1), np.asarray(expect_p, np.float32))
    np.testing.assert_array_equal(out_len, np.asarray(lens) + added)
    np.testing.assert_array_equal(out_cum[:-1], cum[:-1] + np.arange(4) * added)


def test_legacy_append_matches_torch_cat():
    rng = np.random.default_rng(1)
    lens = [2, 3, 0, 1, 4, 2]
    states = rng.standard_normal((2, 3, 2, 5)).astype(np.float32)
    cache = _rows(rng, sum(lens), 5)
    got = kv_ops.append_flattened_cache(cache, states, lens)
    parts, offset = [], 0
    t_cache, t_states = torch.from_numpy(cache), torch.from_numpy(states)
    for flat, length in enumerate(lens):
        parts.append(t_cache[offset:offset + length])
        parts.append(t_states[flat // 3, flat % 3])
        offset += length
    np.testing.assert_array_equal(got, torch.cat(parts).numpy())


def test_merge_of_disjoint_heads_is_sorted_permutation():
    rng = np.random.default_rng(2)
    lens = [6, 4]
    universe = [rng.permutation(40)[:10] for _ in lens]
    old = np.concatenate([np.sort(u[:n]) for u, n in zip(universe, lens)])
    meta = np.asarray([(3, h, p) for h, u in enumerate(universe) for p in u[lens[h]:lens[h] + 3]])
    mapping, new_lens = kv_ops.merge_plan(old, lens, meta)
    assert new_lens == [9, 7]
    keys = old.astype(np.float32)[:, None]
    recalled = np.stack((meta[:, 2], meta[:, 2]), axis=1).astype(np.float32)[:, :, None]
    mk, mv, mp = kv_ops.merge(keys, keys, old.astype(np.float32), recalled,
                              meta[:, 2].astype(np.float32), mapping)
    start = 0
    for h, n in enumerate(new_lens):
        seg = mp[start:start + n, 0]
        assert np.all(np.diff(seg) > 0)
        np.testing.assert_array_equal(np.sort(seg), np.sort(np.concatenate(
            (old[sum(lens[:h]):sum(lens[:h + 1])], meta[meta[:, 1] == h, 2]))))
        start += n
    np.testing.assert_array_equal(mk[:, 0], mp[:, 0])
    with pytest.raises(ValueError):
        kv_ops.merge_plan(old, lens, np.asarray([(0, 0, old[0])]))


@pytest.mark.parametrize("width", [1, 3, 7, 9])
def test_pool_matches_max_pool1d(width):
    rng = np.random.default_rng(width)
    lengths = [1, 5, 13, 2, 40]
    ends = np.cumsum(lengths)
    scores = rng.standard_normal(ends[-1]).astype(np.float32)
    scores[1::5] = scores[::5][: len(scores[1::5])]  # plateaus/ties
    got = kv_ops.pool(scores, np.concatenate(([0], ends)), width)
    start = 0
    for end in ends:
        seg = torch.from_numpy(scores[start:end]).reshape(1, 1, -1)
        expect = F.max_pool1d(seg, kernel_size=width, stride=1, padding=width // 2).reshape(-1)
        np.testing.assert_array_equal(got[start:end], expect.numpy())
        start = end


def test_batch_append_equals_per_request_append():
    rng = np.random.default_rng(3)
    heads, dim = 3, 4
    lengths = [[2, 0, 3], [1, 4, 1]]
    keys = [_rows(rng, sum(l), dim) for l in lengths]
    values = [_rows(rng, sum(l), dim) for l in lengths]
    positions = [np.arange(sum(l), dtype=np.float32) for l in lengths]
    nk = rng.standard_normal((2, heads, 1, dim)).astype(np.float32)
    nv = rng.standard_normal((2, heads, 1, dim)).astype(np.float32)
    pk, pv, pp = kv_ops.batch_append(keys, values, positions, nk, nv, lengths, [7, 9])
    expect_k = np.concatenate([kv_ops.append_flattened_cache(keys[r], nk[r:r + 1], lengths[r])
                               for r in range(2)])
    np.testing.assert_array_equal(pk, expect_k)
    assert pp.shape == (sum(map(sum, lengths)) + 2 * heads, 1)
    assert set(pp[np.cumsum([l + 1 for ls in lengths for l in ls]) - 1, 0]) == {7.0, 9.0}


def test_pack_metadata_truncates_positions():
    keys = np.arange(12, dtype=np.float32).reshape(6, 2)
    pos = np.asarray([0, 1.0, 2.0, 16777215.0, 4, 5], dtype=np.float32)
    payload, meta = kv_ops.pack(keys, keys + 100, pos, [3, 1], [2, 0], 5)
    np.testing.assert_array_equal(payload[:, 0], keys[[3, 1]])
    np.testing.assert_array_equal(payload[:, 1], keys[[3, 1]] + 100)
    np.testing.assert_array_equal(meta, [[5, 2, 16777215], [5, 0, 1]])
