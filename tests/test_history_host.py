"""The query-history oracle and the host-side checks of the device ring (no GPU needed).

The oracle (oracle/history.py, history.py:11-63) is pinned by what a bounded window fixes:
after n appends ``layer`` holds exactly the last min(n, W) appended queries in append order
(a list slice of everything appended), with their positions. The ring's slot arithmetic
(append k at row k mod W and k mod W + W of a 2W ring; the window starts at n mod W once
n >= W) is checked by brute force against the same slice on a host model of the ring.
"""

import numpy as np
import pytest
import torch

from code_for_iclr27_amd.history import QueryHistory
from oracle import history as ohistory


def queries(rng, layers, heads, dim):
    return [rng.standard_normal((1, heads, 1, dim)).astype(np.float32) for _ in range(layers)]


@pytest.mark.parametrize("window", [1, 3, 8])
def test_oracle_window_is_the_last_appended_queries(window):
    rng = np.random.default_rng(window)
    layers, heads, dim = 3, 4, 5
    oracle = ohistory.QueryHistory(layers, window)
    appended, positions = [], []
    for step in range(3 * window + 2):
        q = queries(rng, layers, heads, dim)
        oracle.append(q, 10 + 3 * step)
        appended.append(q)
        positions.append(10 + 3 * step)
        n = min(len(appended), window)
        for layer in range(layers):
            got, got_pos = oracle.layer(layer)
            expect = np.concatenate([a[layer] for a in appended[-n:]], axis=2)
            np.testing.assert_array_equal(got, expect)
            np.testing.assert_array_equal(got_pos, positions[-n:])


def test_oracle_rejects_like_the_reference():
    oracle = ohistory.QueryHistory(2, 4)
    with pytest.raises(ValueError, match="temporal window must be positive"):
        ohistory.QueryHistory(2, 0)
    with pytest.raises(RuntimeError, match="No query history for layer 1"):
        oracle.layer(1)
    with pytest.raises(RuntimeError, match="layer count mismatch"):
        oracle.append([np.zeros((1, 2, 1, 3))], 5)
    oracle.append([np.zeros((1, 2, 1, 3))] * 2, 5)
    with pytest.raises(RuntimeError, match="strictly increasing"):
        oracle.append([np.zeros((1, 2, 1, 3))] * 2, 5)


@pytest.mark.parametrize("window", [1, 2, 5, 250])
def test_ring_slots_reproduce_the_window(window):
    """The doubled-ring rule on a host array, against the list slice, for 2.5 windows."""
    ring = np.full(2 * window, -1, np.int64)
    appended = []
    for k in range(int(2.5 * window) + 1):
        slot = k % window
        ring[slot] = ring[slot + window] = k
        appended.append(k)
        n = len(appended)
        start = n % window if n >= window else 0
        count = min(n, window)
        np.testing.assert_array_equal(ring[start:start + count], appended[-count:])


def test_device_ring_checks_before_writing():
    history = QueryHistory(2, 4)
    with pytest.raises(ValueError, match="temporal window must be positive"):
        QueryHistory(2, 0)
    with pytest.raises(RuntimeError, match="No query history for layer 0"):
        history.layer(0)
    with pytest.raises(RuntimeError, match="layer count mismatch"):
        history.append([torch.zeros(1, 2, 1, 8)], 3)
    with pytest.raises(RuntimeError, match="Expected one decode query at layer 1"):
        history.append([torch.zeros(1, 2, 1, 8), torch.zeros(1, 2, 2, 8)], 3)
    with pytest.raises(RuntimeError, match="must be CUDA tensors"):
        history.append([torch.zeros(1, 2, 1, 8)] * 2, 3)
    assert history.size == 0 and history.positions == () and history.retained_bytes == 0
