"""GPU parity of the device query-history ring against the oracle's deques (history.py:11-63),
bit-exact, and of an audit step that scores straight from the ring's strided window against
the same step on contiguous copies of that window."""

import dataclasses

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import audit, workloads
from code_for_iclr27_amd.history import QueryHistory
from oracle import history as ohistory

pytestmark = pytest.mark.gpu


def host_bits(t):
    if t.dtype == torch.float32:
        return t.cpu().numpy().view(np.int32)
    return t.cpu().view(torch.int16).numpy()


@pytest.mark.parametrize("layers,heads,dim,window,dtype", [
    (3, 8, 128, 5, torch.bfloat16),     # 16-byte granules
    (2, 4, 3, 4, torch.float32),        # 12-byte rows: 4-byte granules
    (2, 3, 3, 1, torch.bfloat16),       # 6-byte rows: 2-byte granules, window of one
    (130, 2, 64, 3, torch.bfloat16),    # more layers than one launch carries (128)
])
def test_ring_matches_oracle(device, layers, heads, dim, window, dtype):
    print(f"history ring L{layers} H{heads} d{dim} W{window} {dtype}", flush=True)
    gen = torch.Generator(device=device).manual_seed(layers * 100 + dim)
    history = QueryHistory(layers, window)
    oracle = ohistory.QueryHistory(layers, window)
    for step in range(2 * window + 3):
        step_queries = [torch.randn((1, heads, 1, dim), generator=gen, device=device).to(dtype)
                        for _ in range(layers)]
        position = 100 + 7 * step
        history.append(step_queries, position)
        oracle.append([host_bits(q) for q in step_queries], position)
        for layer in sorted({0, layers // 2, layers - 1}):
            got, got_pos = history.layer(layer)
            expect, expect_pos = oracle.layer(layer)
            assert got.shape == expect.shape
            np.testing.assert_array_equal(host_bits(got.contiguous()), expect)
            np.testing.assert_array_equal(got_pos.cpu().numpy(), expect_pos)
        assert history.positions == tuple(int(p) for p in expect_pos)
        assert history.size == min(step + 1, window)
        assert history.retained_bytes == layers * history.size * heads * dim * got.element_size()


def test_ring_rejects_mismatched_layers(device):
    history = QueryHistory(2, 4)
    q = torch.zeros((1, 4, 1, 64), dtype=torch.bfloat16, device=device)
    history.append([q, q], 1)
    with pytest.raises(RuntimeError, match="layer shape mismatch"):
        history.append([q, q.float()], 2)
    with pytest.raises(RuntimeError, match="layer shape mismatch"):
        history.append([q, torch.zeros((1, 2, 1, 64), dtype=torch.bfloat16, device=device)], 2)
    with pytest.raises(RuntimeError, match="strictly increasing"):
        history.append([q, q], 1)
    assert history.size == 1


@pytest.mark.parametrize("queue_order", [False, True])
def test_audit_from_ring_window_equals_contiguous(device, queue_order):
    """A wrapped ring window (strided [Hq, W, d] views) scores, selects and compacts exactly as
    contiguous copies of the same queries do."""
    head_lengths = [[400, 380, 35, 410], [390, 10, 400, 402]]
    groups, dim, window = 4, 128, 80
    layers, _ = workloads.make_layers(head_lengths, groups, dim, window, device, seed=21)
    hq = len(head_lengths[0]) * groups
    history = QueryHistory(len(layers), window)
    gen = torch.Generator(device=device).manual_seed(21)
    for step in range(window + 17):   # wraps: the window starts mid-ring
        history.append([torch.randn((1, hq, 1, dim), generator=gen, device=device)
                        .to(torch.bfloat16) for _ in layers], 300 + step)
    views, positions = history.audit_window()
    assert views[0].stride(0) == 2 * window * dim and not views[0].is_contiguous()
    ring_layers = [dataclasses.replace(layer, queries=view) for layer, view in zip(layers, views)]
    copy_layers = [dataclasses.replace(layer, queries=view.contiguous())
                   for layer, view in zip(layers, views)]
    margin = torch.tensor([2.0], device=device)
    step = audit.AuditStep()
    for native in (True, False):
        a = step.run(ring_layers, positions, margin, 500, queue_order=queue_order, native=native)
        b = step.run(copy_layers, positions.clone(), margin, 500, queue_order=queue_order,
                     native=native)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(a.scores.cpu().numpy(), b.scores.cpu().numpy())
        assert a.head_lens == b.head_lens and a.removed == b.removed
        for x, y in zip(a.layers, b.layers):
            assert torch.equal(x.keys, y.keys) and torch.equal(x.positions, y.positions)
        if queue_order:
            np.testing.assert_array_equal(a.selection.references().positions,
                                          b.selection.references().positions)
