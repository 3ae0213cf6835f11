"""Reinsertion of recalled rows into every layer at once (code_for_iclr27_amd.reinsert, the
device plan + scatter merge) against the oracle: per layer, oracle kv_ops.merge_plan (the
reference's stable argsort per head) and kv_ops.merge, bit-exact on keys, values and positions,
with the new head lengths and each recalled entry's row in its merged head derived from the
oracle's mapping. Payloads from pinned host memory and from device memory, a PackedLayers
input, a layer and heads with nothing recalled, metadata in any order, duplicate identities
refused, and one full-size cfg3 reinsertion (32 layers x 8 heads x 33,792 + 512 per head)."""

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _lib, audit, reinsert, workloads
from code_for_iclr27_amd.scoring import LayerState
from oracle import kv_ops

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def make_case(device, head_lengths, recalled_per_head, dim, seed, skip_layer=None):
    """Resident positions: an ascending subset of 0..; recalled: the holes, shuffled."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    layers, meta = [], []
    for l, lengths in enumerate(head_lengths):
        pos_parts = []
        for h, n in enumerate(lengths):
            r = 0 if l == skip_layer else recalled_per_head[(l + h) % len(recalled_per_head)]
            universe = np.sort(rng.choice(n + r + 50, n + r, replace=False))
            holes = rng.choice(n + r, r, replace=False)
            keep = np.ones(n + r, bool)
            keep[holes] = False
            pos_parts.append(universe[keep])
            meta.extend((l, h, int(p)) for p in universe[~keep])
        rows = int(sum(lengths))
        keys = torch.randn((rows, dim), generator=gen).to(torch.bfloat16).to(device)
        values = torch.randn((rows, dim), generator=gen).to(torch.bfloat16).to(device)
        positions = torch.from_numpy(np.concatenate(pos_parts).astype(np.float32)).to(device)
        layers.append(LayerState(keys, values, positions, list(lengths), None, None, None))
    meta = np.asarray(meta, dtype=np.int64).reshape(-1, 3)
    meta = meta[rng.permutation(len(meta))]
    payload = torch.randn((len(meta), 2, dim), generator=gen).to(torch.bfloat16)
    return layers, payload, meta


def check(outcome, layers, payload, meta):
    payload_bits = payload.view(torch.int16).cpu().numpy()
    recalled_rows = outcome.recalled_rows.cpu().numpy()
    for l, layer in enumerate(layers):
        rows = np.flatnonzero(meta[:, 0] == l)
        old_pos = layer.positions.cpu().numpy().reshape(-1)
        mapping, lengths = kv_ops.merge_plan(old_pos, layer.head_lens, meta[rows])
        assert list(outcome.head_lens[l]) == list(lengths)
        ek, ev, ep = kv_ops.merge(bits(layer.keys), bits(layer.values), old_pos,
                                  payload_bits[rows], meta[rows, 2].astype(np.float32),
                                  np.asarray(mapping))
        got = outcome.layers[l]
        np.testing.assert_array_equal(bits(got.keys), ek)
        np.testing.assert_array_equal(bits(got.values), ev)
        np.testing.assert_array_equal(got.positions.cpu().numpy().reshape(-1), ep.reshape(-1))
        bounds = np.concatenate(([0], np.cumsum(lengths)))
        for out_row in np.flatnonzero(np.asarray(mapping) < 0):
            local = -int(mapping[out_row]) - 1
            head = int(meta[rows[local], 1])
            assert recalled_rows[rows[local]] == out_row - bounds[head]


def metadata_as(meta, form, device):
    """The identities as the host path takes them (numpy) or as the device-grouped path does
    (an int64 tensor in device or pinned host memory)."""
    if form == "host":
        return meta
    tensor = torch.from_numpy(np.ascontiguousarray(meta))
    return tensor.to(device) if form == "device" else tensor.pin_memory()


@pytest.mark.parametrize("meta_form", ["host", "device", "pinned"])
@pytest.mark.parametrize("on_device,grouped", [(False, False), (True, False), (False, True)])
def test_reinsert_matches_merge_plan(device, on_device, grouped, meta_form):
    """Identities in any order, or already grouped by (layer, head) in slot order (the host
    planner then copies instead of scattering them), with empty slots and a layer without
    recalls; grouped on the host or, from device or pinned metadata, on the device."""
    head_lengths = [[300, 41, 280, 1], [170, 300, 33, 299], [64, 200, 310, 90]]
    layers, payload, meta = make_case(device, head_lengths, [17, 0, 5, 129, 1], 128, seed=3,
                                      skip_layer=1)
    if grouped:
        order = np.argsort(meta[:, 0] * 4 + meta[:, 1], kind="stable")
        meta, payload = meta[order], payload[torch.from_numpy(order)]
    source = payload.to(device) if on_device else payload.pin_memory()
    outcome = reinsert.Reinserter().run(layers, source, metadata_as(meta, meta_form, device))
    torch.cuda.synchronize()
    assert outcome.inserted == len(meta)
    check(outcome, layers, payload, meta)


def test_reinsert_into_packed_layers_and_empty_batch(device):
    """The input is an audit's PackedLayers; then a reinsertion of nothing copies the layers."""
    layers, qpos = workloads.make_layers([[300, 260, 200], [180, 333, 250]], 4, 64, 32, device,
                                         seed=4)
    outcome = audit.AuditStep().run(layers, qpos, torch.tensor([2.0], device=device), 200)
    packed = outcome.layers
    # recall positions past every resident one (new tokens) and in the middle (holes)
    meta, rng = [], np.random.default_rng(5)
    for l in range(2):
        for h in range(3):
            start = sum(packed.kept[l][:h])
            resident = set(packed[l].positions[start:start + packed.kept[l][h]].cpu().numpy().astype(int).tolist())
            free = [p for p in range(0, 400) if p not in resident]
            meta.extend((l, h, int(p)) for p in rng.choice(free, 7, replace=False))
    meta = np.asarray(meta, np.int64)
    payload = torch.randn((len(meta), 2, 64)).to(torch.bfloat16)
    merged = reinsert.Reinserter().run(packed, payload.pin_memory(), meta)
    torch.cuda.synchronize()
    check(merged, [packed[l] for l in range(2)], payload, meta)
    empty = reinsert.Reinserter().run(merged.layers, torch.empty((0, 2, 64), dtype=torch.bfloat16),
                                      np.empty((0, 3), np.int64))
    for l in range(2):
        assert torch.equal(empty.layers[l].keys, merged.layers[l].keys)
        assert torch.equal(empty.layers[l].positions, merged.layers[l].positions)


@pytest.mark.parametrize("meta_form", ["host", "device"])
def test_reinsert_refuses_duplicates_and_bad_identities(device, meta_form):
    layers, payload, meta = make_case(device, [[100, 80]], [5], 64, seed=6)
    resident = int(layers[0].positions[3].item())
    bad = np.concatenate((meta, [[0, 0, resident]]))
    extra = torch.cat((payload, payload[:1]))
    runner = reinsert.Reinserter()
    with pytest.raises(ValueError, match="duplicate physical KV identities"):
        runner.run(layers, extra.pin_memory(), metadata_as(bad, meta_form, device))
    repeated = np.concatenate((meta, meta[:1]))
    with pytest.raises(ValueError, match="duplicate physical KV identities"):
        runner.run(layers, extra.pin_memory(), metadata_as(repeated, meta_form, device))
    for wrong in ([0, 2, 5], [1, 0, 5], [0, 0, -3]):
        with pytest.raises(ValueError, match="Invalid recall identity"):
            runner.run(layers, payload.pin_memory(),
                       metadata_as(np.concatenate((meta[:-1], [wrong])), meta_form, device))
    with pytest.raises(ValueError, match="shape mismatch"):
        runner.run(layers, payload[:-1].pin_memory(), metadata_as(meta, meta_form, device))
    # the same runner still merges correctly after the refusals
    outcome = runner.run(layers, payload.pin_memory(), metadata_as(meta, meta_form, device))
    torch.cuda.synchronize()
    check(outcome, layers, payload, meta)


@pytest.mark.parametrize("meta_form", ["host", "device"])
def test_reinsert_long_runs_sorted_both_ways(device, meta_form):
    """The plan sorts runs of up to 1,024 recalled rows by rank counting (one, two or four
    entries per thread) and longer ones with the bitonic network: heads with 2,000, 1,024, 700
    and 300 recalled rows, bit-exact against merge_plan and merge."""
    layers, payload, meta = make_case(device, [[300, 500, 200, 64]], [2000, 1024, 700, 300], 64,
                                      seed=9)
    outcome = reinsert.Reinserter().run(layers, payload.pin_memory(),
                                        metadata_as(meta, meta_form, device))
    torch.cuda.synchronize()
    check(outcome, layers, payload, meta)


def test_reinsert_device_grouped_head_limit(device):
    """More than LR_REINSERT_MAX_PER_HEAD recalled rows for one head: refused from the device
    flag, with every launch staying inside its buffers."""
    limit = _lib.LR_REINSERT_MAX_PER_HEAD
    layers, payload, meta = make_case(device, [[64, 32]], [limit + 3, 2], 64, seed=8)
    with pytest.raises(ValueError, match="Too many recalled rows for one head"):
        reinsert.Reinserter().run(layers, payload.pin_memory(),
                                  metadata_as(meta, "device", device))
    torch.cuda.synchronize()


def test_reinsert_full_size_cfg3(device):
    """cfg3: 32 layers x 8 KV heads x 33,792 resident rows, 512 recalled per head from pinned
    host memory; sampled layers bit-exact, every head's length and ascending positions."""
    L, H, d, T, M = 32, 8, 128, 33792, 512
    rng = np.random.default_rng(13)
    gen = torch.Generator(device=device).manual_seed(13)
    layers, meta = [], []
    for l in range(L):
        parts = []
        for h in range(H):
            holes = rng.choice(T + M, M, replace=False)
            keep = np.ones(T + M, bool)
            keep[holes] = False
            parts.append(np.flatnonzero(keep))
            meta.extend((l, h, int(p)) for p in holes)
        keys = torch.randn((H * T, d), generator=gen, device=device).to(torch.bfloat16)
        values = torch.randn((H * T, d), generator=gen, device=device).to(torch.bfloat16)
        positions = torch.from_numpy(np.concatenate(parts).astype(np.float32)).to(device)
        layers.append(LayerState(keys, values, positions, [T] * H, None, None, None))
    meta = np.asarray(meta, np.int64)
    payload = torch.randn((len(meta), 2, d), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    outcome = reinsert.Reinserter().run(layers, payload.pin_memory(),
                                        torch.from_numpy(meta).pin_memory())
    torch.cuda.synchronize()
    assert outcome.head_lens == [[T + M] * H] * L
    for l in range(L):
        merged = outcome.layers[l].positions.reshape(H, T + M).cpu().numpy()
        np.testing.assert_array_equal(merged, np.tile(np.arange(T + M, dtype=np.float32), (H, 1)))
    sampled = [0, 17, 31]
    rows = np.flatnonzero(np.isin(meta[:, 0], sampled))
    check_layers = [layers[l] for l in sampled]
    remapped = meta[rows].copy()
    remapped[:, 0] = np.searchsorted(sampled, remapped[:, 0])

    class Subset:
        def __init__(self, outcome):
            self.layers = [outcome.layers[l] for l in sampled]
            self.head_lens = [outcome.head_lens[l] for l in sampled]
            self.recalled_rows = outcome.recalled_rows[torch.from_numpy(rows).to(device)]

    check(Subset(outcome), check_layers, payload[torch.from_numpy(rows)], remapped)
