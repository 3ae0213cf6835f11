"""GPU parity of the data-movement ops against the oracle: bit-exact for every dtype, row
width (16/8/4/2-byte granules), ragged layout and edge case the reference handles."""

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _C, _legacy_C, _lib
from oracle import kv_ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32, torch.float64]
INT_VIEW = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32,
            torch.float64: torch.int64}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern on the host (bit-exact comparison, NaN-safe)."""
    t = t.detach().contiguous()
    return t.view(INT_VIEW.get(t.dtype, t.dtype)).cpu().numpy() if t.dtype in INT_VIEW else t.cpu().numpy()


def rand(shape, dtype, device, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(device)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", [128, 64, 96, 3, 1])
@pytest.mark.parametrize("pattern", ["random", "none", "all", "runs", "ends"])
def test_compact(device, dtype, dim, pattern):
    rows = 8 * 301
    keys, values = rand((rows, dim), dtype, device, 1), rand((rows, dim), dtype, device, 2)
    positions = torch.randperm(rows, generator=torch.Generator().manual_seed(3)).float().to(device)[:, None]
    rng = np.random.default_rng(dim)
    removed = {"random": np.sort(rng.choice(rows, rows // 9, replace=False)),
               "none": np.zeros(0, np.int64), "all": np.arange(rows),
               "runs": np.concatenate([np.arange(10, 60), np.arange(700, 1300)]),
               "ends": np.asarray([0, 1, rows - 2, rows - 1])}[pattern].astype(np.int64)
    got = _C.compact(keys, values, positions, torch.from_numpy(removed).to(device))
    expect = kv_ops.compact(bits(keys), bits(values), bits(positions), removed)
    for g, e in zip(got, expect):
        np.testing.assert_array_equal(bits(g).reshape(e.shape), e)
    assert got[2].shape == (rows - removed.size, 1)


def test_compact_llama8b_layer(device):
    """One cfg1 layer: 8 heads x 2250 rows, d=128, 250 evicted per head."""
    lengths = [2250] * 8
    rows = sum(lengths)
    keys, values = rand((rows, 128), torch.bfloat16, device, 4), rand((rows, 128), torch.bfloat16, device, 5)
    positions = torch.cat([torch.arange(n) for n in lengths]).float().to(device)[:, None]
    rng = np.random.default_rng(0)
    removed = np.sort(np.concatenate([h * 2250 + rng.choice(2218, 250, replace=False) for h in range(8)]))
    got = _C.compact(keys, values, positions, torch.from_numpy(removed).to(device))
    expect = kv_ops.compact(bits(keys), bits(values), bits(positions), removed)
    for g, e in zip(got, expect):
        np.testing.assert_array_equal(bits(g).reshape(e.shape), e)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dim", [128, 64, 3])
def test_compact_heads(device, dtype, dim):
    """lr_compact_heads over ragged head slots: several 256-row output chunks per head, a
    removal list longer than the LDS-staged limit (4096), a head without a score segment, a
    head losing every row, an empty head; packed in head-slot order."""
    from code_for_iclr27_amd import _lib

    rng = np.random.default_rng(dim)
    lengths = [700, 9000, 0, 300, 257, 1]
    segment_of = [0, 1, -1, 2, 3, -1]
    removals = {0: np.sort(rng.choice(700, 90, replace=False)),
                1: np.sort(rng.choice(9000, 5000, replace=False)),
                2: np.arange(300),
                3: np.asarray([0, 255, 256])}
    keys = [rand((n, dim), dtype, device, 40 + h) for h, n in enumerate(lengths)]
    values = [rand((n, dim), dtype, device, 50 + h) for h, n in enumerate(lengths)]
    positions = [torch.from_numpy(rng.permutation(n).astype(np.float32)).to(device) for n in lengths]
    table = np.zeros((len(lengths), 6), np.int64)
    for h, n in enumerate(lengths):
        table[h, :5] = [keys[h].data_ptr(), values[h].data_ptr(), positions[h].data_ptr(), n,
                        segment_of[h]]
    quotas = np.asarray([len(removals[s]) for s in range(4)], np.int64)
    offsets = np.concatenate(([0], np.cumsum(quotas)[:-1])).astype(np.int64)
    flat = np.concatenate([removals[s] for s in range(4)]).astype(np.int64)
    out_rows = sum(lengths) - int(quotas.sum())
    out_k = torch.empty((out_rows, dim), dtype=dtype, device=device)
    out_v = torch.empty_like(out_k)
    out_p = torch.empty((out_rows,), dtype=torch.float32, device=device)
    on = lambda a: torch.from_numpy(a).to(device)
    table_d, quotas_d, offsets_d, flat_d = on(table), on(quotas), on(offsets), on(flat)
    _lib.call("lr_compact_heads", table_d.data_ptr(), len(lengths), quotas_d.data_ptr(),
              offsets_d.data_ptr(), flat_d.data_ptr(), dim, out_k.element_size(), max(lengths),
              out_rows, out_k.data_ptr(), out_v.data_ptr(), out_p.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    expect_k, expect_v, expect_p = [], [], []
    for h, n in enumerate(lengths):
        gone = removals[segment_of[h]] if segment_of[h] >= 0 else np.zeros(0, np.int64)
        ek, ev, ep = kv_ops.compact(bits(keys[h]), bits(values[h]), positions[h].cpu().numpy(),
                                    gone.astype(np.int64))
        expect_k.append(ek), expect_v.append(ev), expect_p.append(ep.reshape(-1))
    np.testing.assert_array_equal(bits(out_k), np.concatenate(expect_k))
    np.testing.assert_array_equal(bits(out_v), np.concatenate(expect_v))
    np.testing.assert_array_equal(out_p.cpu().numpy(), np.concatenate(expect_p))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("added", [1, 3])
@pytest.mark.parametrize("dim", [128, 5])
def test_append(device, dtype, added, dim):
    lengths = [7, 0, 300, 1, 64, 2, 9, 33]
    heads = len(lengths)
    rows = sum(lengths)
    keys, values = rand((rows, dim), dtype, device, 6), rand((rows, dim), dtype, device, 7)
    positions = torch.arange(rows).float().to(device)[:, None]
    new_k = rand((1, heads, added, dim), dtype, device, 8)
    new_v = rand((1, heads, added, dim), dtype, device, 9)
    cumulative = torch.tensor(np.concatenate(([0], np.cumsum(lengths))), dtype=torch.int32, device=device)
    got = _C.append(keys, values, positions, new_k, new_v, cumulative, 4242, max(lengths))
    expect = kv_ops.append(bits(keys), bits(values), bits(positions).view(np.float32), bits(new_k),
                           bits(new_v), cumulative.cpu().numpy(), 4242, max(lengths))
    np.testing.assert_array_equal(bits(got[0]), expect[0])
    np.testing.assert_array_equal(bits(got[1]), expect[1])
    np.testing.assert_array_equal(got[2].cpu().numpy(), expect[2])
    np.testing.assert_array_equal(got[3].cpu().numpy(), expect[3])
    np.testing.assert_array_equal(got[4].cpu().numpy(), expect[4])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("added,max_length", [(1, 40), (3, 63), (2, 0)])
def test_append_rows_beyond_max_length_stay_unwritten(device, dtype, added, max_length):
    """maximum_length sizes the grid as in the reference (csrc/scoring.cu:264-292): a head keeps
    only its first maximum_length + added rows, old rows first. Through the C-ABI into zeroed
    outputs, so the rows it must not write read as the oracle's zeros."""
    lengths, dim = [7, 0, 300, 1, 64, 2, 9, 33], 128
    heads, rows = len(lengths), sum(lengths)
    keys, values = rand((rows, dim), dtype, device, 16), rand((rows, dim), dtype, device, 17)
    positions = torch.arange(rows).float().to(device)[:, None] + 0.25
    new_k = rand((1, heads, added, dim), dtype, device, 18)
    new_v = rand((1, heads, added, dim), dtype, device, 19)
    cumulative = torch.tensor(np.concatenate(([0], np.cumsum(lengths))), dtype=torch.int32, device=device)
    out_rows = rows + heads * added
    out_k = torch.zeros((out_rows, dim), dtype=dtype, device=device)
    out_v = torch.zeros((out_rows, dim), dtype=dtype, device=device)
    out_p = torch.zeros((out_rows, 1), device=device)
    out_c = torch.zeros(heads + 1, dtype=torch.int32, device=device)
    out_l = torch.zeros(heads, dtype=torch.int32, device=device)
    _lib.call("lr_append", keys.data_ptr(), values.data_ptr(), positions.data_ptr(), rows,
              new_k.data_ptr(), new_v.data_ptr(), cumulative.data_ptr(), heads, added, dim,
              keys.element_size(), 777, max_length, out_k.data_ptr(), out_v.data_ptr(),
              out_p.data_ptr(), out_c.data_ptr(), out_l.data_ptr(), _lib.stream_of(keys))
    expect = kv_ops.append(bits(keys), bits(values), positions.cpu().numpy(), bits(new_k),
                           bits(new_v), cumulative.cpu().numpy(), 777, max_length)
    np.testing.assert_array_equal(bits(out_k), expect[0])
    np.testing.assert_array_equal(bits(out_v), expect[1])
    np.testing.assert_array_equal(out_p.cpu().numpy(), expect[2])
    np.testing.assert_array_equal(out_c.cpu().numpy(), expect[3])
    np.testing.assert_array_equal(out_l.cpu().numpy(), expect[4])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("added,dim", [(1, 128), (3, 64), (2, 3)])
def test_append_layers_matches_per_layer_append(device, dtype, added, dim):
    """One launch for every layer (packed outputs) equals the oracle's per-layer append, with
    per-layer lengths (an empty layer and empty heads included) and logical starts."""
    heads = 8
    layer_lengths = [[7, 0, 300, 1, 64, 2, 9, 33], [0] * heads, [250] * heads,
                     [1, 2, 3, 4, 5, 6, 7, 8]]
    args = {name: [] for name in ("keys", "values", "positions", "new_k", "new_v", "cumulative")}
    starts = [4242, 4241, 17, 0]
    for l, lengths in enumerate(layer_lengths):
        rows = sum(lengths)
        args["keys"].append(rand((rows, dim), dtype, device, 20 + l))
        args["values"].append(rand((rows, dim), dtype, device, 40 + l))
        args["positions"].append(torch.arange(rows).float().to(device)[:, None] * 2 + l)
        args["new_k"].append(rand((1, heads, added, dim), dtype, device, 60 + l))
        args["new_v"].append(rand((1, heads, added, dim), dtype, device, 80 + l))
        args["cumulative"].append(torch.tensor(np.concatenate(([0], np.cumsum(lengths))),
                                               dtype=torch.int32, device=device))
    maximum = max(max(lengths) for lengths in layer_lengths)
    keys, values, positions, cumulative, lengths_out, first = _C.append_layers(
        args["keys"], args["values"], args["positions"], args["new_k"], args["new_v"],
        args["cumulative"], starts, maximum)
    for l in range(len(layer_lengths)):
        expect = kv_ops.append(bits(args["keys"][l]), bits(args["values"][l]),
                               bits(args["positions"][l]).view(np.float32), bits(args["new_k"][l]),
                               bits(args["new_v"][l]), args["cumulative"][l].cpu().numpy(),
                               starts[l], maximum)
        rows = slice(first[l], first[l + 1])
        np.testing.assert_array_equal(bits(keys[rows]), expect[0])
        np.testing.assert_array_equal(bits(values[rows]), expect[1])
        np.testing.assert_array_equal(positions[rows].cpu().numpy(), expect[2])
        np.testing.assert_array_equal(cumulative[l].cpu().numpy(), expect[3])
        np.testing.assert_array_equal(lengths_out[l].cpu().numpy(), expect[4])
    with pytest.raises(RuntimeError, match="Invalid cumulative lengths"):
        _C.append_layers(args["keys"], args["values"], args["positions"], args["new_k"],
                         args["new_v"], args["cumulative"][:-1] + [args["cumulative"][0][:3]],
                         starts, maximum)


def _append_layer_inputs(layer_lengths, heads, added, dim, device, seed):
    args = {name: [] for name in ("keys", "values", "positions", "new_k", "new_v", "cumulative")}
    for l, lengths in enumerate(layer_lengths):
        rows = sum(lengths)
        args["keys"].append(rand((rows, dim), torch.bfloat16, device, seed + 3 * l))
        args["values"].append(rand((rows, dim), torch.bfloat16, device, seed + 3 * l + 1))
        args["positions"].append(torch.arange(rows).float().to(device)[:, None] + l)
        args["new_k"].append(rand((1, heads, added, dim), torch.bfloat16, device, seed + 3 * l + 2))
        args["new_v"].append(rand((1, heads, added, dim), torch.bfloat16, device, seed + 3 * l + 3))
        args["cumulative"].append(torch.tensor(np.concatenate(([0], np.cumsum(lengths))),
                                               dtype=torch.int32, device=device))
    return args


def test_append_layers_beyond_the_inline_table(device):
    """50 layers: more than the 48 whose table travels in the kernel arguments, so the table goes
    up as a device copy; every layer bit-exact against the oracle's per-layer append."""
    heads, added, dim = 2, 1, 64
    layer_lengths = [[(7 * l) % 13, (3 * l + 1) % 11] for l in range(50)]
    args = _append_layer_inputs(layer_lengths, heads, added, dim, device, 300)
    starts = [1000 + l for l in range(50)]
    maximum = max(max(lengths) for lengths in layer_lengths)
    keys, values, positions, cumulative, lengths_out, first = _C.append_layers(
        args["keys"], args["values"], args["positions"], args["new_k"], args["new_v"],
        args["cumulative"], starts, maximum)
    for l in range(50):
        expect = kv_ops.append(bits(args["keys"][l]), bits(args["values"][l]),
                               bits(args["positions"][l]).view(np.float32), bits(args["new_k"][l]),
                               bits(args["new_v"][l]), args["cumulative"][l].cpu().numpy(),
                               starts[l], maximum)
        rows = slice(first[l], first[l + 1])
        np.testing.assert_array_equal(bits(keys[rows]), expect[0])
        np.testing.assert_array_equal(bits(values[rows]), expect[1])
        np.testing.assert_array_equal(positions[rows].cpu().numpy(), expect[2])
        np.testing.assert_array_equal(cumulative[l].cpu().numpy(), expect[3])
        np.testing.assert_array_equal(lengths_out[l].cpu().numpy(), expect[4])


def test_append_layers_host_table_through_the_abi(device):
    """lr_append_layers_host (the table in the launch's kernel arguments) against
    lr_append_layers (the same table in device memory), bit-exact, with the host table
    overwritten right after the call while the device is still held (the overwrite describes
    the same layers with other logical starts, so a late read would change the positions)."""
    heads, added, dim, L = 8, 1, 128, 32
    layer_lengths = [[40 + (5 * l + h) % 17 for h in range(heads)] for l in range(L)]
    args = _append_layer_inputs(layer_lengths, heads, added, dim, device, 500)
    table = np.zeros((L, 12), dtype=np.int64)
    total = 0
    for l, lengths in enumerate(layer_lengths):
        table[l, :9] = [args["keys"][l].data_ptr(), args["values"][l].data_ptr(),
                        args["positions"][l].data_ptr(), sum(lengths), args["cumulative"][l].data_ptr(),
                        args["new_k"][l].data_ptr(), args["new_v"][l].data_ptr(), 2000 + l, total]
        total += sum(lengths) + heads * added
    maximum = max(max(lengths) for lengths in layer_lengths)
    outs = [(torch.empty((total, dim), dtype=torch.bfloat16, device=device),
             torch.empty((total, dim), dtype=torch.bfloat16, device=device),
             torch.empty((total, 1), device=device),
             torch.empty((L, heads + 1), dtype=torch.int32, device=device),
             torch.empty((L, heads), dtype=torch.int32, device=device)) for _ in range(2)]
    stream = _lib.stream_of(args["keys"][0])
    device_table = torch.from_numpy(table.copy()).to(device)
    ptrs = lambda o: [t.data_ptr() for t in o]
    _lib.call("lr_append_layers", device_table.data_ptr(), L, heads, added, dim, 2, maximum,
              *ptrs(outs[0]), stream)
    torch.cuda._sleep(5_000_000)
    _lib.call("lr_append_layers_host", table.ctypes.data, L, heads, added, dim, 2, maximum,
              *ptrs(outs[1]), stream)
    table[:, 7] += 77
    torch.cuda.synchronize()
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(bits(a) if a.dtype == torch.bfloat16 else a.cpu().numpy(),
                                      bits(b) if b.dtype == torch.bfloat16 else b.cpu().numpy())
    expect = kv_ops.append(bits(args["keys"][3]), bits(args["values"][3]),
                           bits(args["positions"][3]).view(np.float32), bits(args["new_k"][3]),
                           bits(args["new_v"][3]), args["cumulative"][3].cpu().numpy(), 2003,
                           maximum)
    rows = slice(int(table[3, 8]), int(table[4, 8]))
    np.testing.assert_array_equal(bits(outs[1][0][rows]), expect[0])
    np.testing.assert_array_equal(outs[1][2][rows].cpu().numpy(), expect[2])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 8, 1, 1), (2, 4, 3, 128), (1, 8, 2, 64)])
def test_append_flattened_cache(device, dtype, shape):
    batch, heads, new, dim = shape
    lengths = [(5 * i + 3) % 17 for i in range(batch * heads)]
    cache = rand((sum(lengths), dim), dtype, device, 10)
    states = rand(shape, dtype, device, 11)
    head_lens = torch.tensor(lengths, dtype=torch.int32, device=device)
    cu = torch.tensor(np.concatenate(([0], np.cumsum(lengths))), dtype=torch.int32, device=device)
    got = _legacy_C.append_flattened_cache(cache, states, head_lens, cu)
    expect = kv_ops.append_flattened_cache(bits(cache), bits(states), lengths)
    np.testing.assert_array_equal(bits(got), expect)


@pytest.mark.parametrize("dtype", DTYPES)
def test_compact_flattened_kv(device, dtype):
    keys, values = rand((500, 72), dtype, device, 12), rand((500, 72), dtype, device, 13)
    keep = np.random.default_rng(1).choice(500, 333, replace=True).astype(np.int64)
    got = _legacy_C.compact_flattened_kv(keys, values, torch.from_numpy(keep).to(device))
    expect = kv_ops.compact_flattened_kv(bits(keys), bits(values), keep)
    np.testing.assert_array_equal(bits(got[0]), expect[0])
    np.testing.assert_array_equal(bits(got[1]), expect[1])
    empty = _legacy_C.compact_flattened_kv(keys, values, torch.zeros(0, dtype=torch.long, device=device))
    assert empty[0].shape == (0, 72)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_merge_with_plan(device, dtype):
    rng = np.random.default_rng(5)
    heads, dim, per_head, recalled_per_head = 4, 128, 400, 37
    old_pos, meta = [], []
    for h in range(heads):
        universe = rng.permutation(2000)[:per_head + recalled_per_head]
        old_pos.append(np.sort(universe[:per_head]))
        meta.extend((3, h, p) for p in universe[per_head:])
    old_pos = np.concatenate(old_pos)
    meta = np.asarray(meta, dtype=np.int64)[rng.permutation(len(meta))]
    mapping, lengths = kv_ops.merge_plan(old_pos, [per_head] * heads, meta)
    keys, values = rand((old_pos.size, dim), dtype, device, 14), rand((old_pos.size, dim), dtype, device, 15)
    positions = torch.from_numpy(old_pos.astype(np.float32)).to(device)[:, None]
    recalled = rand((len(meta), 2, dim), dtype, device, 16)
    recalled_pos = torch.from_numpy(meta[:, 2].astype(np.float32)).to(device)
    got = _C.merge(keys, values, positions, recalled, recalled_pos, torch.from_numpy(mapping).to(device))
    expect = kv_ops.merge(bits(keys), bits(values), old_pos.astype(np.float32), bits(recalled),
                          meta[:, 2].astype(np.float32), mapping)
    np.testing.assert_array_equal(bits(got[0]), expect[0])
    np.testing.assert_array_equal(bits(got[1]), expect[1])
    np.testing.assert_array_equal(got[2].cpu().numpy(), expect[2])
    start = 0
    for n in lengths:
        assert np.all(np.diff(got[2][start:start + n, 0].cpu().numpy()) > 0)
        start += n


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_into_staging_view(device, dtype):
    keys, values = rand((900, 128), dtype, device, 17), rand((900, 128), dtype, device, 18)
    positions = (torch.arange(900).float() * 3 + 0.75).to(device)[:, None]
    archive = torch.zeros((2, 64, 2, 128), dtype=dtype, device=device)
    archive_meta = torch.full((2, 64, 3), -1, dtype=torch.int64, device=device)
    indices = np.asarray([5, 899, 0, 450, 451, 17], dtype=np.int64)
    heads = np.asarray([0, 7, 0, 3, 3, 1], dtype=np.int64)
    _C.pack(keys, values, positions, torch.from_numpy(indices).to(device),
            torch.from_numpy(heads).to(device), 11, archive[1, 10:16], archive_meta[1, 10:16])
    payload, meta = kv_ops.pack(bits(keys), bits(values), positions.cpu().numpy(), indices, heads, 11)
    np.testing.assert_array_equal(bits(archive[1, 10:16]), payload)
    np.testing.assert_array_equal(archive_meta[1, 10:16].cpu().numpy(), meta)
    assert int((archive_meta[0] != -1).sum()) == 0 and int((archive_meta[1, :10] != -1).sum()) == 0


@pytest.mark.parametrize("case,message", [
    ("short", "Head lengths do not cover cache rows"),
    ("negative", "Invalid head length"),
    ("overrun", "Invalid head length"),
    ("logical", "Invalid positions or head metadata"),
    ("heads", "Invalid positions or head metadata"),
    ("dtype", "Cache K/V mismatch"),
    ("cpu", "Contiguous CUDA cache required"),
])
def test_batch_append_rejects_bad_metadata(device, case, message):
    """The descriptor checks of csrc/batch_append.cu:49-80 (the host planner raises them
    before anything is launched)."""
    heads, dim = 2, 64
    lengths = [[3, 4], [5, 0]]
    keys = [rand((sum(l), dim), torch.bfloat16, device, 60 + r) for r, l in enumerate(lengths)]
    values = [rand((sum(l), dim), torch.bfloat16, device, 70 + r) for r, l in enumerate(lengths)]
    positions = [torch.zeros((sum(l), 1), device=device) for l in lengths]
    logical = [10, 11]
    if case == "short":
        lengths = [[3, 3], [5, 0]]
    elif case == "negative":
        lengths = [[3, 4], [6, -1]]
    elif case == "overrun":
        lengths = [[3, 5], [5, 0]]
    elif case == "logical":
        logical = [10, 1 << 24]
    elif case == "heads":
        lengths = [[3, 4], [5]]
    elif case == "dtype":
        values[1] = values[1].float()
    elif case == "cpu":
        keys[0] = keys[0].cpu()
    nk = rand((2, heads, 1, dim), torch.bfloat16, device, 80)
    nv = rand((2, heads, 1, dim), torch.bfloat16, device, 81)
    with pytest.raises(RuntimeError, match=message):
        _C.batch_append(keys, values, positions, nk, nv, lengths, logical)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_batch_append_over_packed_views(device, dtype):
    """Requests' caches are views into the previous packed output, as append_packed leaves
    them (batch_attention.py:54-63); a retired request shrinks the next batch."""
    heads, dim = 8, 128
    rng = np.random.default_rng(6)
    lengths = [list(rng.integers(0, 90, heads)) for _ in range(3)]
    lengths[1][2] = 0
    keys = [rand((int(sum(l)), dim), dtype, device, 20 + r) for r, l in enumerate(lengths)]
    values = [rand((int(sum(l)), dim), dtype, device, 30 + r) for r, l in enumerate(lengths)]
    positions = [torch.arange(int(sum(l))).float().to(device)[:, None] for l in lengths]
    for step in range(3):
        requests = len(keys)
        nk = rand((requests, heads, 1, dim), dtype, device, 40 + step)
        nv = rand((requests, heads, 1, dim), dtype, device, 50 + step)
        logical = [1000 + 10 * r + step for r in range(requests)]
        pk, pv, pp = _C.batch_append(keys, values, positions, nk, nv, lengths, logical)
        ek, ev, ep = kv_ops.batch_append([bits(k) for k in keys], [bits(v) for v in values],
                                         [p.cpu().numpy() for p in positions], bits(nk), bits(nv),
                                         lengths, logical)
        np.testing.assert_array_equal(bits(pk), ek)
        np.testing.assert_array_equal(bits(pv), ev)
        np.testing.assert_array_equal(pp.cpu().numpy(), ep)
        start, keys, values, positions = 0, [], [], []
        new_lengths = []
        for r, head_lengths in enumerate(lengths):
            end = start + int(sum(head_lengths)) + heads
            if not (step == 0 and r == 1):  # request 1 hits EOS after the first step
                keys.append(pk[start:end])
                values.append(pv[start:end])
                positions.append(pp[start:end])
                new_lengths.append([int(x) + 1 for x in head_lengths])
            start = end
        lengths = new_lengths


def test_batch_append_staging_ring_reuse(device):
    """Tables of more than 64 (request, head) descriptors go through a ring of 64 host-coherent
    buffers, one event per up to 8 consecutive buffers of one stream. 150 calls of 72 segments
    while the device is held, switching between two streams every 5 calls, so the host reuses
    buffers whose readers are still queued and must wait for the right event. Every call has the
    same lengths (a stale descriptor would only point at another call's inputs), and every
    output is bit-exact for its own inputs."""
    heads, dim, calls, requests = 8, 16, 150, 9
    lengths = [[(3 * r + h) % 6 for h in range(heads)] for r in range(requests)]
    rows = [int(sum(l)) for l in lengths]
    inputs = []
    for i in range(calls):
        keys = [rand((n, dim), torch.bfloat16, device, 100000 + 16 * i + r) for r, n in enumerate(rows)]
        values = [rand((n, dim), torch.bfloat16, device, 200000 + 16 * i + r) for r, n in enumerate(rows)]
        positions = [(torch.arange(n).float() + i).to(device)[:, None] for n in rows]
        nk = rand((requests, heads, 1, dim), torch.bfloat16, device, 3000 + i)
        nv = rand((requests, heads, 1, dim), torch.bfloat16, device, 4000 + i)
        inputs.append((keys, values, positions, nk, nv, [100 * r + i for r in range(requests)]))
    torch.cuda.synchronize()
    streams = [torch.cuda.current_stream(device), torch.cuda.Stream(device)]
    for stream in streams:
        with torch.cuda.stream(stream):
            torch.cuda._sleep(5_000_000)
    outputs = []
    for i, (keys, values, positions, nk, nv, logical) in enumerate(inputs):
        with torch.cuda.stream(streams[(i // 5) % 2]):
            outputs.append(_C.batch_append(keys, values, positions, nk, nv, lengths, logical))
    torch.cuda.synchronize()
    for (keys, values, positions, nk, nv, logical), (pk, pv, pp) in zip(inputs, outputs):
        ek, ev, ep = kv_ops.batch_append([bits(k) for k in keys], [bits(v) for v in values],
                                         [p.cpu().numpy() for p in positions], bits(nk), bits(nv),
                                         lengths, logical)
        np.testing.assert_array_equal(bits(pk), ek)
        np.testing.assert_array_equal(bits(pv), ev)
        np.testing.assert_array_equal(pp.cpu().numpy(), ep)


def _descriptor_table(keys, values, positions, lengths, logical):
    """The 7-word rows of csrc/batch_append.cu:49-80 for device inputs."""
    table, destination = [], 0
    for r, head_lengths in enumerate(lengths):
        source = 0
        for n in head_lengths:
            table.append([keys[r].data_ptr(), values[r].data_ptr(), positions[r].data_ptr(),
                          source, int(n), destination, logical[r]])
            source += int(n)
            destination += int(n) + 1
    return np.asarray(table, dtype=np.int64), destination


@pytest.mark.parametrize("requests,heads", [(1, 1), (8, 8)])
def test_batch_append_host_descriptors_through_the_abi(device, requests, heads):
    """lr_batch_append_host (descriptors in the launch's kernel arguments) against
    lr_batch_append (the same table in device memory) and the oracle, bit-exact. The host table
    is overwritten right after the call while the device is still held: the overwrite describes
    a second, valid set of inputs of the same shape, so a late read of the table would show up
    as that set's rows."""
    dim = 128
    rng = np.random.default_rng(requests * 100 + heads)
    lengths = [list(rng.integers(0, 40, heads)) for _ in range(requests)]
    sets = []
    for k in range(2):
        keys = [rand((int(sum(l)), dim), torch.bfloat16, device, 10 * k + r) for r, l in enumerate(lengths)]
        values = [rand((int(sum(l)), dim), torch.bfloat16, device, 50 + 10 * k + r) for r, l in enumerate(lengths)]
        positions = [(torch.arange(int(sum(l))).float() + 0.5 + k).to(device)[:, None] for l in lengths]
        logical = [300 + r + k for r in range(requests)]
        sets.append((keys, values, positions, logical))
    nk = rand((requests, heads, 1, dim), torch.bfloat16, device, 90)
    nv = rand((requests, heads, 1, dim), torch.bfloat16, device, 91)
    keys, values, positions, logical = sets[0]
    table, rows = _descriptor_table(keys, values, positions, lengths, logical)
    other, _ = _descriptor_table(*sets[1][:3], lengths, sets[1][3])
    segments = requests * heads
    max_rows = max(int(n) + 1 for l in lengths for n in l)
    outs = [(torch.empty((rows, dim), dtype=torch.bfloat16, device=device),
             torch.empty((rows, dim), dtype=torch.bfloat16, device=device),
             torch.empty((rows, 1), dtype=torch.float32, device=device)) for _ in range(2)]
    stream = _lib.stream_of(nk)
    device_table = torch.from_numpy(table.copy()).to(device)
    _lib.call("lr_batch_append", device_table.data_ptr(), segments, nk.data_ptr(), nv.data_ptr(),
              dim, 2, max_rows, outs[0][0].data_ptr(), outs[0][1].data_ptr(),
              outs[0][2].data_ptr(), stream)
    torch.cuda._sleep(5_000_000)
    _lib.call("lr_batch_append_host", table.ctypes.data, segments, nk.data_ptr(), nv.data_ptr(),
              dim, 2, max_rows, outs[1][0].data_ptr(), outs[1][1].data_ptr(),
              outs[1][2].data_ptr(), stream)
    table[...] = other
    torch.cuda.synchronize()
    ek, ev, ep = kv_ops.batch_append([bits(k) for k in keys], [bits(v) for v in values],
                                     [p.cpu().numpy() for p in positions], bits(nk), bits(nv),
                                     lengths, logical)
    for pk, pv, pp in outs:
        np.testing.assert_array_equal(bits(pk), ek)
        np.testing.assert_array_equal(bits(pv), ev)
        np.testing.assert_array_equal(pp.cpu().numpy(), ep)


def test_batch_append_descriptors_beyond_a_staging_share(device):
    """1,200 (request, head) descriptors (67 KB, more than a staging buffer's first 64 KB share)
    in two consecutive calls: the buffers grow on their own, outputs bit-exact."""
    heads, dim, requests = 8, 16, 150
    rng = np.random.default_rng(12)
    for call in range(2):
        lengths = [list(rng.integers(0, 4, heads)) for _ in range(requests)]
        keys = [rand((int(sum(l)), dim), torch.bfloat16, device, 500 + r) for r, l in enumerate(lengths)]
        values = [rand((int(sum(l)), dim), torch.bfloat16, device, 700 + r) for r, l in enumerate(lengths)]
        positions = [torch.arange(int(sum(l))).float().to(device)[:, None] for l in lengths]
        nk = rand((requests, heads, 1, dim), torch.bfloat16, device, 900 + call)
        nv = rand((requests, heads, 1, dim), torch.bfloat16, device, 901 + call)
        logical = [50 + r for r in range(requests)]
        pk, pv, pp = _C.batch_append(keys, values, positions, nk, nv, lengths, logical)
        ek, ev, ep = kv_ops.batch_append([bits(k) for k in keys], [bits(v) for v in values],
                                         [p.cpu().numpy() for p in positions], bits(nk), bits(nv),
                                         lengths, logical)
        np.testing.assert_array_equal(bits(pk), ek)
        np.testing.assert_array_equal(bits(pv), ev)
        np.testing.assert_array_equal(pp.cpu().numpy(), ep)


@pytest.mark.parametrize("width", [1, 3, 7, 9, 4099])
def test_pool(device, width):
    rng = np.random.default_rng(width)
    lengths = [1, 2218, 5, 2, 700, 4500]
    ends = np.cumsum(lengths)
    scores = rng.standard_normal(ends[-1]).astype(np.float32)
    scores[100:140] = 0.5  # plateau
    scores[2000] = np.nan
    bounds = np.concatenate(([0], ends)).astype(np.int64)
    got = _C.pool(torch.from_numpy(scores).to(device), torch.from_numpy(bounds).to(device),
                  max(lengths), width)
    expect = kv_ops.pool(scores, bounds, width)
    np.testing.assert_array_equal(got.cpu().numpy(), expect)


def test_validation_messages(device):
    keys = torch.zeros((4, 8), dtype=torch.bfloat16, device=device)
    positions = torch.zeros((4, 1), device=device)
    with pytest.raises(RuntimeError, match="Invalid removals"):
        _C.compact(keys, keys, positions, torch.zeros(5, dtype=torch.long, device=device))
    with pytest.raises(RuntimeError, match="Invalid pool configuration"):
        _C.pool(torch.zeros(4, device=device), torch.tensor([0, 4], device=device), 4, 2)
    with pytest.raises(RuntimeError, match="Mapping must be int64"):
        _C.merge(keys, keys, positions, torch.zeros((1, 2, 8), dtype=torch.bfloat16, device=device),
                 torch.zeros(1, device=device), torch.zeros(5, dtype=torch.int32, device=device))


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes", [16, 16 * 1023, 16 * 1024, 16 * 4097 + 16 * 3, 37 << 20])
def test_stream_copy(device, nbytes):
    """The calibration copy (nontemporal loads and stores) is an exact byte copy, including a
    partial last block, and leaves the bytes after the range alone."""
    generator = torch.Generator(device="cpu").manual_seed(nbytes)
    source = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=generator).to(device)
    target = torch.zeros((nbytes + 64,), dtype=torch.uint8, device=device)
    _lib.call("lr_stream_copy", source.data_ptr(), target.data_ptr(), nbytes,
              torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize(device)
    assert torch.equal(target[:nbytes], source)
    assert int(target[nbytes:].count_nonzero()) == 0
