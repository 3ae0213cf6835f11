"""GPU parity of packed attention (the HIP kernel behind code_for_iclr27_amd.attention, called
through the C ABI) against the f64 oracle: decode over ragged per-(request, KV head) segments at
the cfg1/cfg2 shapes, d64/d128/d256, grouped queries with 1..8 groups, bf16 and f16, causal
prefill (square and with history, including segments shorter than the query block), strided
queries, edge lengths around the 16-key MFMA block and the key chunks, and repeated calls that
reuse the workspace.

Tolerance (floating point; the output is rounded to the 16-bit input type): every element within
one output ulp of the f64 result plus 1e-4 * max|V| (|got - ref| <= 2^-8|ref| + 1e-4 max|V| for
bf16, 2^-11|ref| + ... for f16), and at least 97% of the elements equal to the round-to-nearest
16-bit value of the f64 result.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import attention
from oracle import attention as oattention

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def make(device, batch, kv_heads, groups, length, dim, lengths, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    lengths = np.asarray(lengths, np.int64)
    assert lengths.size == batch * kv_heads
    total = int(lengths.sum())
    queries = torch.randn((batch, kv_heads * groups, length, dim), generator=g).to(dtype)
    keys = torch.randn((total, dim), generator=g).to(dtype)
    values = torch.randn((total, dim), generator=g).to(dtype)
    cumulative = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    metadata = SimpleNamespace(
        cu_seqlens_k=torch.from_numpy(cumulative).to(device),
        max_seqlen_k=int(lengths.max(initial=0)),
        decoding_cu_seqlens_q=torch.arange(batch * kv_heads + 1, dtype=torch.int32, device=device))
    return queries, keys, values, cumulative, metadata


def check(got, queries, keys, values, cumulative, kv_heads):
    expect = oattention.packed_attention(queries.float().numpy(), keys.float().numpy(),
                                         values.float().numpy(), cumulative, kv_heads)
    got32 = got.float().cpu().numpy()
    assert got.shape == expect.shape
    bound = ULP[got.dtype] * np.abs(expect) + 1e-4 * float(np.abs(values.float().numpy()).max(initial=0.0))
    error = np.abs(got32 - expect)
    assert np.all(error <= bound), float((error - bound).max())
    rounded = torch.from_numpy(expect).to(got.dtype).float().numpy()
    assert np.mean(got32 == rounded) >= 0.97


def run(device, queries, keys, values, metadata, length, kv_heads):
    return attention.packed_attention(queries.to(device), keys.to(device), values.to(device),
                                      metadata, length, kv_heads)


@pytest.mark.parametrize("shape", ["cfg1", "cfg2"])
def test_decode_llama_shapes(device, shape):
    rng = np.random.default_rng(5)
    batch = 1 if shape == "cfg1" else 8
    lengths = [2250] * 8 if shape == "cfg1" else rng.integers(1500, 2251, batch * 8)
    q, k, v, cu, meta = make(device, batch, 8, 4, 1, 128, lengths, seed=1)
    check(run(device, q, k, v, meta, 1, 8), q, k, v, cu, 8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,groups,kv_heads", [(64, 4, 8), (128, 8, 2), (256, 6, 4), (128, 1, 4),
                                                 (64, 3, 2)])
def test_decode_dims_groups_dtypes(device, dtype, dim, groups, kv_heads):
    rng = np.random.default_rng(dim + groups)
    lengths = rng.integers(1, 1200, 2 * kv_heads)
    q, k, v, cu, meta = make(device, 2, kv_heads, groups, 1, dim, lengths, dtype, seed=dim)
    check(run(device, q, k, v, meta, 1, kv_heads), q, k, v, cu, kv_heads)


def test_edge_lengths(device):
    lengths = [0, 1, 2, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 256, 257, 1000]
    q, k, v, cu, meta = make(device, 2, 8, 4, 1, 128, lengths, seed=7)
    check(run(device, q, k, v, meta, 1, 8), q, k, v, cu, 8)


def test_all_segments_empty(device):
    q, k, v, cu, meta = make(device, 1, 2, 4, 1, 64, [0, 0], seed=8)
    got = run(device, q, k, v, meta, 1, 2)
    assert torch.count_nonzero(got).item() == 0


@pytest.mark.parametrize("groups", [4, 6])
def test_square_causal_prefill(device, groups):
    length = 37
    q, k, v, cu, meta = make(device, 1, 2, groups, length, 128, [length, length], seed=9)
    check(run(device, q, k, v, meta, length, 2), q, k, v, cu, 2)


def test_prefill_with_history_and_short_segments(device):
    length = 5  # segments shorter than the query block leave their first queries with no key
    q, k, v, cu, meta = make(device, 2, 4, 4, length, 64, [300, 5, 3, 0, 700, 1, 64, 6], seed=10)
    check(run(device, q, k, v, meta, length, 4), q, k, v, cu, 4)


def test_long_prefill_many_chunks(device):
    length = 600
    q, k, v, cu, meta = make(device, 1, 1, 4, length, 128, [1500], seed=11)
    check(run(device, q, k, v, meta, length, 1), q, k, v, cu, 1)


def test_strided_queries_as_the_reference_builds_them(device):
    # q_proj(x).view(B, L, Hq, d).transpose(1, 2): a non-contiguous [B, Hq, L, d] view.
    g = torch.Generator().manual_seed(12)
    batch, length, kv_heads, groups, dim = 1, 3, 2, 4, 128
    flat = torch.randn((batch, length, kv_heads * groups, dim), generator=g).bfloat16()
    _, k, v, cu, meta = make(device, 1, kv_heads, groups, length, dim, [40, 9], seed=13)
    strided = flat.to(device).transpose(1, 2)
    assert not strided.is_contiguous()
    got = attention.packed_attention(strided, k.to(device), v.to(device), meta, length, kv_heads)
    check(got, flat.transpose(1, 2).contiguous(), k, v, cu, kv_heads)


def test_repeated_calls_reuse_the_workspace(device):
    first = make(device, 8, 8, 4, 1, 128, np.full(64, 2000), seed=14)
    second = make(device, 1, 8, 4, 1, 128, np.full(8, 777), seed=15)
    outputs = []
    for q, k, v, cu, meta in (first, second, first, second):
        outputs.append(run(device, q, k, v, meta, 1, 8))
    torch.cuda.synchronize()
    assert torch.equal(outputs[0], outputs[2]) and torch.equal(outputs[1], outputs[3])
    check(outputs[2], *first[:4], 8)
    check(outputs[3], *second[:4], 8)


def test_rejects_like_the_reference(device):
    q, k, v, cu, meta = make(device, 1, 2, 4, 1, 64, [3, 4], seed=16)
    with pytest.raises(RuntimeError, match="fp16 and bf16"):
        attention.packed_attention(q.float().to(device), k.float().to(device),
                                   v.float().to(device), meta, 1, 2)
    bad = SimpleNamespace(cu_seqlens_k=meta.cu_seqlens_k[:2], max_seqlen_k=4,
                          decoding_cu_seqlens_q=meta.decoding_cu_seqlens_q)
    with pytest.raises(RuntimeError, match="cu_seqlens_k"):
        run(device, q, k, v, bad, 1, 2)
    with pytest.raises(RuntimeError, match="backward"):
        attention.packed_attention(q.to(device).requires_grad_(True), k.to(device), v.to(device),
                                   meta, 1, 2)


def appended(device, keys, values, cumulative, batch, kv_heads, dim, new_keys, new_values):
    """The packed cache with each segment's new row after its cached rows (_C.append's layout)
    and its metadata."""
    from code_for_iclr27_amd import _C
    lengths = np.diff(cumulative)
    positions = torch.zeros((keys.shape[0],), dtype=torch.float32, device=device)
    k, v, _, cu, _ = _C.append(keys.to(device), values.to(device), positions,
                               new_keys.reshape(1, batch * kv_heads, 1, dim).to(device),
                               new_values.reshape(1, batch * kv_heads, 1, dim).to(device),
                               torch.from_numpy(cumulative).to(device), 0,
                               int(lengths.max(initial=0)))
    meta = SimpleNamespace(cu_seqlens_k=cu, max_seqlen_k=int(lengths.max(initial=0)) + 1,
                           decoding_cu_seqlens_q=torch.arange(batch * kv_heads + 1,
                                                              dtype=torch.int32, device=device))
    return k, v, meta


@pytest.mark.parametrize("case", ["cfg1", "cfg2", "block_edge", "d64", "d256", "f16", "empty"])
def test_pending_row_equals_attention_over_the_appended_cache(device, case):
    """A decode step's own token attended to before it is appended (the pending row) gives the
    same output, bit for bit, as the call on the cache with that token appended; the f64
    oracle on the appended cache bounds both. block_edge: cached lengths that fill whole key
    blocks, so that the pending row starts a block (and a split) of its own."""
    rng = np.random.default_rng(11)
    dim, groups, dtype, batch, kv_heads = 128, 4, torch.bfloat16, 1, 8
    if case == "cfg1":
        lengths = [2250] * 8
    elif case == "cfg2":
        batch = 8
        lengths = rng.integers(1500, 2251, batch * kv_heads)
    elif case == "block_edge":
        lengths = [16, 64, 192, 768, 1536, 3072, 48 * 4, 48 * 4 * 3]
    elif case == "d64":
        dim, lengths = 64, rng.integers(1, 400, 8)
    elif case == "d256":
        dim, groups, kv_heads, lengths = 256, 6, 4, [9216, 5, 700, 1]
    elif case == "f16":
        dtype, lengths = torch.float16, rng.integers(0, 900, 8)
    else:
        lengths = [0, 0, 3, 0, 0, 0, 0, 1]
    q, k, v, cu, meta = make(device, batch, kv_heads, groups, 1, dim, lengths, dtype, seed=4)
    g = torch.Generator().manual_seed(9)
    new_k = torch.randn((batch, kv_heads, 1, dim), generator=g).to(dtype)
    new_v = torch.randn((batch, kv_heads, 1, dim), generator=g).to(dtype)
    got = attention.packed_attention(q.to(device), k.to(device), v.to(device), meta, 1, kv_heads,
                                     pending=(new_k.to(device), new_v.to(device)))
    k_app, v_app, meta_app = appended(device, k, v, cu, batch, kv_heads, dim, new_k, new_v)
    want = attention.packed_attention(q.to(device), k_app, v_app, meta_app, 1, kv_heads)
    assert torch.equal(got, want)
    check(got, q, k_app.cpu(), v_app.cpu(), meta_app.cu_seqlens_k.cpu().numpy(), kv_heads)


def test_pending_rows_refused_for_prefill_and_bad_shapes(device):
    q, k, v, cu, meta = make(device, 1, 2, 2, 3, 64, [10, 20], seed=2)
    new = torch.zeros((1, 2, 1, 64), dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="one query per segment"):
        attention.packed_attention(q.to(device), k.to(device), v.to(device), meta, 3, 2,
                                   pending=(new, new))
    q, k, v, cu, meta = make(device, 1, 2, 2, 1, 64, [10, 20], seed=2)
    with pytest.raises(RuntimeError, match=r"\[batch, kv_heads, 1, head_dim\]"):
        attention.packed_attention(q.to(device), k.to(device), v.to(device), meta, 1, 2,
                                   pending=(new[:, :1], new[:, :1]))


def test_decode_step_with_appends_deferred_to_one_launch(device):
    """A decode step over four layers as the reference runs it (per layer: _C.append, then
    attention over the appended cache) and with the appends deferred: per layer, attention
    with the step's token pending; then one _C.append_layers for every layer. Outputs and the
    caches after the step are identical."""
    from code_for_iclr27_amd import _C
    L, H, G, d, seen = 4, 8, 4, 128, 5000
    rng = np.random.default_rng(3)
    g = torch.Generator().manual_seed(3)
    caches = []
    for _ in range(L):
        lengths = rng.integers(1500, 2251, H)
        rows = int(lengths.sum())
        caches.append(dict(
            keys=torch.randn((rows, d), generator=g).to(torch.bfloat16).to(device),
            values=torch.randn((rows, d), generator=g).to(torch.bfloat16).to(device),
            positions=torch.from_numpy(rng.permutation(rows).astype(np.float32)).to(device),
            cu=torch.from_numpy(np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)).to(device),
            longest=int(lengths.max())))
    step = [dict(q=torch.randn((1, H * G, 1, d), generator=g).to(torch.bfloat16).to(device),
                 k=torch.randn((1, H, 1, d), generator=g).to(torch.bfloat16).to(device),
                 v=torch.randn((1, H, 1, d), generator=g).to(torch.bfloat16).to(device))
            for _ in range(L)]
    decode_q = torch.arange(H + 1, dtype=torch.int32, device=device)
    # the reference's order: append, then attend, layer by layer (logical start: the token
    # index for layer 0, as cache.py:38 computes it after the first layer's update)
    eager_out, eager_cache = [], []
    for l in range(L):
        c, t = caches[l], step[l]
        k, v, p, cu, _ = _C.append(c["keys"], c["values"], c["positions"], t["k"], t["v"], c["cu"],
                                   seen, c["longest"])
        meta = SimpleNamespace(cu_seqlens_k=cu, max_seqlen_k=c["longest"] + 1,
                               decoding_cu_seqlens_q=decode_q)
        eager_out.append(attention.packed_attention(t["q"], k, v, meta, 1, H))
        eager_cache.append((k, v, p, cu))
    # deferred: attend with the token pending, then one append launch for all layers
    deferred_out = []
    for l in range(L):
        c, t = caches[l], step[l]
        meta = SimpleNamespace(cu_seqlens_k=c["cu"], max_seqlen_k=c["longest"],
                               decoding_cu_seqlens_q=decode_q)
        deferred_out.append(attention.packed_attention(t["q"], c["keys"], c["values"], meta, 1, H,
                                                       pending=(t["k"], t["v"])))
    keys, values, positions, cumulative, lengths, first = _C.append_layers(
        [c["keys"] for c in caches], [c["values"] for c in caches],
        [c["positions"] for c in caches], [t["k"] for t in step], [t["v"] for t in step],
        [c["cu"] for c in caches], [seen] * L, max(c["longest"] for c in caches))
    for l in range(L):
        assert torch.equal(deferred_out[l], eager_out[l]), l
        k, v, p, cu = eager_cache[l]
        rows = slice(int(first[l]), int(first[l + 1]))
        assert torch.equal(keys[rows], k) and torch.equal(values[rows], v)
        assert torch.equal(positions[rows].reshape(-1), p.reshape(-1))
        assert torch.equal(cumulative[l], cu)
