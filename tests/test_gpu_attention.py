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
