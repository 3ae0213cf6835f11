"""The packed-attention oracle (oracle/attention.py) pinned against things other than itself:
torch-CPU scaled_dot_product_attention in f64 (decode and square causal prefill), a brute-force
per-query Python loop for bottom-right causal masks with history (L < n), and closed forms
(one visible key returns its value row, equal logits average the value rows, a query that sees
no key outputs zeros, each query head reads only its own KV head)."""

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention


def ragged(seed, batch, kv_heads, groups, length, dim, lengths):
    rng = np.random.default_rng(seed)
    queries = rng.standard_normal((batch, kv_heads * groups, length, dim))
    total = int(sum(lengths))
    keys = rng.standard_normal((total, dim))
    values = rng.standard_normal((total, dim))
    cumulative = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    return queries, keys, values, cumulative


def test_decode_matches_torch_sdpa():
    batch, kv_heads, groups, dim = 3, 2, 4, 16
    lengths = [5, 17, 1, 9, 30, 2]
    q, k, v, cu = ragged(0, batch, kv_heads, groups, 1, dim, lengths)
    got = attention.packed_attention(q, k, v, cu, kv_heads)
    for b in range(batch):
        for h in range(kv_heads):
            s = b * kv_heads + h
            kk = torch.from_numpy(k[cu[s]:cu[s + 1]])[None, None]
            vv = torch.from_numpy(v[cu[s]:cu[s + 1]])[None, None]
            qq = torch.from_numpy(q[b, h * groups:(h + 1) * groups])[None]  # [1, G, 1, d]
            expect = F.scaled_dot_product_attention(qq, kk.expand(1, groups, -1, -1),
                                                    vv.expand(1, groups, -1, -1))
            got_heads = got[b, 0].reshape(kv_heads * groups, dim)[h * groups:(h + 1) * groups]
            np.testing.assert_allclose(got_heads, expect[0, :, 0].numpy(), rtol=1e-12, atol=1e-12)


def test_square_prefill_matches_torch_causal_sdpa():
    dim, groups, length = 8, 2, 11
    q, k, v, cu = ragged(1, 1, 1, groups, length, dim, [length])
    got = attention.packed_attention(q, k, v, cu, 1).reshape(length, groups, dim)
    expect = F.scaled_dot_product_attention(torch.from_numpy(q),
                                            torch.from_numpy(k)[None, None].expand(1, groups, -1, -1),
                                            torch.from_numpy(v)[None, None].expand(1, groups, -1, -1),
                                            is_causal=True)[0]
    np.testing.assert_allclose(got, expect.permute(1, 0, 2).numpy(), rtol=1e-12, atol=1e-12)


def test_bottom_right_causal_against_brute_force():
    dim, groups, length = 4, 3, 5
    lengths = [9, 3, 5]  # more keys than queries, fewer (first queries see nothing), equal
    q, k, v, cu = ragged(2, 1, 3, groups, length, dim, lengths)
    got = attention.packed_attention(q, k, v, cu, 3).reshape(length, 3 * groups, dim)
    for h, n in enumerate(lengths):
        for g in range(groups):
            head = h * groups + g
            for i in range(length):
                visible = [j for j in range(n) if j <= i + n - length]
                if not visible:
                    assert np.all(got[i, head] == 0.0)
                    continue
                logits = [sum(q[0, head, i, e] * k[cu[h] + j, e] for e in range(dim)) / math.sqrt(dim)
                          for j in visible]
                peak = max(logits)
                weights = [math.exp(x - peak) for x in logits]
                total = sum(weights)
                expect = [sum(w * v[cu[h] + j, e] for w, j in zip(weights, visible)) / total
                          for e in range(dim)]
                np.testing.assert_allclose(got[i, head], expect, rtol=1e-12, atol=1e-14)


def test_closed_forms():
    dim = 8
    rng = np.random.default_rng(3)
    v = rng.standard_normal((4, dim))
    q = rng.standard_normal((1, 2, 1, dim))
    # One visible key: the output is that key's value row, whatever the logit.
    out = attention.packed_attention(q, rng.standard_normal((1, dim)), v[:1], np.array([0, 1]), 1)
    np.testing.assert_allclose(out.reshape(2, dim), np.repeat(v[:1], 2, axis=0), rtol=0, atol=1e-15)
    # Zero keys: equal logits, so the output is the mean of the value rows.
    out = attention.packed_attention(q, np.zeros((4, dim)), v, np.array([0, 4]), 1)
    np.testing.assert_allclose(out.reshape(2, dim), np.repeat(v.mean(0, keepdims=True), 2, 0),
                               rtol=1e-14, atol=1e-15)
    # An empty segment outputs zeros.
    out = attention.packed_attention(q, np.zeros((0, dim)), np.zeros((0, dim)), np.array([0, 0]), 1)
    assert np.all(out == 0.0)


def test_query_heads_read_their_own_kv_head():
    dim, groups = 4, 2
    q = np.ones((1, 4, 1, dim))
    keys = np.zeros((2, dim))
    values = np.stack([np.full(dim, 1.0), np.full(dim, -7.0)])
    out = attention.packed_attention(q, keys, values, np.array([0, 1, 2]), 2).reshape(4, dim)
    np.testing.assert_array_equal(out[:groups], 1.0)
    np.testing.assert_array_equal(out[groups:], -7.0)
