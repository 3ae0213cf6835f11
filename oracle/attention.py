"""Oracle (test infrastructure only): attention over the packed ragged KV layout.

Restates the result of src/lazy_recall/attention.py:15-35, i.e. flash_attn_varlen_func with
causal=True, softmax_scale = dim^-0.5 and one KV head per (request, KV head) segment, in f64
numpy. flash_attn (not vendored under the reference; pinned nowhere in its pyproject) documents
varlen causal masking as aligned to the bottom-right of each sequence's score matrix: query i of
L sees key j iff j <= i + n - L; a query that sees no key outputs 0. Query heads h*G .. h*G+G-1
share KV head h (grouped-query attention); the output is [batch, L, Hq * dim]
(attention.py:20-35).
"""

from __future__ import annotations

import numpy as np


def packed_attention(queries: np.ndarray, keys: np.ndarray, values: np.ndarray,
                     cumulative: np.ndarray, kv_heads: int, scale: float | None = None
                     ) -> np.ndarray:
    """queries [B, Hq, L, d], keys/values [N, d], cumulative [B*kv_heads + 1] -> f64 [B, L, Hq*d]."""
    batch, query_heads, length, dim = queries.shape
    groups = query_heads // kv_heads
    scale = dim ** -0.5 if scale is None else scale
    q = queries.astype(np.float64)
    k_all = keys.astype(np.float64)
    v_all = values.astype(np.float64)
    out = np.zeros((batch, length, query_heads, dim), dtype=np.float64)
    for b in range(batch):
        for h in range(kv_heads):
            s = b * kv_heads + h
            start, end = int(cumulative[s]), int(cumulative[s + 1])
            k, v = k_all[start:end], v_all[start:end]
            n = end - start
            limits = np.arange(length) + n - length  # query i sees keys j <= limits[i]
            visible = np.arange(n)[None, :] <= limits[:, None]  # [L, n]
            for g in range(groups):
                head = h * groups + g
                logits = q[b, head] @ k.T * scale  # [L, n]
                logits = np.where(visible, logits, -np.inf)
                peak = logits.max(axis=1, keepdims=True) if n else np.zeros((length, 1))
                seen = visible.any(axis=1)
                weights = np.where(visible, np.exp(logits - np.where(seen[:, None], peak, 0.0)), 0.0)
                total = weights.sum(axis=1, keepdims=True)
                rows = np.divide(weights @ v, total, out=np.zeros((length, dim)), where=total > 0)
                out[b, :, head] = rows
    return out.reshape(batch, length, query_heads * dim)
