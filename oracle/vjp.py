"""Oracle (test infrastructure only): the audit's margin objective and its gradients, in f64.

Restates src/lazy_recall/_core/scoring.py:27-76 (one_vs_rest_margin,
last_token_logits_float32, one_vs_rest_hidden_gradient), batch_audit.py:11-24 (row_margins,
row_hidden_gradients) and the pre-projection gradient of scoring.py:228-237.
"""

from __future__ import annotations

import numpy as np


def head_logits(hidden: np.ndarray, weight: np.ndarray, bias: np.ndarray | None = None):
    """_core/scoring.py:34-52: F.linear(hidden.float(), W.float(), b) -> [rows, vocab]."""
    out = hidden.astype(np.float64) @ weight.astype(np.float64).T
    return out if bias is None else out + bias.astype(np.float64)


def margin_stats(logits: np.ndarray, targets: np.ndarray | None = None):
    """_core/scoring.py:27-31 / batch_audit.py:11-15 -> (margins, targets, M, S) per row.
    targets default to torch.argmax (first index of the largest logit)."""
    logits = np.asarray(logits, dtype=np.float64)
    if targets is None:
        targets = logits.argmax(axis=1)  # numpy also returns the first maximal index
    targets = np.asarray(targets, dtype=np.int64)
    rows = np.arange(logits.shape[0])
    competitors = logits.copy()
    competitors[rows, targets] = -np.inf
    peak = competitors.max(axis=1)
    total = np.exp(competitors - peak[:, None]).sum(axis=1)
    margins = logits[rows, targets] - (peak + np.log(total))
    return margins, targets, peak, total


def hidden_gradient(logits: np.ndarray, targets: np.ndarray, weight: np.ndarray,
                    due: np.ndarray | None = None):
    """_core/scoring.py:55-76 / batch_audit.py:18-24: (W[t] - softmax(competitors) @ W) * due."""
    logits = np.asarray(logits, dtype=np.float64)
    w = weight.astype(np.float64)
    rows = np.arange(logits.shape[0])
    competitors = logits.copy()
    competitors[rows, targets] = -np.inf
    p = np.exp(competitors - competitors.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    out = w[targets] - p @ w
    return out if due is None else out * np.asarray(due, dtype=np.float64)[:, None]


def pre_gradient(post: np.ndarray, o_weight: np.ndarray, gate: np.ndarray | None = None):
    """scoring.py:228-237: post @ o_proj.weight.float() (* gate) -> [width]."""
    out = post.astype(np.float64) @ o_weight.astype(np.float64)
    return out if gate is None else out * gate.astype(np.float64)
