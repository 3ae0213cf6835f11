"""Scoring oracle (numpy; test infrastructure only).

Restates the reference GPU scorer op by op:
  temporal_probabilities  csrc/scoring.cu:32-66   (256-thread strided partials + LDS tree)
  temporal_risk           csrc/scoring.cu:68-128
  head_scores             src/lazy_recall/scoring.py:152-195 (pv GEMM, bf16 Q.K^T, the two
                          ops above, maximum over query chunks)
  decision_risk_scores    csrc/cache_legacy.cu:63-135 (legacy scorer)
Float32 arithmetic is done operation by operation in float32 (the reference builds with
--fmad=false, so products and sums are rounded separately). exp is evaluated in float64 and
rounded once, i.e. a correctly rounded expf.
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import round_f32_to_bf16, round_f64_to_bf16

F32 = np.float32


def reference_block_sum(values: np.ndarray) -> np.ndarray:
    """Row sums in the reference kernel's order (csrc/scoring.cu:15-30,52-57): 256 per-thread
    partials over positions t, t+256, ... accumulated in order, then a tree with strides
    128, 64, ..., 1."""
    values = np.asarray(values, dtype=F32)
    rows, length = values.shape
    blocks = max(1, -(-length // 256))
    padded = np.zeros((rows, blocks * 256), dtype=F32)
    padded[:, :length] = values
    partial = np.zeros((rows, 256), dtype=F32)
    for b in range(blocks):
        partial = (partial + padded[:, b * 256:(b + 1) * 256]).astype(F32)
    stride = 128
    while stride:
        partial[:, :stride] = (partial[:, :stride] + partial[:, stride:2 * stride]).astype(F32)
        stride //= 2
    return partial[:, 0]


def expf(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore", invalid="ignore"):
        return np.exp(np.asarray(x, dtype=np.float64)).astype(F32)


def round_logits(values: np.ndarray, dtype: str) -> np.ndarray:
    """static_cast<float>(static_cast<scalar_t>(x)) for the logits dtype."""
    if dtype == "bf16":
        return round_f32_to_bf16(values)
    if dtype == "f16":
        return np.asarray(values, dtype=F32).astype(np.float16).astype(F32)
    return np.asarray(values, dtype=F32)


def temporal_probabilities(logits, projected, query_positions, key_positions, scale,
                           dtype: str = "bf16"):
    """csrc/scoring.cu:32-66. logits [W, G, T] holding values of ``dtype``; returns
    (probabilities f32 [W, G, T], output_projection f32 [W, G])."""
    logits = np.asarray(logits, dtype=F32)
    window, groups, length = logits.shape
    scale = F32(scale)
    rounded = round_logits((logits * scale).astype(F32), dtype)
    # float key position <= int64 query position promoted to float (csrc/scoring.cu:46)
    qpos = np.asarray(query_positions).astype(F32).reshape(window, 1, 1)
    kpos = np.asarray(key_positions, dtype=F32).reshape(1, 1, length)
    masked = np.where(kpos <= qpos, rounded, F32(-np.inf)).astype(F32)
    rows = masked.reshape(window * groups, length)
    with np.errstate(invalid="ignore"):
        maximum = np.fmax.reduce(rows, axis=1, initial=-np.inf).astype(F32)
        weights = expf(rows - maximum[:, None])
        denominator = reference_block_sum(weights)
        probabilities = (weights / denominator[:, None]).astype(F32)
        pv = np.asarray(projected, dtype=F32)
        group_of_row = np.tile(np.arange(groups), window)
        products = (probabilities * pv[group_of_row]).astype(F32)
    projection = reference_block_sum(products)
    return probabilities.reshape(window, groups, length), projection.reshape(window, groups)


def softplus64(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return np.where(v > 20.0, v, np.log1p(np.exp(np.minimum(v, 20.0))))


def risk64(margin: float, drop: np.ndarray) -> np.ndarray:
    """csrc/scoring.cu:68-75: max(0, sigma(m) * (m - (m - d)) - softplus(m) + softplus(m - d))
    evaluated in float64."""
    m = np.float64(margin)
    p = 1.0 / (1.0 + math.exp(-m))
    compared = m - np.asarray(drop, dtype=F32).astype(np.float64)
    return np.maximum(0.0, p * (m - compared) - softplus64(m) + softplus64(compared))


def temporal_risk(probabilities, output_projection, projected, margin, first, last, epsilon):
    """csrc/scoring.cu:77-128: per candidate in [first, last), min and max over queries of
    sum_g p/max(1-p, eps) * (pv - op) (groups summed in order), any non-finite drop -> NaN."""
    probabilities = np.asarray(probabilities, dtype=F32)
    window, groups, _ = probabilities.shape
    op = np.asarray(output_projection, dtype=F32).reshape(window, groups)
    pv = np.asarray(projected, dtype=F32)
    eps = F32(epsilon)
    drop = np.zeros((window, last - first), dtype=F32)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for g in range(groups):
            p = probabilities[:, g, first:last]
            ratio = (p / np.maximum((F32(1.0) - p).astype(F32), eps)).astype(F32)
            difference = (pv[g, first:last][None, :] - op[:, g][:, None]).astype(F32)
            drop = (drop + (ratio * difference).astype(F32)).astype(F32)
    bad = ~np.isfinite(drop).all(axis=0)
    lo = drop.min(axis=0) if window else np.zeros(last - first, F32)
    hi = drop.max(axis=0) if window else np.zeros(last - first, F32)
    m = float(np.asarray(margin, dtype=F32).reshape(-1)[0])
    with np.errstate(invalid="ignore"):
        score = np.maximum(risk64(m, lo), risk64(m, hi)).astype(F32)
    score[bad] = np.nan
    return score


def exact_logits(queries, keys) -> np.ndarray:
    """bf16(Q . K^T) with the dot product formed exactly (float64) and rounded once: the value
    every fp32-accumulating bf16 GEMM approximates (scoring.py:184). queries [W, G, d]."""
    q = np.asarray(queries, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    return round_f64_to_bf16(np.einsum("wgd,td->wgt", q, k))


def projected_values(gradient, values) -> np.ndarray:
    """scoring.py:175: float32 grad [G, d] x values^T [d, T], formed exactly and rounded."""
    return (np.asarray(gradient, dtype=np.float64) @ np.asarray(values, dtype=np.float64).T).astype(F32)


def head_scores(queries, query_positions, keys, key_positions, values, first, last, gradient,
                margin, epsilon, logits=None, chunk=None):
    """src/lazy_recall/scoring.py:152-195 for one KV head. queries [W, G, d] (bf16 values),
    keys/values [T, d] (bf16 values), gradient [G, d] f32. ``logits`` [W, G, T] overrides the
    exact-rounded Q.K^T. Query chunks give the same result as one chunk (risk is convex with
    its minimum at zero drop); ``chunk`` evaluates them literally."""
    queries = np.asarray(queries, dtype=F32)
    window = queries.shape[0]
    pv = projected_values(gradient, values)
    if logits is None:
        logits = exact_logits(queries, keys)
    scale = F32(1.0 / math.sqrt(keys.shape[-1]))
    result = None
    step = chunk or window
    for start in range(0, window, step):
        end = min(start + step, window)
        probabilities, projection = temporal_probabilities(
            logits[start:end], pv, np.asarray(query_positions)[start:end], key_positions, scale)
        scores = temporal_risk(probabilities, projection, pv, margin, first, last, epsilon)
        result = scores if result is None else np.maximum(result, scores)
    return result


def stable_sigmoid(v: float) -> float:
    if v >= 0.0:
        return 1.0 / (1.0 + math.exp(-v))
    e = math.exp(v)
    return e / (1.0 + e)


def stable_softplus(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return np.where(v > 20.0, v + np.log1p(np.exp(-np.abs(v))), np.log1p(np.exp(np.minimum(v, 20.0))))


def decision_risk_scores(probabilities, values, head_outputs, gradients, base_margin, epsilon):
    """csrc/cache_legacy.cu:81-135: per candidate, sum over (group, dim) of
    grad * (alpha / max(1-alpha, eps) * (v - head_out)) in the kernel's 256-strided + tree
    order, then the Bernoulli KL in float64 clamped at zero."""
    alpha = np.asarray(probabilities, dtype=F32)  # [G, C]
    v = np.asarray(values, dtype=F32)              # [C, d]
    ho = np.asarray(head_outputs, dtype=F32)       # [G, d]
    grad = np.asarray(gradients, dtype=F32)        # [G, d]
    groups, candidates = alpha.shape
    eps = F32(epsilon)
    den = np.maximum((F32(1.0) - alpha).astype(F32), eps)
    ratio = (alpha / den).astype(F32)                                   # [G, C]
    diff = (v[None, :, :] - ho[:, None, :]).astype(F32)                  # [G, C, d]
    local = (ratio[:, :, None] * diff).astype(F32)
    terms = (grad[:, None, :] * local).astype(F32)                       # [G, C, d]
    flat = np.transpose(terms, (1, 0, 2)).reshape(candidates, -1)        # index = g*d + dim
    partial = reference_block_sum(flat)
    m = float(base_margin)
    compared = m - partial.astype(np.float64)
    kl = stable_sigmoid(m) * (m - compared) - stable_softplus(m) + stable_softplus(compared)
    return np.maximum(kl, 0.0).astype(F32)


def bernoulli_kl(p: float, q: np.ndarray) -> np.ndarray:
    """Textbook KL(Ber(p) || Ber(q)) — the closed form risk64 rewrites (used to pin it)."""
    q = np.asarray(q, dtype=np.float64)
    return p * np.log(p / q) + (1.0 - p) * np.log((1.0 - p) / (1.0 - q))
