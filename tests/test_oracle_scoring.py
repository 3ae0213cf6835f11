"""Pins the scoring oracle against independent checks (CPU only).

bf16 rounding        torch's float->bfloat16 conversion; exact rational arithmetic for f64->bf16
block sums           math.fsum
probabilities        float64 softmax, row sums, masking
risk64               the textbook Bernoulli KL closed form it rewrites
temporal_risk        float64 brute force on tiny inputs
head_scores          the reference CPU math path (torch ops) on inputs whose logits are exact,
                     chunked == unchunked, and W=1, G=1 == the legacy single-query scorer
decision_risk        the reference's torch formulation (_core/cuda_ops.py:125-170)
"""

import math
from fractions import Fraction

import numpy as np
import torch
import torch.nn.functional as F

from oracle import bf16, cpu_path, scoring


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        # exact midpoints between bf16 neighbours, and one ulp of float32 either side
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        ((np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000) + 1).view(np.float32),
        ((np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000) - 1).view(np.float32),
        np.asarray([0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-39], dtype=np.float32),
    ])
    expect = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16.f32_to_bf16_bits(x), expect)


def _exact_bf16_round(value: float) -> float:
    """Nearest bf16 to a float64 by exact rational comparison (ties to even)."""
    f = np.float32(value)
    bits = int(np.asarray([f]).view(np.uint32)[0]) & 0xFFFF0000
    candidates = []
    for step in range(-2, 3):
        b = (bits + (step << 16)) & 0xFFFFFFFF
        c = float(np.asarray([b], dtype=np.uint32).view(np.float32)[0])
        if math.isfinite(c):
            candidates.append((abs(Fraction(c) - Fraction(value)), (b >> 16) & 1, c))
    candidates.sort(key=lambda t: (t[0], t[1]))
    return candidates[0][2]


def test_round_f64_to_bf16_exact():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(3000) * 37.0
    mids = [(float(np.asarray([(b << 16) | 0x8000], np.uint32).view(np.float32)[0]))
            for b in range(0x3F00, 0x3F40)]
    x = np.concatenate([x, mids, [m + 1e-12 for m in mids], [m - 1e-12 for m in mids]])
    got = bf16.round_f64_to_bf16(x)
    expect = np.asarray([_exact_bf16_round(v) for v in x], dtype=np.float32)
    np.testing.assert_array_equal(got, expect)


def test_block_sum_close_to_fsum():
    rng = np.random.default_rng(2)
    v = rng.random((7, 2250)).astype(np.float32)
    got = scoring.reference_block_sum(v)
    expect = [math.fsum(row.astype(np.float64)) for row in v]
    np.testing.assert_allclose(got, expect, rtol=2e-6)


def _inputs(rng, window=6, groups=3, length=50, dim=16):
    logits = bf16.random_bf16(rng, (window, groups, length), 4.0)
    pv = rng.standard_normal((groups, length)).astype(np.float32) * 5
    qpos = np.arange(length - window, length, dtype=np.int64)
    kpos = rng.permutation(length).astype(np.float32)
    return logits, pv, qpos, kpos


def test_probabilities_against_float64_softmax():
    rng = np.random.default_rng(3)
    logits, pv, qpos, kpos = _inputs(rng)
    scale = np.float32(0.25)
    p, op = scoring.temporal_probabilities(logits, pv, qpos, kpos, scale)
    z = bf16.round_f32_to_bf16(logits * scale).astype(np.float64)
    mask = kpos[None, None, :] <= qpos[:, None, None].astype(np.float32)
    z = np.where(mask, z, -np.inf)
    e = np.exp(z - z.max(axis=-1, keepdims=True))
    expect = e / e.sum(axis=-1, keepdims=True)
    np.testing.assert_allclose(p, expect, rtol=2e-6, atol=1e-12)
    assert np.all(p[~np.broadcast_to(mask, p.shape)] == 0)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(op, (expect * pv[None]).sum(-1), rtol=1e-4, atol=1e-5)


def test_risk64_is_bernoulli_kl():
    margin = 2.0
    drops = np.linspace(-6, 6, 241).astype(np.float32).astype(np.float64)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    expect = scoring.bernoulli_kl(sig(margin), sig(margin - drops))
    got = scoring.risk64(margin, drops.astype(np.float32))
    np.testing.assert_allclose(got, expect, rtol=1e-9, atol=1e-15)
    assert scoring.risk64(margin, np.zeros(1, np.float32))[0] == 0.0


def test_temporal_risk_brute_force():
    rng = np.random.default_rng(4)
    logits, pv, qpos, kpos = _inputs(rng, window=4, groups=2, length=20)
    p, op = scoring.temporal_probabilities(logits, pv, qpos, kpos, 0.5)
    first, last, eps, margin = 3, 17, 1e-6, np.float32(1.5)
    got = scoring.temporal_risk(p, op, pv, margin, first, last, eps)
    expect = []
    for t in range(first, last):
        drops = []
        for w in range(4):
            d = 0.0
            for g in range(2):
                pp = float(p[w, g, t])
                d += pp / max(1 - pp, eps) * (float(pv[g, t]) - float(op[w, g]))
            drops.append(d)
        kl = [scoring.bernoulli_kl(1 / (1 + math.exp(-1.5)), np.asarray([1 / (1 + math.exp(-(1.5 - x)))]))[0]
              for x in (min(drops), max(drops))]
        expect.append(max(kl))
    np.testing.assert_allclose(got, expect, rtol=2e-4, atol=1e-12)


def test_temporal_risk_nonfinite_is_nan():
    rng = np.random.default_rng(5)
    logits, pv, qpos, kpos = _inputs(rng, window=3, groups=2, length=12)
    p, op = scoring.temporal_probabilities(logits, pv, qpos, kpos, 0.5)
    pv = pv.copy()
    pv[1, 4] = np.inf
    got = scoring.temporal_risk(p, op, pv, np.float32(2), 0, 10, 1e-6)
    assert np.isnan(got[4]) and np.isfinite(np.delete(got, 4)).all()


def _exact_head(rng, window=12, groups=2, length=80, dim=64):
    """Inputs whose Q.K^T values are exact in bf16 and whose scale 1/sqrt(64) is a power of
    two, so every formulation of the logits agrees bit for bit."""
    q = (rng.integers(-1, 2, (window, groups, dim)) * 0.25).astype(np.float32)
    k = (rng.integers(-1, 2, (length, dim)) * 0.25).astype(np.float32)
    v = bf16.random_bf16(rng, (length, dim))
    kpos = np.arange(length, dtype=np.float32)
    qpos = np.arange(length - window, length, dtype=np.int64)
    grad = np.abs(rng.standard_normal((groups, dim))).astype(np.float32)
    return q, qpos, k, kpos, v, grad


def test_head_scores_match_reference_cpu_path():
    rng = np.random.default_rng(6)
    q, qpos, k, kpos, v, grad = _exact_head(rng)
    first, last, margin, eps = 0, 80 - 32, np.float32(2.0), 1e-6
    got = scoring.head_scores(q, qpos, k, kpos, v, first, last, grad, margin, eps)
    t = lambda a, dt=torch.bfloat16: torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    expect = cpu_path.temporal_head_scores_cpu(
        t(q), torch.from_numpy(qpos), t(k), torch.from_numpy(kpos), t(v), first, last,
        torch.from_numpy(grad), torch.tensor(float(margin)), eps, 250).numpy()
    np.testing.assert_allclose(got, expect, rtol=1e-5, atol=1e-12)


def test_head_scores_chunked_equals_unchunked():
    rng = np.random.default_rng(7)
    q, qpos, k, kpos, v, grad = _exact_head(rng, window=20)
    a = scoring.head_scores(q, qpos, k, kpos, v, 5, 48, grad, np.float32(2), 1e-6)
    b = scoring.head_scores(q, qpos, k, kpos, v, 5, 48, grad, np.float32(2), 1e-6, chunk=3)
    np.testing.assert_array_equal(a, b)


def test_single_query_head_score_is_legacy_decision_risk():
    """With W = 1 and G = 1 the temporal score reduces to the legacy scorer: both are the
    Bernoulli KL of the leave-one-out margin drop (pv - op = grad . (v - head_output))."""
    rng = np.random.default_rng(8)
    length, dim = 60, 64
    q, qpos, k, kpos, v, grad = _exact_head(rng, window=1, groups=1, length=length, dim=dim)
    qpos = np.asarray([length - 1])
    got = scoring.head_scores(q, qpos, k, kpos, v, 0, length, grad, np.float32(2), 1e-6)
    logits = scoring.exact_logits(q, k)
    p, _ = scoring.temporal_probabilities(logits, np.zeros((1, length), np.float32), qpos, kpos,
                                          np.float32(0.125))
    probs = p[0]  # [1, T]
    head_out = (probs.astype(np.float64) @ v.astype(np.float64)).astype(np.float32)
    expect = scoring.decision_risk_scores(probs, v, head_out, grad, 2.0, 1e-6)
    np.testing.assert_allclose(got, expect, rtol=1e-4, atol=1e-10)


def test_decision_risk_matches_reference_torch_formulation():
    rng = np.random.default_rng(9)
    groups, candidates, dim = 3, 40, 32
    alpha = rng.random((groups, candidates)).astype(np.float32) * 0.1
    values = rng.standard_normal((candidates, dim)).astype(np.float32)
    head_out = rng.standard_normal((groups, dim)).astype(np.float32)
    grads = rng.standard_normal((groups, dim)).astype(np.float32)
    got = scoring.decision_risk_scores(alpha, values, head_out, grads, 1.25, 1e-6)
    a = torch.from_numpy(alpha)
    local = a[:, :, None] / (1.0 - a).clamp_min(1e-6)[:, :, None] * (
        torch.from_numpy(values)[None] - torch.from_numpy(head_out)[:, None])
    drop = (local * torch.from_numpy(grads)[:, None]).sum(dim=(0, 2))
    m = torch.tensor(1.25, dtype=torch.float64)
    compared = m - drop.to(torch.float64)
    kl = (torch.sigmoid(m) * (m - compared) - F.softplus(m) + F.softplus(compared)).clamp_min(0.0)
    np.testing.assert_allclose(got, kl.float().numpy(), rtol=1e-5, atol=1e-12)
