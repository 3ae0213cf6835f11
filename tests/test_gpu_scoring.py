"""GPU parity of the scoring ops.

Tolerances (float32 arithmetic, north-star bar rtol 1e-5):
  temporal_probabilities  rtol 1e-5 on p and output_projection (exp and summation order may
                          differ from the oracle in the last bits)
  temporal_risk           rtol 1e-5, same probabilities fed to both sides
  decision_risk_scores    rtol 1e-5
  fused scorer logits     equal to bf16(exact Q.K^T) except for < 0.1% of logits whose exact
                          value is within the MFMA's fp32 accumulation error (2^-19 sum|q k|)
                          of a bf16 rounding midpoint
  fused scorer scores     rtol 1e-5 (atol 1e-12) against the oracle fed the same logits;
                          NaN exactly where the oracle has NaN
"""

import math

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _C, _legacy_C, _lib, scoring, workloads
from oracle import bf16 as obf16
from oracle import scoring as oscoring

pytestmark = pytest.mark.gpu


def to_np(t):
    return t.detach().float().cpu().numpy()


def rand(shape, dtype, device, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(250, 4, 2250), (7, 3, 5000), (1, 1, 33)])
def test_temporal_probabilities(device, dtype, shape):
    window, groups, length = shape
    logits = rand(shape, dtype, device, 1, scale=math.sqrt(128))
    pv = rand((groups, length), torch.float32, device, 2, scale=10)
    qpos = torch.arange(length - window, length, device=device)
    kpos = torch.arange(length, device=device).float()
    scale = 1.0 / math.sqrt(128)
    p, op = _C.temporal_probabilities(logits, pv, qpos, kpos, scale)
    name = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]
    ep, eop = oscoring.temporal_probabilities(to_np(logits), to_np(pv), qpos.cpu().numpy(),
                                              kpos.cpu().numpy(), np.float32(scale), name)
    np.testing.assert_allclose(to_np(p), ep, rtol=1e-5, atol=1e-30)
    np.testing.assert_allclose(to_np(op), eop, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape,first,last", [((250, 4, 2250), 0, 2218), ((5, 6, 300), 17, 299)])
def test_temporal_risk(device, shape, first, last):
    window, groups, length = shape
    logits = rand(shape, torch.bfloat16, device, 3, scale=math.sqrt(128))
    pv = rand((groups, length), torch.float32, device, 4, scale=10)
    qpos = torch.arange(length - window, length, device=device)
    kpos = torch.arange(length, device=device).float()
    p, op = _C.temporal_probabilities(logits, pv, qpos, kpos, 1.0 / math.sqrt(128))
    margin = torch.tensor([2.0], device=device)
    got = _C.temporal_risk(p, op, pv, margin, first, last, 1e-6)
    expect = oscoring.temporal_risk(to_np(p), to_np(op), to_np(pv), np.float32(2.0), first, last, 1e-6)
    np.testing.assert_allclose(to_np(got), expect, rtol=1e-5, atol=1e-12)


def test_temporal_risk_nonfinite(device):
    p = torch.full((3, 2, 10), 0.1, device=device)
    op = torch.zeros((3, 2), device=device)
    pv = torch.ones((2, 10), device=device)
    pv[1, 4] = float("nan")
    got = _C.temporal_risk(p, op, pv, torch.tensor([2.0], device=device), 0, 10, 1e-6)
    assert torch.isnan(got[4]) and bool(torch.isfinite(torch.cat([got[:4], got[5:]])).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
def test_decision_risk_scores(device, dtype):
    groups, candidates, dim = 4, 513, 128
    g = torch.Generator().manual_seed(5)
    probs = (torch.rand((groups, candidates), generator=g) * 0.05).to(device)
    values = rand((candidates, dim), dtype, device, 6)
    head_out = rand((groups, dim), torch.float32, device, 7)
    grads = rand((groups, dim), torch.float32, device, 8)
    got = _legacy_C.decision_risk_scores(probs, values, head_out, grads, 1.5, 1e-6)
    expect = oscoring.decision_risk_scores(to_np(probs), to_np(values), to_np(head_out),
                                           to_np(grads), 1.5, 1e-6)
    np.testing.assert_allclose(to_np(got), expect, rtol=1e-5, atol=1e-12)


def _check_segment_logits(plan, layers, segment, device):
    """Returns the fused scorer's logits [W, G, T] after checking them against bf16(exact)."""
    seg = plan.segments[segment]
    layer = layers[seg.layer]
    groups, window = plan.groups, plan.window
    start = plan.head_starts[segment]
    length = int(plan.table[segment, 5])
    raw = scoring.debug_segment_logits(plan, segment, device)  # [G, W, T]
    gpu = np.transpose(to_np(raw), (1, 0, 2))
    q = to_np(layer.queries[seg.head * groups:(seg.head + 1) * groups]).transpose(1, 0, 2)
    k = to_np(layer.keys[start:start + length])
    exact = np.einsum("wgd,td->wgt", q.astype(np.float64), k.astype(np.float64))
    expect = obf16.round_f64_to_bf16(exact)
    mismatch = gpu != expect
    if mismatch.any():
        # gpu = bf16(acc) where the MFMA's fp32 accumulation gives |acc - exact| <= eps * M,
        # M = sum_k |q_k k_k|; hence |gpu - exact| <= half a bf16 ulp of gpu + eps * M. Only
        # logits within that distance of a rounding midpoint can round the other way.
        magnitude = np.einsum("wgd,td->wgt", np.abs(q).astype(np.float64), np.abs(k).astype(np.float64))
        g = gpu[mismatch].astype(np.float64)
        error = np.abs(g - exact[mismatch])
        assert np.all(error <= np.abs(g) * 2.0 ** -8 + 2.0 ** -19 * magnitude[mismatch])
        assert mismatch.mean() < 1e-3, mismatch.mean()
    return gpu


@pytest.mark.parametrize("dim,groups,window", [(128, 4, 250), (64, 4, 40), (256, 6, 77), (128, 3, 33),
                                               (128, 8, 70), (128, 1, 100), (128, 16, 40),
                                               (64, 16, 65), (256, 16, 33)])
def test_fused_scorer_matches_oracle(device, dim, groups, window):
    head_lengths = [[300, 41, 280, 2], [170, 300, 33, 299]]
    prompts = [[0, 0, 5, 0], [12, 0, 0, 0]]
    layers, qpos = workloads.make_layers(head_lengths, groups, dim, window, device, seed=dim + groups,
                                         prompt_lengths=prompts)
    margin = torch.tensor([2.0], device=device)
    plan = scoring.plan_segments(layers, protect_prompt=True, protect_recent=32)
    scores = to_np(scoring.score_plan(plan, qpos, margin))
    assert len(plan.segments) == 7  # the length-2 head has no candidate after recent protection
    offset = 0
    for segment, seg in enumerate(plan.segments):
        layer = layers[seg.layer]
        start = plan.head_starts[segment]
        length = int(plan.table[segment, 5])
        logits = _check_segment_logits(plan, layers, segment, device)
        q = to_np(layer.queries[seg.head * groups:(seg.head + 1) * groups]).transpose(1, 0, 2)
        expect = oscoring.head_scores(
            q, qpos.cpu().numpy(), to_np(layer.keys[start:start + length]),
            to_np(layer.positions[start:start + length]), to_np(layer.values[start:start + length]),
            seg.position_start, seg.position_start + seg.count,
            to_np(layer.gradient[seg.head * groups:(seg.head + 1) * groups]), np.float32(2.0), 1e-6,
            logits=logits)
        got = scores[offset:offset + seg.count]
        np.testing.assert_allclose(got, expect, rtol=1e-5, atol=1e-12,
                                   err_msg=f"segment {segment} layer {seg.layer} head {seg.head}")
        offset += seg.count
    assert offset == scores.size


def _peaked_layers(dim, groups, window, query_scale, device):
    head_lengths = [[300, 190], [260, 75]]
    layers, qpos = workloads.make_layers(head_lengths, groups, dim, window, device,
                                         seed=dim + groups + 7)
    for layer in layers:  # scale half of the query heads: some rows peaked, the rest ordinary
        q = layer.queries.float()
        q[: q.size(0) // 2] *= query_scale
        layer.queries.copy_(q.to(layer.queries.dtype))
    return layers, qpos


@pytest.mark.parametrize("dim,groups,window,query_scale,epsilon", [
    (128, 4, 90, 2.0, 1e-6),    # peaked rows (S < 2 in some): the clamped (general) form
    (256, 6, 77, 2.0, 1e-6),
    (64, 4, 70, 1.0, 0.4),      # eps * S > 1/2 in most rows: the general form almost everywhere
    (128, 4, 90, 1.0, 0.4)])
def test_fused_scorer_general_form_rows(device, dim, groups, window, query_scale, epsilon):
    """Rows the fast forms may not take: peaked attention (queries scaled up, so S is below 2)
    and a large denominator epsilon (eps * S > 1/2), mixed with ordinary rows; the scores against
    the oracle at rtol 1e-5."""
    layers, qpos = _peaked_layers(dim, groups, window, query_scale, device)
    margin = torch.tensor([2.0], device=device)
    plan = scoring.plan_segments(layers, protect_prompt=True, protect_recent=32)
    scores = to_np(scoring.score_plan(plan, qpos, margin, denominator_epsilon=epsilon))
    offset = 0
    for segment, seg in enumerate(plan.segments):
        layer = layers[seg.layer]
        start = plan.head_starts[segment]
        length = int(plan.table[segment, 5])
        logits = _check_segment_logits(plan, layers, segment, device)
        q = to_np(layer.queries[seg.head * groups:(seg.head + 1) * groups]).transpose(1, 0, 2)
        expect = oscoring.head_scores(
            q, qpos.cpu().numpy(), to_np(layer.keys[start:start + length]),
            to_np(layer.positions[start:start + length]), to_np(layer.values[start:start + length]),
            seg.position_start, seg.position_start + seg.count,
            to_np(layer.gradient[seg.head * groups:(seg.head + 1) * groups]), np.float32(2.0),
            epsilon, logits=logits)
        got = scores[offset:offset + seg.count]
        np.testing.assert_allclose(got, expect, rtol=1e-5, atol=1e-12,
                                   err_msg=f"segment {segment} layer {seg.layer} head {seg.head}")
        offset += seg.count
    assert offset == scores.size


@pytest.mark.parametrize("dim,groups", [(128, 4), (256, 6)])
def test_fused_scorer_sharply_peaked_rows(device, dim, groups):
    """Sharply peaked rows (queries scaled 6x: the top key's p within 1e-3 or less of 1). The
    ratio p / (1 - p) of that key is then ill-conditioned in f32 for any implementation of the
    formula (the reference's divides by 1 - p in f32, scoring.cu:101): an error of a few f32
    ulps in the row sum S becomes a relative error of about ulps * S / (S - 1) in the ratio.
    Scores must agree with the f64 oracle within that conditioning bound, and nine in ten of
    them within rtol 1e-5."""
    window = 90
    layers, qpos = _peaked_layers(dim, groups, window, 6.0, device)
    margin = torch.tensor([2.0], device=device)
    plan = scoring.plan_segments(layers, protect_prompt=True, protect_recent=32)
    scores = to_np(scoring.score_plan(plan, qpos, margin))
    offset = 0
    within = total = 0
    for segment, seg in enumerate(plan.segments):
        layer = layers[seg.layer]
        start = plan.head_starts[segment]
        length = int(plan.table[segment, 5])
        logits = _check_segment_logits(plan, layers, segment, device)
        positions = to_np(layer.positions[start:start + length])
        q = to_np(layer.queries[seg.head * groups:(seg.head + 1) * groups]).transpose(1, 0, 2)
        expect = oscoring.head_scores(
            q, qpos.cpu().numpy(), to_np(layer.keys[start:start + length]), positions,
            to_np(layer.values[start:start + length]), seg.position_start,
            seg.position_start + seg.count,
            to_np(layer.gradient[seg.head * groups:(seg.head + 1) * groups]), np.float32(2.0),
            1e-6, logits=logits)
        # conditioning of the segment's worst row: S / max(S - 1, eps * S) with S = sum
        # exp(z - max z) (the clamp bounds it by 1 / eps)
        z = logits.astype(np.float64)
        visible = positions[None, None, :] <= qpos.cpu().numpy()[:, None, None]
        z = np.where(visible, z, -np.inf)
        row_sum = np.exp(z - z.max(axis=2, keepdims=True)).sum(axis=2)
        condition = float(np.max(row_sum / np.maximum(row_sum - 1.0, 1e-6 * row_sum)))
        bound = max(1e-5, 64 * 2.0 ** -24 * condition)
        got = scores[offset:offset + seg.count]
        np.testing.assert_allclose(got, expect, rtol=bound, atol=1e-12,
                                   err_msg=f"segment {segment}: conditioning {condition:.3g}")
        within += int(np.sum(np.abs(got - expect) <= 1e-5 * np.abs(expect) + 1e-12))
        total += got.size
        offset += seg.count
    assert within >= 0.9 * total, (within, total)


def _scores_with_stages(plan, qpos, margin, stages, device):
    segments = plan.segment_count
    nbytes = _lib.load().lr_score_workspace_bytes(segments, plan.groups, plan.window,
                                                  segments * plan.groups * plan.max_length)
    table = plan.part("table").to(device)
    workspace = torch.empty((nbytes,), dtype=torch.uint8, device=device)
    scores = torch.full((plan.total,), -1.0, dtype=torch.float32, device=device)
    _lib.call("lr_score_segments", table.data_ptr(), segments, plan.groups, plan.window,
              plan.dim, plan.max_length, plan.max_candidates, plan.query_stride,
              qpos.data_ptr(), margin.data_ptr(), float(1.0 / math.sqrt(plan.dim)), 1e-6,
              workspace.data_ptr(), nbytes, scores.data_ptr(), None, stages,
              torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize(device)
    return to_np(scores)


@pytest.mark.parametrize("dim,groups,window", [(64, 4, 250), (256, 6, 77), (256, 6, 512), (128, 4, 90)])
def test_power_of_two_scale_path_equals_general_form(device, dim, groups, window):
    """For d = 64 and 256 the scale 1/sqrt(d) is a power of two: the passes then skip the second
    bf16 rounding of each logit and fold the scale into the exp2 constant. That is exact, so
    the scores must equal, bit for bit, those of the general form (stages bit 8 forces it),
    including masked keys (some keys after every query) and NaN rows. d = 128 takes the
    general form either way."""
    head_lengths = [[700, 41, 680, 300], [170, 900, 33, 299]]
    layers, qpos = workloads.make_layers(head_lengths, groups, dim, window, device, seed=dim + window,
                                         gradient="lognormal")
    layers[0].positions[50:70] += 1.0e5   # head 0 of layer 0: keys after every query
    layers[1].queries.mul_(3.0)            # larger logits: more of them far from the row max
    plan = scoring.plan_segments(layers, protect_prompt=True, protect_recent=32)
    margin = torch.tensor([2.0], device=device)
    fast = _scores_with_stages(plan, qpos, margin, 0, device)
    general = _scores_with_stages(plan, qpos, margin, 8, device)
    assert np.isfinite(fast).mean() > 0.5
    np.testing.assert_array_equal(fast, general)


def test_fused_scorer_matches_reference_host_path(device):
    """Fused scores vs this package's drop-in of the reference host loop (torch.matmul logits +
    _C.temporal_probabilities + _C.temporal_risk). The only allowed differences come from
    torch's GEMM rounding a logit to the other bf16 neighbour."""
    config = workloads.AuditConfig("small", 2, 2, 4, 128, 700, 250, 50)
    layers, qpos, margin = workloads.make_audit(config, device, seed=3)
    table = scoring.compute_score_table(layers, qpos, margin)
    fused = to_np(table.scores)
    parts = []
    for seg in table.segments:
        layer = layers[seg.layer]
        start = seg.head * config.length
        rows = slice(start, start + config.length)
        mapped = layer.queries[seg.head * 4:(seg.head + 1) * 4].permute(1, 0, 2)
        parts.append(to_np(scoring.temporal_head_scores(
            mapped, qpos, layer.keys[rows], layer.positions[rows], layer.values[rows],
            seg.position_start, seg.position_start + seg.count,
            layer.gradient[seg.head * 4:(seg.head + 1) * 4], margin, 1e-6, 250)))
    reference = np.concatenate(parts)
    close = np.isclose(fused, reference, rtol=1e-5, atol=1e-12)
    assert close.mean() > 0.97, close.mean()
    np.testing.assert_allclose(fused, reference, rtol=2e-2)


def test_fused_scorer_nan_rules(device):
    """A fully masked query row, or a non-finite value row (it enters every row's output
    projection), makes every score of its head NaN (csrc/scoring.cu:46-66,103-121); other
    heads are unaffected."""
    layers, qpos = workloads.make_layers([[200, 200, 200]], 4, 64, 40, device, seed=9)
    layers[0].positions[0:200] += 1000.0  # head 0: every key is after every query
    layers[0].values[200 + 17, 3] = float("inf")  # head 1
    table = scoring.compute_score_table(layers, qpos, torch.tensor([2.0], device=device),
                                        check_finite=False)
    s = to_np(table.scores)
    assert np.isnan(s[:168]).all() and np.isnan(s[168:336]).all()
    assert np.isfinite(s[336:]).all()
    with pytest.raises(RuntimeError, match="non-finite"):
        scoring.compute_score_table(layers, qpos, torch.tensor([2.0], device=device))
