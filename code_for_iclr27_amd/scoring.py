"""Score-table construction on the GPU.

Two entry points:

* ``temporal_head_scores`` — the reference's GPU host path for one KV head
  (src/lazy_recall/scoring.py:152-195), calling this package's ``_C.temporal_probabilities``
  and ``_C.temporal_risk`` exactly where the reference calls ``lazy_recall._C``.
* ``compute_score_table`` — the same scores for every (layer, KV head) of an audit in one
  fused launch sequence (``lr_score_segments``), replacing the reference's per-head Python
  loop (src/lazy_recall/scoring.py:218-287). Segment rules (prompt protection, recent
  protection, skipped heads, cumulative ends) follow that loop.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _C, _lib


@dataclass(frozen=True)
class ScoreSegment:
    """_core/scoring.py:198-203"""
    layer: int
    head: int
    position_start: int
    count: int


@dataclass
class ScoreTable:
    """_core/scoring.py:206-211"""
    scores: torch.Tensor
    segments: List[ScoreSegment]
    cumulative_ends: List[int]
    score_ms: float


@dataclass
class LayerState:
    """What the scorer reads from one layer of a LazyRecallCache plus its query history:
    keys/values [rows, d] bf16 in the flat per-head layout (_core/cache.py:104-105), positions
    [rows] or [rows, 1] f32 (cache.py:21), per-head lengths and frozen prompt lengths
    (_core/cache.py:15-26), the query history [Hq, W, d] bf16 (history.py:51-63 without the
    leading batch axis) and the pre-projection margin gradient [Hq, d] f32 (scoring.py:228-237)."""
    keys: torch.Tensor
    values: torch.Tensor
    positions: torch.Tensor
    head_lens: Sequence[int]
    prompt_lens: Optional[Sequence[int]]
    queries: torch.Tensor
    gradient: torch.Tensor


def temporal_head_scores(queries, query_positions, keys, key_positions, values, candidate_start,
                         candidate_end, margin_gradient, base_margin, denominator_epsilon,
                         query_chunk_size):
    """scoring.py:152-195 (GPU branch) with this package's ``_C`` ops."""
    if not keys.is_cuda:
        raise RuntimeError("temporal_head_scores requires CUDA tensors (no CPU fallback)")
    if queries.ndim != 3 or queries.shape[-1] != keys.shape[-1]:
        raise ValueError("Invalid temporal query dimensions")
    if keys.shape != values.shape or key_positions.numel() != keys.shape[0]:
        raise ValueError("KV and position shapes differ")
    if query_positions.numel() != queries.shape[0] or queries.shape[0] == 0:
        raise ValueError("Query positions do not match the nonempty history")
    if not 0 <= candidate_start < candidate_end <= keys.shape[0]:
        raise ValueError("Invalid candidate interval")
    if query_chunk_size <= 0 or denominator_epsilon <= 0:
        raise ValueError("Chunk size and denominator epsilon must be positive")
    projected = torch.matmul(margin_gradient.float(), values.float().transpose(0, 1)).contiguous()
    key_positions = key_positions.to(dtype=torch.float32).contiguous()
    query_positions = query_positions.to(dtype=torch.int64).contiguous()
    margin = base_margin.to(device=keys.device, dtype=torch.float32).reshape(1).contiguous()
    bytes_per_query = queries.shape[1] * keys.shape[0] * (keys.element_size() + 4)
    chunk = min(query_chunk_size, max(1, (64 * 1024 ** 2) // bytes_per_query))
    result = None
    for start in range(0, queries.shape[0], chunk):
        end = min(start + chunk, queries.shape[0])
        logits = torch.matmul(queries[start:end].to(keys.dtype), keys.transpose(0, 1))
        probabilities, projection = _C.temporal_probabilities(
            logits.contiguous(), projected, query_positions[start:end], key_positions,
            1.0 / math.sqrt(keys.shape[-1]))
        scores = _C.temporal_risk(probabilities, projection, projected, margin, candidate_start,
                                  candidate_end, denominator_epsilon)
        result = scores if result is None else torch.maximum(result, scores)
    return result


@dataclass
class SegmentPlan:
    table: np.ndarray            # int64 [segments, LR_SEG_WORDS]
    segments: List[ScoreSegment]
    cumulative_ends: List[int]
    head_starts: List[int]       # row offset of each segment's head inside its layer
    groups: int
    window: int
    dim: int
    max_length: int
    max_candidates: int
    projected_floats: int
    layer_of: Optional[np.ndarray] = None   # segment -> layer
    head_of: Optional[np.ndarray] = None    # segment -> KV head
    head_lengths: Optional[np.ndarray] = None  # [layers, heads] lengths of every head
    pointers: Optional[np.ndarray] = None   # [layers, 5] keys/values/positions/queries/gradient

    @property
    def total(self) -> int:
        return self.cumulative_ends[-1] if self.cumulative_ends else 0


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _validate_layer(layer: LayerState, hq: int, window: int, dim: int, device) -> None:
    """Detailed checks with the error messages; only run when the fast check fails."""
    keys, values, positions = layer.keys, layer.values, layer.positions
    for tensor in (keys, values, positions, layer.queries, layer.gradient):
        _require(tensor.is_cuda and tensor.is_contiguous() and tensor.device == device,
                 "Expected contiguous CUDA tensor")
    _require(keys.dtype == torch.bfloat16 and values.dtype == torch.bfloat16
             and layer.queries.dtype == torch.bfloat16,
             "The fused scorer takes bf16 keys, values and queries")
    _require(keys.dim() == 2 and keys.shape == values.shape and keys.size(1) == dim,
             "Invalid KV layout")
    _require(positions.dtype == torch.float32 and positions.numel() == keys.size(0),
             "Invalid positions")
    _require(tuple(layer.queries.shape) == (hq, window, dim), "Historical query-head count changed")
    _require(layer.gradient.dtype == torch.float32 and tuple(layer.gradient.shape) == (hq, dim),
             "Invalid margin gradient")
    for tensor in (keys, values, layer.queries):
        _require(tensor.data_ptr() % 16 == 0, "bf16 operands must be 16-byte aligned")
    heads = len(layer.head_lens)
    _require(heads > 0 and hq % heads == 0, "Query heads must be a multiple of KV heads")
    _require(int(np.sum(layer.head_lens)) == keys.size(0), "Position/KV lengths differ")
    raise RuntimeError("Inconsistent layer state")


def plan_segments(layers: Sequence[LayerState], protect_prompt: bool = True,
                  protect_recent: int = 32) -> SegmentPlan:
    """Validate the layers and build the device segment table (host side, no GPU work).
    Every head of every layer is planned in one vectorised pass."""
    _require(len(layers) > 0, "No layers to score")
    first_layer = layers[0]
    hq, window, dim = first_layer.queries.shape
    device = first_layer.keys.device
    bf16, f32 = torch.bfloat16, torch.float32
    count = len(layers)
    pointers = np.empty((count, 5), dtype=np.int64)
    rows = np.empty(count, dtype=np.int64)
    heads = len(first_layer.head_lens)
    lengths_list, prompts_list = [], []
    any_prompt = False
    qshape, gshape = (hq, window, dim), (hq, dim)
    for index, layer in enumerate(layers):
        k, v, p, q, g = layer.keys, layer.values, layer.positions, layer.queries, layer.gradient
        kp, vp, qp = k.data_ptr(), v.data_ptr(), q.data_ptr()
        ok = (k.dtype == bf16 and v.dtype == bf16 and q.dtype == bf16 and p.dtype == f32
              and g.dtype == f32 and k.device == device and v.device == device
              and p.device == device and q.device == device and g.device == device
              and k.dim() == 2 and k.shape == v.shape and k.shape[1] == dim
              and p.numel() == k.shape[0] and q.shape == qshape and g.shape == gshape
              and k.is_contiguous() and v.is_contiguous() and p.is_contiguous()
              and q.is_contiguous() and g.is_contiguous() and (kp | vp | qp) % 16 == 0
              and len(layer.head_lens) == heads and k.is_cuda)
        if not ok:
            _require(len(layer.head_lens) == heads, "Every layer must have the same number of KV heads")
            _validate_layer(layer, hq, window, dim, device)
        pointers[index] = (kp, vp, p.data_ptr(), qp, g.data_ptr())
        rows[index] = k.shape[0]
        lengths_list.append(layer.head_lens)
        if protect_prompt and layer.prompt_lens is not None:
            any_prompt = True
        prompts_list.append(layer.prompt_lens)
    _require(heads > 0 and hq % heads == 0, "Query heads must be a multiple of KV heads")
    groups = hq // heads
    lengths = np.asarray(lengths_list, dtype=np.int64)                      # [L, H]
    if not np.array_equal(lengths.sum(axis=1), rows):
        for layer in layers:
            _validate_layer(layer, hq, window, dim, device)
    bases = np.cumsum(lengths, axis=1) - lengths                            # row of each head
    starts = np.zeros_like(lengths)
    if any_prompt:
        for index, prompt in enumerate(prompts_list):
            if prompt is not None:
                starts[index] = np.asarray(prompt, dtype=np.int64)
    ends = np.maximum(starts, lengths - protect_recent)
    layer_of, head_of = np.nonzero(ends > starts)                            # row-major order
    if not layer_of.size:
        raise RuntimeError("No eligible KV remains after prompt/recent protection")
    base = bases[layer_of, head_of]
    seg_lengths = lengths[layer_of, head_of]
    seg_starts = starts[layer_of, head_of]
    seg_ends = ends[layer_of, head_of]
    counts = seg_ends - seg_starts
    table = np.zeros((layer_of.size, _lib.LR_SEG_WORDS), dtype=np.int64)
    table[:, 0] = pointers[layer_of, 0] + base * dim * 2
    table[:, 1] = pointers[layer_of, 1] + base * dim * 2
    table[:, 2] = pointers[layer_of, 2] + base * 4
    table[:, 3] = pointers[layer_of, 3] + head_of * groups * window * dim * 2
    table[:, 4] = pointers[layer_of, 4] + head_of * groups * dim * 4
    table[:, 5] = seg_lengths
    table[:, 6] = seg_starts
    table[:, 7] = seg_ends
    cumulative = np.cumsum(counts)
    table[:, 8] = cumulative - counts
    table[:, 9] = np.arange(layer_of.size, dtype=np.int64) * groups * window
    projected = np.cumsum(groups * seg_lengths)
    table[:, 10] = projected - groups * seg_lengths
    segments = list(map(ScoreSegment, layer_of.tolist(), head_of.tolist(), seg_starts.tolist(),
                        counts.tolist()))
    return SegmentPlan(table, segments, cumulative.tolist(), base.tolist(), groups, window, dim,
                       int(seg_lengths.max()), int(counts.max()), int(projected[-1]),
                       layer_of, head_of, lengths, pointers)


def score_plan(plan: SegmentPlan, query_positions: torch.Tensor, margin: torch.Tensor,
               denominator_epsilon: float = 1e-6, device=None) -> torch.Tensor:
    """Launch the fused scorer for a prepared plan; returns scores f32 [plan.total]."""
    device = device or query_positions.device
    _require(query_positions.is_cuda and query_positions.dtype == torch.int64
             and query_positions.numel() == plan.window, "Query positions do not match the window")
    margin = margin.to(device=device, dtype=torch.float32).reshape(1).contiguous()
    query_positions = query_positions.contiguous()
    segments = len(plan.segments)
    workspace_bytes = _lib.load().lr_score_workspace_bytes(
        segments, plan.groups, plan.window, segments * plan.groups * plan.max_length)
    with torch.cuda.device(device):
        table = _C.upload_int64(plan.table, device)
        workspace = torch.empty((workspace_bytes,), dtype=torch.uint8, device=device)
        scores = torch.empty((plan.total,), dtype=torch.float32, device=device)
        _lib.call("lr_score_segments", table.data_ptr(), segments, plan.groups, plan.window,
                  plan.dim, plan.max_length, plan.max_candidates, plan.window,
                  query_positions.data_ptr(), margin.data_ptr(),
                  float(1.0 / math.sqrt(plan.dim)), float(denominator_epsilon),
                  workspace.data_ptr(), workspace_bytes, scores.data_ptr(), None, 0,
                  _lib.stream_of(scores))
    return scores


def compute_score_table(layers: Sequence[LayerState], query_positions: torch.Tensor,
                        margin: torch.Tensor, protect_prompt: bool = True,
                        protect_recent: int = 32, denominator_epsilon: float = 1e-6,
                        check_finite: bool = True) -> ScoreTable:
    """All segments' temporal scores in one fused pass (replaces scoring.py:218-293)."""
    started = time.perf_counter()
    plan = plan_segments(layers, protect_prompt, protect_recent)
    scores = score_plan(plan, query_positions, margin, denominator_epsilon)
    if check_finite and not bool(torch.isfinite(scores).all()):
        raise RuntimeError("LazyRecall produced non-finite scores; refusing to construct a deletion queue")
    return ScoreTable(scores, plan.segments, plan.cumulative_ends,
                      (time.perf_counter() - started) * 1000.0)


def debug_segment_logits(plan: SegmentPlan, segment: int, device) -> torch.Tensor:
    """Raw bf16 logits [G, W, T] of one segment, formed by the same MFMA sequence as the fused
    scorer (test hook for the parity suite)."""
    length = int(plan.table[segment, 5])
    with torch.cuda.device(device):
        table = _C.upload_int64(plan.table, device)
        out = torch.empty((plan.groups, plan.window, length), dtype=torch.bfloat16, device=device)
        _lib.call("lr_debug_segment_logits", table.data_ptr(), segment, plan.groups, plan.window,
                  plan.dim, length, plan.window, out.data_ptr(), _lib.stream_of(out))
    return out
