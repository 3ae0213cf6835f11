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


@dataclass(slots=True)
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


def _planner():
    try:
        from . import _plan
    except ImportError as error:
        raise _lib.LazyRecallLibraryError(
            "the host planner module _plan is not built; run `python -m code_for_iclr27_amd.build`"
        ) from error
    return _plan


class SegmentPlan:
    """Validated layers and the int64 metadata block of one audit (host side, no GPU work),
    built by the C++ planner in one pass (csrc/host_plan.cpp). Block layout:
    [segment table S x LR_SEG_WORDS | pool bounds S+1 | segment ends S | position starts S |
    head table (L*H) x LR_HEAD_WORDS]."""

    def __init__(self, block: torch.Tensor, meta, segment_info: torch.Tensor,
                 head_info: torch.Tensor, heads: int):
        self.block = block
        (self.segment_count, self.groups, self.window, self.dim, self.max_length,
         self.max_candidates, self.total, self.projected_floats, self.head_slots,
         self.rows_total, self.max_head_length, self.query_stride) = meta
        self.heads = heads
        self.segment_info = segment_info.numpy()     # [4, S]: layer, head, first, count
        self.head_info = head_info.numpy()           # [2, L*H]: segment or -1, length
        self._segments = None
        words = self.segment_count * _lib.LR_SEG_WORDS
        s = self.segment_count
        # (offset, length) of each part of the block, in words
        self.parts = {"table": (0, words), "bounds": (words, s + 1), "ends": (words + s + 1, s),
                      "starts": (words + 2 * s + 1, s),
                      "heads": (words + 3 * s + 1, self.head_slots * _lib.LR_HEAD_WORDS)}

    def part(self, name: str, source=None):
        offset, length = self.parts[name]
        return (self.block if source is None else source)[offset:offset + length]

    @property
    def table(self) -> np.ndarray:
        return self.part("table").numpy().reshape(self.segment_count, _lib.LR_SEG_WORDS)

    @property
    def cumulative_ends(self) -> List[int]:
        return self.part("ends").tolist()

    @property
    def layer_of(self) -> np.ndarray:
        return self.segment_info[0]

    @property
    def head_of(self) -> np.ndarray:
        return self.segment_info[1]

    @property
    def head_lengths(self) -> np.ndarray:
        return self.head_info[1].reshape(-1, self.heads)

    @property
    def head_starts(self) -> List[int]:
        """Row offset of each segment's head inside its layer."""
        lengths = self.head_lengths
        bases = np.cumsum(lengths, axis=1) - lengths
        return bases[self.layer_of, self.head_of].tolist()

    @property
    def segments(self) -> List[ScoreSegment]:
        if self._segments is None:
            info = self.segment_info
            self._segments = list(map(ScoreSegment, info[0].tolist(), info[1].tolist(),
                                      info[2].tolist(), info[3].tolist()))
        return self._segments


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def plan_segments(layers: Sequence[LayerState], protect_prompt: bool = True,
                  protect_recent: int = 32, pinned: bool = False) -> SegmentPlan:
    """Validate the layers and build the metadata block for every (layer, KV head) segment.
    Candidates of a head are [prompt_len, len - protect_recent) as in scoring.py:259-265; heads
    with none are skipped. Raises RuntimeError with the reference's messages on bad input."""
    _require(len(layers) > 0, "No layers to score")
    block, meta, segment_info, head_info = _planner().plan_audit(
        [layer.keys for layer in layers], [layer.values for layer in layers],
        [layer.positions for layer in layers], [layer.queries for layer in layers],
        [layer.gradient for layer in layers], [list(layer.head_lens) for layer in layers],
        [None if layer.prompt_lens is None else list(layer.prompt_lens) for layer in layers],
        bool(protect_prompt), int(protect_recent), bool(pinned))
    return SegmentPlan(block, meta, segment_info, head_info, len(layers[0].head_lens))


def score_plan(plan: SegmentPlan, query_positions: torch.Tensor, margin: torch.Tensor,
               denominator_epsilon: float = 1e-6, device=None) -> torch.Tensor:
    """Launch the fused scorer for a prepared plan; returns scores f32 [plan.total]."""
    device = device or query_positions.device
    _require(query_positions.is_cuda and query_positions.dtype == torch.int64
             and query_positions.numel() == plan.window, "Query positions do not match the window")
    margin = margin.to(device=device, dtype=torch.float32).reshape(1).contiguous()
    query_positions = query_positions.contiguous()
    segments = plan.segment_count
    workspace_bytes = _lib.load().lr_score_workspace_bytes(
        segments, plan.groups, plan.window, segments * plan.groups * plan.max_length)
    with torch.cuda.device(device):
        table = plan.part("table").to(device)
        workspace = torch.empty((workspace_bytes,), dtype=torch.uint8, device=device)
        scores = torch.empty((plan.total,), dtype=torch.float32, device=device)
        _lib.call("lr_score_segments", table.data_ptr(), segments, plan.groups, plan.window,
                  plan.dim, plan.max_length, plan.max_candidates, plan.query_stride,
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
        table = plan.part("table").to(device)
        out = torch.empty((plan.groups, plan.window, length), dtype=torch.bfloat16, device=device)
        _lib.call("lr_debug_segment_logits", table.data_ptr(), segment, plan.groups, plan.window,
                  plan.dim, length, plan.query_stride, out.data_ptr(), _lib.stream_of(out))
    return out
