"""Synthetic inputs of the benchmark configurations (no weights, no datasets).

cfg0  Llama-3.2-1B cache: L16 H8 d64, G=4, T=2250, W=250, evict 250 per (layer, head)
cfg1  Llama-3.1-8B cache: L32 H8 d128, G=4, T=2250, W=250, evict 250 per (layer, head)
cfg2  Llama-3.1-8B static batch of 8 requests, lengths U[1500, 2250], one-token batch append
cfg3  Llama-3.1-8B long budget: T=33792, 512 recalled rows per (layer, head), W=250
cfg4  Qwen3.5-style hybrid: 16 managed layers, H4 d256, G=6 (24 query heads, assumed),
      T=9216, W=512, evict 1024 per (layer, head), lognormal(0, 1.5) gradient weights

Distributions: K, V, Q ~ bf16(N(0,1)); key positions 0..T-1 per head; query positions
T-W..T-1; margin gradient |N(0,1)| (cfg4: lognormal(0, 1.5)); base margin 2.0.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from .scoring import LayerState


@dataclass(frozen=True)
class AuditConfig:
    name: str
    layers: int
    heads: int
    groups: int
    dim: int
    length: int
    window: int
    evict_per_head: int
    gradient: str = "abs_normal"
    margin: float = 2.0
    protect_recent: int = 32
    pool_kernel: int = 7
    epsilon: float = 1e-6

    @property
    def count(self) -> int:
        return self.evict_per_head * self.layers * self.heads


CONFIGS = {
    "cfg0": AuditConfig("cfg0-llama3.2-1b", 16, 8, 4, 64, 2250, 250, 250),
    "cfg1": AuditConfig("cfg1-llama3.1-8b", 32, 8, 4, 128, 2250, 250, 250),
    "cfg3": AuditConfig("cfg3-llama3.1-8b-long", 32, 8, 4, 128, 33792, 250, 1024),
    "cfg4": AuditConfig("cfg4-qwen3.5-hybrid", 16, 4, 6, 256, 9216, 512, 1024, "lognormal"),
}


def _randn(generator: torch.Generator, shape, device, dtype=torch.bfloat16) -> torch.Tensor:
    if generator.device.type == "cpu":
        return torch.randn(shape, generator=generator, dtype=torch.float32).to(device=device, dtype=dtype)
    return torch.randn(shape, generator=generator, device=device, dtype=torch.float32).to(dtype)


def make_layers(head_lengths: Sequence[Sequence[int]], groups: int, dim: int, window: int,
                device, seed: int = 0, gradient: str = "abs_normal",
                prompt_lengths: Optional[Sequence[Sequence[int]]] = None,
                generator_device: str = "cpu"):
    """Seeded layer states with per-head lengths ``head_lengths[layer][head]``. Key positions
    run 0..len-1 per head; queries sit at positions max_len-W .. max_len-1."""
    generator = torch.Generator(device=generator_device)
    generator.manual_seed(seed)
    layers: List[LayerState] = []
    max_len = max(max(lengths) for lengths in head_lengths)
    for layer_index, lengths in enumerate(head_lengths):
        heads = len(lengths)
        rows = int(sum(lengths))
        keys = _randn(generator, (rows, dim), device)
        values = _randn(generator, (rows, dim), device)
        positions = torch.cat([torch.arange(n, dtype=torch.float32) for n in lengths]).to(device)
        queries = _randn(generator, (heads * groups, window, dim), device)
        if gradient == "lognormal":
            grad = torch.exp(1.5 * _randn(generator, (heads * groups, dim), device, torch.float32))
        else:
            grad = _randn(generator, (heads * groups, dim), device, torch.float32).abs()
        prompts = None if prompt_lengths is None else list(prompt_lengths[layer_index])
        layers.append(LayerState(keys, values, positions, list(lengths), prompts,
                                 queries.contiguous(), grad.contiguous()))
    query_positions = torch.arange(max_len - window, max_len, dtype=torch.int64, device=device)
    return layers, query_positions


def make_audit(config: AuditConfig, device, seed: int = 0, generator_device: str = "cpu"):
    lengths = [[config.length] * config.heads for _ in range(config.layers)]
    layers, query_positions = make_layers(lengths, config.groups, config.dim, config.window,
                                          device, seed, config.gradient,
                                          generator_device=generator_device)
    margin = torch.tensor([config.margin], dtype=torch.float32, device=device)
    return layers, query_positions, margin
