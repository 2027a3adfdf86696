"""Synthetic MSDA workloads: the five BASELINE configurations and small variants.

Shared by the tests and bench.py. Inputs are drawn on the CPU in float64 from a
seeded ``torch.Generator`` and then cast, so every dtype sees the same values:

- value ~ N(0, 1), shape (B, S, H, D);
- attention weights = softmax over L * P of N(0, 1) logits (``logits`` keeps the
  raw N(0, 1) draws for the softmax method);
- locations ~ U[-0.05, 1.05] (configs 0-3), or (config 4) each query's own
  normalized pixel centre at its level plus N(0, 0.05) per (head, level, point,
  coordinate), with a seeded 10% of samples forced out of bounds (x = -0.5 or 1.5);
- grad_out ~ N(0, 1), shape (B, Q, H * D).
"""

from __future__ import annotations

import dataclasses

import torch
from torch import Tensor

__all__ = ["CONFIGS", "Workload", "algorithmic_bytes", "make_workload"]

DETR_LEVELS = ((100, 134), (50, 67), (25, 34), (13, 17))


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    batch: int
    queries: int | None  # None: one query per pyramid position (encoder self-attention)
    levels: tuple[tuple[int, int], ...]
    heads: int = 8
    channels: int = 32
    points: int = 4
    locations: str = "uniform"  # or "reference"
    seed: int = 0


CONFIGS: dict[int, Config] = {
    0: Config("cpu-small", 1, None, ((32, 32), (16, 16), (8, 8)), seed=0),
    1: Config("detr-decoder", 4, 300, DETR_LEVELS, seed=1),
    2: Config("m2f-small", 2, None, ((64, 64), (32, 32), (16, 16)), seed=2),
    3: Config("detr-encoder", 2, None, DETR_LEVELS, seed=3),
    4: Config("m2f-large", 4, None, ((128, 128), (64, 64), (32, 32)), locations="reference", seed=4),
}


@dataclasses.dataclass
class Workload:
    value: Tensor
    spatial_shapes: Tensor
    level_start_index: Tensor
    sampling_locations: Tensor
    attention_weights: Tensor  # softmax-normalized, flat (B, Q, H, L * P)
    logits: Tensor  # the raw N(0, 1) draws
    grad_output: Tensor

    @property
    def sizes(self) -> tuple[int, int, int, int, int, int, int]:
        B, S, H, D = self.value.shape
        Q, L, P = self.sampling_locations.shape[1], self.spatial_shapes.shape[0], self.sampling_locations.shape[4]
        return B, S, H, D, Q, L, P

    def to(self, device: torch.device | str, dtype: torch.dtype, loc_dtype: torch.dtype | None = None) -> Workload:
        loc_dtype = dtype if loc_dtype is None else loc_dtype
        return Workload(
            self.value.to(device, dtype),
            self.spatial_shapes.to(device),
            self.level_start_index.to(device),
            self.sampling_locations.to(device, loc_dtype),
            self.attention_weights.to(device, dtype),
            self.logits.to(device, dtype),
            self.grad_output.to(device, dtype),
        )

    def operands(self, *, softmax: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
        weights = self.logits if softmax else self.attention_weights
        return self.value, self.spatial_shapes, self.level_start_index, self.sampling_locations, weights


def _level_tables(levels: tuple[tuple[int, int], ...]) -> tuple[Tensor, Tensor]:
    shapes = torch.tensor(levels, dtype=torch.int64).reshape(-1, 2)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])
    return shapes, starts


def _reference_points(levels: tuple[tuple[int, int], ...], queries: int) -> Tensor:
    """Normalized pixel centre ``(x, y)`` of each flattened pyramid position, (Q, 2)."""
    points = []
    for h, w in levels:
        ys, xs = torch.meshgrid(
            (torch.arange(h, dtype=torch.float64) + 0.5) / h,
            (torch.arange(w, dtype=torch.float64) + 0.5) / w,
            indexing="ij",
        )
        points.append(torch.stack([xs.flatten(), ys.flatten()], -1))
    ref = torch.cat(points)
    assert ref.shape[0] >= queries
    return ref[:queries]


def make_workload(
    config: Config | int,
    *,
    batch: int | None = None,
    queries: int | None = None,
    heads: int | None = None,
    channels: int | None = None,
    points: int | None = None,
    levels: tuple[tuple[int, int], ...] | None = None,
    locations: str | None = None,
    seed: int | None = None,
) -> Workload:
    """Float64 CPU inputs of a BASELINE configuration, optionally resized."""
    cfg = CONFIGS[config] if isinstance(config, int) else config
    levels = cfg.levels if levels is None else levels
    B = cfg.batch if batch is None else batch
    H = cfg.heads if heads is None else heads
    D = cfg.channels if channels is None else channels
    P = cfg.points if points is None else points
    mode = cfg.locations if locations is None else locations
    shapes, starts = _level_tables(levels)
    S = int((shapes[:, 0] * shapes[:, 1]).sum())
    Q = (cfg.queries if cfg.queries is not None else S) if queries is None else queries
    L = len(levels)
    g = torch.Generator().manual_seed(cfg.seed if seed is None else seed)
    f64 = torch.float64
    value = torch.randn(B, S, H, D, generator=g, dtype=f64)
    logits = torch.randn(B, Q, H, L * P, generator=g, dtype=f64)
    weights = torch.softmax(logits, -1)
    if mode == "uniform":
        loc = torch.rand(B, Q, H, L, P, 2, generator=g, dtype=f64) * 1.1 - 0.05
    elif mode == "reference":
        ref = _reference_points(levels, Q).view(1, Q, 1, 1, 1, 2)
        loc = ref + 0.05 * torch.randn(B, Q, H, L, P, 2, generator=g, dtype=f64)
        out = torch.rand(B, Q, H, L, P, generator=g, dtype=f64) < 0.1
        side = torch.where(torch.rand(B, Q, H, L, P, generator=g, dtype=f64) < 0.5, -0.5, 1.5)
        loc[..., 0] = torch.where(out, side.to(f64), loc[..., 0])
    else:
        raise ValueError(mode)
    grad = torch.randn(B, Q, H * D, generator=g, dtype=f64)
    return Workload(value, shapes, starts, loc, weights, logits, grad)


def algorithmic_bytes(B: int, S: int, H: int, D: int, Q: int, L: int, P: int, es: int, ls: int) -> tuple[int, int]:
    """Compulsory HBM bytes ``(forward, backward)`` of one call.

    forward  = es (B S H D + B Q H D) + ls 2 B Q H L P + es B Q H L P
    backward = reads (value, locations, weights, grad_out) + writes (grad_value,
               grad_loc, grad_attn); the zero-fill of grad_value is not counted.
    """
    samples = B * Q * H * L * P
    fwd = es * (B * S * H * D + B * Q * H * D) + ls * 2 * samples + es * samples
    bwd_reads = es * B * S * H * D + ls * 2 * samples + es * samples + es * B * Q * H * D
    bwd_writes = es * B * S * H * D + ls * 2 * samples + es * samples
    return fwd, bwd_reads + bwd_writes
