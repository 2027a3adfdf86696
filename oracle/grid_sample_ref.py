"""TEST INFRASTRUCTURE ONLY: MSDA as the reference defines it, on grid_sample.

Restates sources/deformops/backends/reference/msda.py:16-97: per level, sample
``value`` viewed as ``(B*H, D, h, w)`` with ``grid_sample(mode="bilinear",
padding_mode="zeros", align_corners=False)`` at ``2 * loc - 1``, then weight and
sum over (level, point). torch's grid_sample and its autograd are the library
routine the reference tests itself against.
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.nn.functional import grid_sample

__all__ = ["grid_sample_msda"]


def grid_sample_msda(
    value: Tensor,
    spatial_shapes: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
) -> Tensor:
    """``(B, Q, H * D)``; weights ``(B, Q, H, L, P)`` or flat, already normalized."""
    batch, _, heads, channels = value.shape
    _, queries, _, levels, points, _ = sampling_locations.shape
    weights = attention_weights.reshape(batch, queries, heads, levels * points)
    weights = weights.transpose(1, 2).reshape(batch * heads, 1, queries, levels * points)
    grid = 2 * sampling_locations - 1
    shapes = [(int(h), int(w)) for h, w in spatial_shapes.tolist()]
    offset = 0
    sampled = []
    for level, (h, w) in enumerate(shapes):
        part = value.narrow(1, offset, h * w)  # (B, h*w, H, D)
        offset += h * w
        image = part.flatten(2).transpose(1, 2).reshape(batch * heads, channels, h, w)
        g = grid[:, :, :, level].transpose(1, 2).flatten(0, 1)  # (B*H, Q, P, 2)
        sampled.append(
            grid_sample(image, g, mode="bilinear", padding_mode="zeros", align_corners=False)
        )  # (B*H, D, Q, P)
    stacked = torch.stack(sampled, dim=-2).flatten(-2)  # (B*H, D, Q, L*P)
    out = (stacked * weights).sum(-1)  # (B*H, D, Q)
    return out.view(batch, heads * channels, queries).transpose(1, 2).contiguous()
