"""TEST INFRASTRUCTURE ONLY: torch restatement of the reference eager MSDA backend.

Follows sources/deformops/backends/eager/msda_pytorch.py:23-112: the pixel map
``loc * size - 0.5`` in the input dtype, ``floor``, four clamped corner gathers by
advanced indexing, per-corner two-sided masks folded into the bilinear weights,
and the weighted sum over (level, point). It materializes ``(B, Q, H, L, P, D)``
per corner. Differentiable: torch autograd through it is the reference's own
backward (the eager backend has no hand-written one), so it pins the C oracle's
gradients independently. Also the CPU baseline that bench.py times (the
reference's CPU path, run with torch's CPU threads).

NaN or infinite locations give NaN here, as in the reference eager backend; the
GPU kernels and the C oracle skip such samples, as the reference CUDA kernel does.
"""

from __future__ import annotations

import torch
from torch import Tensor

__all__ = ["eager_msda", "softmax_weights"]


def softmax_weights(attention_weights: Tensor) -> Tensor:
    """Softmax over the joint ``L * P`` axis, for flat or split weights."""
    if attention_weights.dim() == 5:  # noqa: PLR2004
        return torch.softmax(attention_weights.flatten(-2), -1).view_as(attention_weights)
    return torch.softmax(attention_weights, -1)


def eager_msda(
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
    *,
    softmax: bool = False,
) -> Tensor:
    """``(B, Q, H * D)`` in the dtype of value; weights flat or split."""
    batch, _, heads, channels = value.shape
    _, queries, _, levels, points, _ = sampling_locations.shape
    weights = softmax_weights(attention_weights) if softmax else attention_weights
    weights = weights.reshape(batch, queries, heads, levels, points)

    dtype, device = value.dtype, value.device
    level_h = spatial_shapes[:, 0].long().view(1, 1, 1, levels, 1)
    level_w = spatial_shapes[:, 1].long().view(1, 1, 1, levels, 1)
    level_start = level_start_index.long().view(1, 1, 1, levels, 1)

    px = sampling_locations[..., 0] * level_w.to(dtype) - 0.5
    py = sampling_locations[..., 1] * level_h.to(dtype) - 0.5
    left = torch.floor(px).long()
    top = torch.floor(py).long()
    fx = px - left.to(px.dtype)
    fy = py - top.to(py.dtype)

    batch_ix = torch.arange(batch, device=device).view(batch, 1, 1, 1, 1)
    head_ix = torch.arange(heads, device=device).view(1, 1, heads, 1, 1)
    out = None
    for oy, ox in ((0, 0), (0, 1), (1, 0), (1, 1)):
        cx, cy = left + ox, top + oy
        inside = (cx >= 0) & (cx < level_w) & (cy >= 0) & (cy < level_h)
        flat = level_start + cy.clamp(min=0).minimum(level_h - 1) * level_w
        flat = flat + cx.clamp(min=0).minimum(level_w - 1)
        corner = value[batch_ix, flat, head_ix]  # (B, Q, H, L, P, D)
        wx = fx if ox else 1 - fx
        wy = fy if oy else 1 - fy
        bilinear = (wx * wy * inside.to(px.dtype)).to(dtype).unsqueeze(-1)
        term = bilinear * corner
        out = term if out is None else out + term
    assert out is not None
    return (out * weights.unsqueeze(-1)).sum(dim=(3, 4)).reshape(batch, queries, heads * channels)
