r"""MSDA on the CPU in torch operators (reference: backends/eager/msda.py:12-36 and
backends/eager/msda_pytorch.py:23-150).

The reference routes CPU tensors to an eager backend (registry/msda.py:204-205);
this is this build's, registered as ``Backend.EAGER`` for CPU contexts only. It
has the kernels' semantics:

- pixel coordinates ``x = loc_x * W - 0.5``, ``y = loc_y * H - 0.5``;
- a sample counts when ``-1 <= x < W`` and ``-1 <= y < H``, and a corner when it
  lies in the level, with zero padding; non-finite locations contribute nothing;
- a level whose shape or start does not fit ``S`` contributes nothing;
- softmax over each (b, q, h)'s ``L * P`` points for ``method="softmax"``.

The work is laid out head-major: each (batch, head) pair is one row block of
``value``, and per level each bilinear corner is one ``gather`` of ``D``-element
rows followed by a batched product with the corner weights, so nothing of size
``[B, Q, H, L, P, D]`` stays alive beyond one corner of one level. 16-bit operands
compute in float32 and float64 in float64; the output takes ``value``'s dtype.
The backward is torch autograd (``gather`` scatters ``grad_value`` with fp32
adds), and levels that share positions of ``S`` sum into shared elements. Only
tensor operations are used (no host reads of the level tables), so the function
traces.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from ...core.runtime import Method, resolve_method
from ...registry import Backend as RegistryBackend
from ...registry import MSDAContext, apply_msda_method, msda

__all__ = ["Backend", "forward", "msda_eager"]


def _compute_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def _level_sum(rows: Tensor, xy: Tensor, weights: Tensor, height: Tensor, width: Tensor,
               start: Tensor, valid: Tensor) -> Tensor:
    """One level's weighted bilinear samples, summed over the points.

    rows ``[N, S, D]``; xy ``[N, Q, P, 2]`` normalized; weights ``[N, Q, P]``;
    height, width, start and valid are 0-dim tensors. Returns ``[N, Q, D]``.
    """
    N, Q, P, _ = xy.shape
    D = rows.shape[-1]
    hf, wf = height.to(xy.dtype), width.to(xy.dtype)
    px = xy[..., 0] * wf - 0.5
    py = xy[..., 1] * hf - 0.5
    inside = valid & (px >= -1) & (px < wf) & (py >= -1) & (py < hf)
    zero = torch.zeros((), dtype=xy.dtype)
    px = torch.where(inside, px, zero)
    py = torch.where(inside, py, zero)
    fx0, fy0 = torch.floor(px), torch.floor(py)
    dx, dy = px - fx0, py - fy0
    ix, iy = fx0.to(torch.int64), fy0.to(torch.int64)
    w_in = torch.where(inside, weights, zero)
    total = rows.new_zeros((N * Q, 1, D))
    for oy, wy in ((0, 1 - dy), (1, dy)):
        cy = iy + oy
        for ox, wx in ((0, 1 - dx), (1, dx)):
            cx = ix + ox
            hit = inside & (cx >= 0) & (cx < width) & (cy >= 0) & (cy < height)
            coef = torch.where(hit, wx * wy * w_in, zero)
            cxc = torch.minimum(cx.clamp(min=0), width - 1)
            cyc = torch.minimum(cy.clamp(min=0), height - 1)
            index = (start + cyc * width + cxc).reshape(N, Q * P, 1).expand(N, Q * P, D)
            picked = torch.gather(rows, 1, index).reshape(N * Q, P, D)
            total = total + torch.bmm(coef.reshape(N * Q, 1, P), picked)
    return total.reshape(N, Q, D)


def forward(value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor, sampling_locations: Tensor,
            attention_weights: Tensor) -> Tensor:
    """MSDA with weights as given: ``(B, Q, H * D)`` in ``value``'s dtype.

    value ``(B, S, H, D)``; spatial_shapes ``(L, 2)`` as (height, width);
    level_start_index ``(L,)``; sampling_locations ``(B, Q, H, L, P, 2)``;
    attention_weights ``(B, Q, H, L * P)`` or ``(B, Q, H, L, P)``.
    """
    B, S, H, D = value.shape
    _, Q, _, L, P, _ = sampling_locations.shape
    ct = _compute_dtype(value.dtype)
    N = B * H
    rows = value.to(ct).transpose(1, 2).reshape(N, S, D)
    xy = sampling_locations.to(ct).transpose(1, 2).reshape(N, Q, L, P, 2)
    weights = attention_weights.to(ct).reshape(B, Q, H, L, P).transpose(1, 2).reshape(N, Q, L, P)
    shapes = spatial_shapes.to(torch.int64)
    starts = level_start_index.to(torch.int64)
    one = torch.ones((), dtype=torch.int64)
    out = rows.new_zeros((N, Q, D))
    for lvl in range(L):
        height, width, start = shapes[lvl, 0], shapes[lvl, 1], starts[lvl]
        valid = (height > 0) & (width > 0) & (start >= 0) & (start + height * width <= S)
        # An invalid level samples a 1 x 1 level at 0 with every weight masked.
        height = torch.where(valid, height, one)
        width = torch.where(valid, width, one)
        start = torch.where(valid, start, 0 * one)
        out = out + _level_sum(rows, xy[:, :, lvl], weights[:, :, lvl], height, width, start, valid)
    return out.reshape(B, H, Q, D).transpose(1, 2).reshape(B, Q, H * D).to(value.dtype)


class Backend:
    """Dispatch adapter of the CPU path (the MSDABackend protocol; reference
    backends/eager/msda_pytorch.py:115-150). It takes CPU tensors only."""

    @property
    def name(self) -> str:
        return "eager"

    def supports(self, context: MSDAContext) -> bool:
        return supports_context(context)

    def forward(self, value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor,
                sampling_locations: Tensor, attention_weights: Tensor, chunk_step: int,  # noqa: ARG002
                method: Method) -> Tensor:
        _check_cpu(value)
        # The softmax runs in the compute dtype, on the weights widened first.
        weights = apply_msda_method(attention_weights.to(_compute_dtype(value.dtype)), method)
        return forward(value, spatial_shapes, level_start_index, sampling_locations, weights)


def supports_context(context: MSDAContext) -> bool:
    """CPU tensors of a floating dtype."""
    return context.device.type == "cpu" and context.dtype.is_floating_point


def _check_cpu(value: Tensor) -> None:
    if value.device.type != "cpu":
        msg = f"the eager MSDA backend runs on CPU tensors only; got a tensor on {value.device}"
        raise RuntimeError(msg)


_BACKEND = Backend()


def msda_eager(
    value: Any,
    spatial_shapes: Any,
    level_start_index: Any,
    sampling_locations: Any,
    attention_weights: Any,
    *,
    chunk_step: int = 128,
    method: Any = None,
    softmax: bool = False,
    **kwargs: Any,  # noqa: ARG001 - backend options of the GPU path (num_points, ...)
) -> Any:
    """Run MSDA on the CPU in torch operators."""
    return _BACKEND.forward(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                            chunk_step, resolve_method(method, softmax=softmax))


msda.register(RegistryBackend.EAGER, msda_eager, supports=supports_context)
