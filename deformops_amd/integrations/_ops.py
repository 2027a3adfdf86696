"""The aggregation call the model integrations share (reference ``integrations/_ops.py:24-93``).

An integration computes its own sampling locations and weights and hands them,
with the projected value pyramid, to :func:`run_msda`.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from ..registry import Backend, MSDABackend, MSDAMethod, msda

__all__ = ["run_msda"]


def level_starts(spatial_shapes: Tensor) -> Tensor:
    """Exclusive prefix sum of ``height * width`` over the levels: ``(L,)``."""
    areas = spatial_shapes[:, 0] * spatial_shapes[:, 1]
    return torch.cat([areas.new_zeros(1), areas.cumsum(0)[:-1]])


def run_msda(  # noqa: PLR0913
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor | None,
    sampling_locations: Tensor,
    attention_weights: Tensor,
    *,
    chunk_step: int,
    backend: Backend | MSDABackend | None,
    method: MSDAMethod = MSDAMethod.LINEAR,
) -> Tensor:
    """Sum the bilinear samples of ``value`` weighted by ``attention_weights``.

    Parameters
    ----------
    value
        ``(B, S, H, D)``: S positions over all levels, H heads of D channels.
    spatial_shapes
        ``(L, 2)`` integer ``(height, width)`` per level.
    level_start_index
        ``(L,)`` start of each level in ``value``; ``None`` derives it from
        ``spatial_shapes``.
    sampling_locations
        ``(B, Q, H, L, P, 2)`` normalized ``(x, y)``.
    attention_weights
        ``(B, Q, H, L * P)`` or ``(B, Q, H, L, P)``.
    chunk_step
        The caller's batch chunk (Hugging Face's ``im2col_step``). Only a pinned
        backend receives it; the public operator has no such argument.
    backend
        A :class:`~deformops_amd.registry.Backend` member, an
        :class:`~deformops_amd.registry.MSDABackend` adapter (called directly, as
        ``torch.export`` needs), or ``None`` for the registry's choice.
    method
        ``LINEAR`` for weights that are already normalized, ``SOFTMAX`` for logits.

    Returns
    -------
    ``(B, Q, H * D)``.
    """
    starts = level_starts(spatial_shapes) if level_start_index is None else level_start_index
    if isinstance(backend, MSDABackend):
        return backend.forward(
            value, spatial_shapes, starts, sampling_locations, attention_weights, chunk_step, method
        )
    options: dict[str, Any] = {"method": method, "backend": backend}
    if backend is not None:
        options["chunk_step"] = chunk_step
    return msda(value, spatial_shapes, starts, sampling_locations, attention_weights, **options)
