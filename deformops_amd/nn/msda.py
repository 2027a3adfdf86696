"""The multi-scale deformable attention layer over the MI355X MSDA operator.

Restates the reference module ``nn/msda.py:24-273`` (``MultiScaleDeformAttn2d``):
the same constructor, parameter names, initialization, state-dict upgrade and
forward contract, with the sampling done by :data:`deformops_amd.registry.msda`
(the HIP kernels). ``MSDAMethod`` is :class:`deformops_amd.core.runtime.Method`.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import Tensor, nn

from ..core.runtime import Method as MSDAMethod
from ..core.sanitize import check_2power, check_msda_params
from ..registry import Backend, MSDABackend

__all__ = ["MSDAMethod", "MultiScaleDeformAttn2d"]

# Deformable DETR's parameter names and this layer's (reference nn/msda.py:132-141).
_LEGACY_NAMES = {
    "sampling_offsets": "proj_offset",
    "attention_weights": "proj_weights",
    "value_proj": "proj_value",
    "output_proj": "proj_output",
}


class MultiScaleDeformAttn2d(nn.Module):
    r"""Multi-scale deformable attention (Deformable DETR, Zhu et al., ICLR 2021).

    For each query and head, a linear map of the query predicts ``num_levels *
    num_points`` sampling offsets around the query's reference point and one weight
    per sample. The projected value pyramid is sampled bilinearly at those places by
    the MSDA operator, the weighted samples are summed per head, and the heads are
    projected out.

    Parameters
    ----------
    dim
        Query and hidden width, split evenly over the heads.
    dim_value
        Width of the value tokens (projected to ``dim``); ``None`` means ``dim``.
    dim_output
        Output width; ``None`` means ``dim``.
    num_heads
        Heads; ``dim // num_heads`` must be a power of two.
    num_levels
        Pyramid levels.
    num_points
        Sampling points per head and level.
    method
        ``"softmax"`` (default) normalizes each head's weights jointly over its
        ``num_levels * num_points`` samples, inside the kernel; ``"linear"`` uses
        them as predicted. A :data:`MSDAMethod` member or its value.
    backend
        A :class:`~deformops_amd.registry.Backend` member; an
        :class:`~deformops_amd.registry.MSDABackend` adapter, called directly; or
        ``None`` for the registry's choice.
    chunk_step
        Passed to a pinned backend, for the reference's signature; the HIP kernels
        take the whole batch at once.

    Raises
    ------
    ValueError
        If a size is not positive, ``dim`` is not a multiple of ``num_heads``, or
        ``dim // num_heads`` is not a power of two.

    Notes
    -----
    Checkpoints saved with Deformable DETR's names (``sampling_offsets``,
    ``attention_weights``, ``value_proj``, ``output_proj``; state-dict metadata
    version below 2) load under this layer's names.
    """

    _version = 2

    def __init__(
        self,
        dim: int,
        dim_value: int | None = None,
        dim_output: int | None = None,
        *,
        num_heads: int,
        num_levels: int,
        num_points: int = 4,
        method: MSDAMethod | str = MSDAMethod.SOFTMAX,
        backend: Backend | MSDABackend | None = None,
        chunk_step: int = 128,
    ) -> None:
        super().__init__()
        check_msda_params(dim, num_heads, num_levels, num_points)
        check_2power(dim // num_heads)
        self.dim = dim
        self.num_heads = num_heads
        self.num_levels = num_levels
        self.num_points = num_points
        self.method = MSDAMethod(method)
        self.backend = backend
        self.chunk_step = chunk_step
        samples = num_heads * num_levels * num_points
        self.proj_offset = nn.Linear(dim, 2 * samples)
        self.proj_weights = nn.Linear(dim, samples)
        self.proj_value = nn.Linear(dim_value or dim, dim)
        self.proj_output = nn.Linear(dim, dim_output or dim)
        self._register_load_state_dict_pre_hook(self._upgrade_state_dict)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        """Deformable DETR's initialization (reference ``nn/msda.py:148-165``).

        Offsets start as a fixed pattern: head h looks along the direction at angle
        2 pi h / num_heads, scaled so that its larger coordinate is 1, and point k
        sits k + 1 steps out on every level. Weights start uniform; the value and
        output projections are Xavier-uniform with zero bias.
        """
        H, L, P = self.num_heads, self.num_levels, self.num_points
        angle = torch.arange(H, dtype=torch.float32) * (2.0 * math.pi / H)
        direction = torch.stack([torch.cos(angle), torch.sin(angle)], dim=-1)
        direction = direction / direction.abs().amax(dim=-1, keepdim=True)
        steps = torch.arange(1, P + 1, dtype=torch.float32).view(1, 1, P, 1)
        pattern = direction.view(H, 1, 1, 2) * steps  # (H, 1, P, 2)
        with torch.no_grad():
            self.proj_offset.weight.zero_()
            self.proj_offset.bias.copy_(pattern.expand(H, L, P, 2).reshape(-1))
            self.proj_weights.weight.zero_()
            self.proj_weights.bias.zero_()
        nn.init.xavier_uniform_(self.proj_value.weight)
        nn.init.zeros_(self.proj_value.bias)
        nn.init.xavier_uniform_(self.proj_output.weight)
        nn.init.zeros_(self.proj_output.bias)

    def _upgrade_state_dict(
        self,
        state_dict: dict[str, Tensor],
        prefix: str,
        local_metadata: dict[str, Any],
        *args: Any,  # noqa: ARG002
        **kwargs: Any,  # noqa: ARG002
    ) -> None:
        version = local_metadata.get("version", 1)
        if isinstance(version, int) and version >= self._version:
            return
        for old, new in _LEGACY_NAMES.items():
            for part in ("weight", "bias"):
                key = f"{prefix}{old}.{part}"
                if key in state_dict:
                    state_dict[f"{prefix}{new}.{part}"] = state_dict.pop(key)
        # Other unknown keys stay, so a strict load still reports them.

    def sampling_locations(self, q: Tensor, p: Tensor, spatial_shapes: Tensor) -> Tensor:
        """The normalized sampling places ``(B, Q, heads, levels, points, 2)``.

        ``p`` holds reference points ``(x, y)`` (offsets are in pixels of each level,
        divided by its width and height) or boxes ``(cx, cy, w, h)`` (offset / points
        * (w, h) / 2 around the centre), per query and level (reference
        ``nn/msda.py:216-228``).
        """
        B, Q, _ = q.shape
        off = self.proj_offset(q).view(B, Q, self.num_heads, self.num_levels, self.num_points, 2)
        if p.shape[-1] == 2:  # noqa: PLR2004
            size = spatial_shapes.flip(-1).to(off.dtype)  # (L, 2): (width, height)
            return p[:, :, None, :, None, :] + off / size[None, None, None, :, None, :]
        if p.shape[-1] == 4:  # noqa: PLR2004
            centre = p[:, :, None, :, None, :2]
            half = p[:, :, None, :, None, 2:] * 0.5
            return centre + off / self.num_points * half
        msg = f"reference points must end in 2 (x, y) or 4 (cx, cy, w, h) values, got {p.shape[-1]}"
        raise ValueError(msg)

    def forward(  # noqa: PLR0913
        self,
        q: Tensor,
        p: Tensor,
        v: Tensor,
        spatial_shapes: Tensor,
        level_start_index: Tensor,
        padding_mask: Tensor | None = None,
    ) -> Tensor:
        """Attend ``v`` at places predicted from ``q``.

        Parameters
        ----------
        q
            Queries ``(B, Q, dim)``.
        p
            Reference points ``(B, Q, levels, 2)`` or boxes ``(B, Q, levels, 4)``,
            normalized to ``[0, 1]``.
        v
            The flattened value pyramid ``(B, N, dim_value)``, levels in the order of
            ``spatial_shapes``.
        spatial_shapes
            Integer ``(height, width)`` per level, ``(levels, 2)``.
        level_start_index
            Integer start of each level in ``v`` (exclusive prefix sum of
            ``height * width``), ``(levels,)``.
        padding_mask
            Boolean ``(B, N)``, ``True`` at padded tokens, whose projected values are
            zeroed; or ``None``.

        Returns
        -------
        The attended queries ``(B, Q, dim_output)``.
        """
        B, Q, _ = q.shape
        N = v.shape[1]
        value = self.proj_value(v)
        if padding_mask is not None:
            value = value.masked_fill(padding_mask[..., None], 0.0)
        value = value.view(B, N, self.num_heads, self.dim // self.num_heads)
        weights = self.proj_weights(q).view(B, Q, self.num_heads, self.num_levels * self.num_points)
        loc = self.sampling_locations(q, p, spatial_shapes)
        if isinstance(self.backend, MSDABackend):
            out = self.backend.forward(
                value, spatial_shapes, level_start_index, loc, weights, self.chunk_step, self.method
            )
        else:
            from ..registry import msda  # noqa: PLC0415

            options: dict[str, Any] = {"method": self.method, "backend": self.backend}
            if self.backend is not None:
                options["chunk_step"] = self.chunk_step
            out = msda(value, spatial_shapes, level_start_index, loc, weights, **options)
        return self.proj_output(out)

    def extra_repr(self) -> str:
        return (
            f"dim={self.dim}, num_heads={self.num_heads}, num_levels={self.num_levels}, "
            f"num_points={self.num_points}, method={self.method.value}"
        )
