"""Hugging Face multi-scale deformable attention on the MI355X MSDA operator.

Restates the reference ``integrations/transformers.py:1-282``: a drop-in for
Deformable DETR's parameter-free attention core, one for Mask2Former's pixel
decoder attention (which keeps the pretrained projections of the module it
replaces), and :func:`patch`, which swaps both kinds in a model. The sampling runs
on the HIP kernels through :func:`~deformops_amd.integrations._ops.run_msda`.
"""

from __future__ import annotations

import importlib.util
from typing import TYPE_CHECKING

import torch
from torch import Tensor, nn

from ._ops import run_msda
from ._patch import patch_modules

if TYPE_CHECKING:
    from ..registry import Backend, MSDABackend

if importlib.util.find_spec("transformers") is None:  # pragma: no cover
    msg = "deformops_amd.integrations.transformers needs the 'transformers' package"
    raise ModuleNotFoundError(msg)

try:
    from transformers.models.deformable_detr import modeling_deformable_detr as _detr
    from transformers.models.mask2former import modeling_mask2former as _m2f

    _UpstreamCore = _detr.MultiScaleDeformableAttention
    _UpstreamM2F = _m2f.Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention
except (ImportError, AttributeError) as exc:  # pragma: no cover
    import transformers

    msg = (
        f"transformers {transformers.__version__} does not define the multi-scale "
        f"deformable attention modules this integration replaces ({type(exc).__name__}: "
        f"{exc})"
    )
    raise ImportError(msg) from exc

__all__ = [
    "Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention",
    "MultiScaleDeformableAttention",
    "patch",
]


class MultiScaleDeformableAttention(_UpstreamCore):
    """Deformable DETR's attention core (no parameters) on the HIP kernels."""

    # Upstream tags the class for replacement by a Hub kernel; no name keeps this
    # forward in place.
    kernel_layer_name = None

    def __init__(self, *, backend: Backend | MSDABackend | None = None) -> None:
        super().__init__()
        self.backend = backend

    def forward(  # noqa: PLR0913
        self,
        value: Tensor,
        value_spatial_shapes: Tensor,
        value_spatial_shapes_list: list[tuple[int, int]],  # noqa: ARG002 - upstream's signature
        level_start_index: Tensor,
        sampling_locations: Tensor,
        attention_weights: Tensor,
        im2col_step: int,
    ) -> Tensor:
        """Upstream's call; the weights arrive normalized, so the method is linear."""
        return run_msda(
            value,
            value_spatial_shapes,
            level_start_index,
            sampling_locations,
            attention_weights,
            chunk_step=im2col_step,
            backend=self.backend,
        )


class Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(_UpstreamM2F):
    """Mask2Former's encoder attention on the HIP kernels.

    Built from the upstream module it replaces: the four projections are that
    module's own ``nn.Linear`` objects (shared, not copied), so pretrained weights
    and optimizer state carry over.
    """

    kernel_layer_name = None

    def __init__(self, other: _UpstreamM2F, *, backend: Backend | MSDABackend | None = None) -> None:
        super().__init__(
            embed_dim=other.d_model,
            num_heads=other.n_heads,
            n_levels=other.n_levels,
            n_points=other.n_points,
        )
        self.chunk_step = other.im2col_step
        self.backend = backend
        self.sampling_offsets = other.sampling_offsets
        self.attention_weights = other.attention_weights
        self.value_proj = other.value_proj
        self.output_proj = other.output_proj

    def forward(  # noqa: PLR0913
        self,
        hidden_states: Tensor,
        attention_mask: Tensor | None = None,
        encoder_hidden_states: Tensor | None = None,
        encoder_attention_mask: Tensor | None = None,  # noqa: ARG002 - upstream's signature
        position_embeddings: Tensor | None = None,
        reference_points: Tensor | None = None,
        spatial_shapes_list: list[tuple[int, int]] | None = None,
        level_start_index: Tensor | None = None,
        output_attentions: bool = False,  # noqa: ARG002, FBT001, FBT002 - upstream's signature
        spatial_shapes: Tensor | None = None,
    ) -> tuple[Tensor, Tensor]:
        """Upstream's contract: ``(output, attention weights (B, Q, H, L, P))``.

        ``attention_mask`` is ``True`` at padded value tokens. The levels come from
        ``spatial_shapes_list`` or, for older callers, the ``spatial_shapes`` tensor.
        """
        if spatial_shapes_list is None:
            if spatial_shapes is None:
                msg = "one of spatial_shapes_list or spatial_shapes is required"
                raise ValueError(msg)
            spatial_shapes_list = [(int(h), int(w)) for h, w in spatial_shapes.tolist()]
        if encoder_hidden_states is None or reference_points is None:
            msg = "encoder_hidden_states and reference_points are required"
            raise ValueError(msg)
        if position_embeddings is not None:
            hidden_states = hidden_states + position_embeddings

        B, Q, _ = hidden_states.shape
        S = encoder_hidden_states.shape[1]
        H, L, P = self.n_heads, self.n_levels, self.n_points
        if sum(h * w for h, w in spatial_shapes_list) != S:
            msg = (
                "Make sure to align the spatial shapes with the sequence length of the "
                "encoder hidden states"
            )
            raise ValueError(msg)

        value = self.value_proj(encoder_hidden_states)
        if attention_mask is not None:
            value = value.masked_fill(attention_mask[..., None], 0)
        value = value.view(B, S, H, self.d_model // H)
        offsets = self.sampling_offsets(hidden_states).view(B, Q, H, L, P, 2)
        weights = nn.functional.softmax(self.attention_weights(hidden_states).view(B, Q, H, L * P), -1)

        coords = reference_points.shape[-1]
        if coords == 2:  # noqa: PLR2004
            # Offsets are in pixels of each level: divide by (width, height).
            size = torch.tensor(
                [[w, h] for h, w in spatial_shapes_list],
                dtype=reference_points.dtype,
                device=reference_points.device,
            )
            locations = reference_points[:, :, None, :, None, :] + offsets / size[None, None, None, :, None, :]
        elif coords == 4:  # noqa: PLR2004
            # Boxes (cx, cy, w, h): offsets span half the box over the points.
            centre = reference_points[:, :, None, :, None, :2]
            half = reference_points[:, :, None, :, None, 2:] * 0.5
            locations = centre + offsets / P * half
        else:
            msg = f"Last dim of reference_points must be 2 or 4, but got {coords}"
            raise ValueError(msg)

        shapes = torch.as_tensor(spatial_shapes_list, dtype=torch.long, device=value.device)
        output = run_msda(
            value,
            shapes,
            level_start_index,
            locations,
            weights,
            chunk_step=self.chunk_step,
            backend=self.backend,
        )
        return self.output_proj(output), weights.view(B, Q, H, L, P)


def patch(
    model: nn.Module,
    *,
    backend: Backend | MSDABackend | None = None,
    strict: bool = True,
) -> nn.Module:
    """Replace the model's Hugging Face MSDA modules of both kinds, in place.

    Parameters
    ----------
    model
        A Hugging Face model (Deformable DETR, Mask2Former, or anything holding
        their attention modules).
    backend
        Backend of every replacement; ``None`` lets the registry choose per call.
    strict
        Raise when nothing matched (the installed ``transformers`` may name the
        modules differently).

    Returns
    -------
    ``model``.

    Raises
    ------
    RuntimeError
        If ``strict`` and no module was replaced.
    """
    return patch_modules(
        model,
        [
            (_UpstreamCore, lambda _old: MultiScaleDeformableAttention(backend=backend)),
            (
                _UpstreamM2F,
                lambda old: Mask2FormerPixelDecoderEncoderMultiscaleDeformableAttention(old, backend=backend),
            ),
        ],
        strict=strict,
    )
