r"""Multi-scale deformable attention (MSDA): call context, policy and registry.

``msda`` is the entry point every caller uses; it keeps the reference's call
surface (sources/deformops/registry/msda.py:274-361): five positional tensors,
the keywords ``method``, ``softmax``, ``chunk_step`` and ``backend``, and the
backend options ``num_points``, ``channels_per_thread``, ``threads_per_block`` and
``fp32acc``, which this build accepts and ignores. ``torch.ops.deformops.msda`` and
``torch.ops.deformops.msda_softmax`` are the public operators with the reference's
schema (:365-412).
"""

from __future__ import annotations

import dataclasses
from typing import Any, Protocol, runtime_checkable

import torch
from torch import Tensor

from ..core.runtime import Method, is_training_from, resolve_method, sm_version_for
from ..core.sanitize import check_msda_call
from ._dispatch import Backend, Registry
from ._public_ops import define_public_op

__all__ = [
    "MSDABackend",
    "MSDAContext",
    "MSDAMethod",
    "apply_msda_method",
    "msda",
    "msda_method_to_aggregate",
    "resolve_method",
    "resolve_msda_attn",
    "select_backend",
]

MSDAMethod = Method


@dataclasses.dataclass(frozen=True)
class MSDAContext:
    """Summary of one call, the memo key of backend selection.

    ``num_queries`` is left out of equality so that varying resolutions do not
    grow the memo (reference registry/msda.py:40-88).
    """

    device: torch.device
    num_levels: int
    num_heads: int
    num_points: int
    dtype: torch.dtype
    sm_version: tuple[int, int]
    is_training: bool
    num_queries: int = dataclasses.field(compare=False)
    method: Method = Method.LINEAR
    #: Channels per head; 0 when unknown.
    head_dim: int = 0

    @classmethod
    def from_call(
        cls,
        value: Tensor,
        spatial_shapes: Tensor,
        sampling_locations: Tensor,
        attention_weights: Tensor,
        method: Method,
    ) -> MSDAContext:
        queries: int | torch.SymInt = sampling_locations.shape[1]
        return cls(
            device=value.device,
            num_levels=int(spatial_shapes.shape[0]),
            num_heads=int(value.shape[2]),
            num_points=int(sampling_locations.shape[4]),
            dtype=value.dtype,
            sm_version=sm_version_for(value.device),
            is_training=is_training_from(value, sampling_locations, attention_weights),
            num_queries=0 if isinstance(queries, torch.SymInt) else int(queries),
            method=method,
            head_dim=int(value.shape[3]),
        )


@runtime_checkable
class MSDABackend(Protocol):
    """What a backend adapter provides (reference registry/msda.py:91-146)."""

    @property
    def name(self) -> str: ...

    def supports(self, context: MSDAContext) -> bool: ...

    def forward(
        self,
        value: Tensor,
        spatial_shapes: Tensor,
        level_start_index: Tensor,
        sampling_locations: Tensor,
        attention_weights: Tensor,
        chunk_step: int,
        method: Method,
    ) -> Tensor: ...


def msda_method_to_aggregate(method: str | Method) -> int:
    """The integer code of a method: 1 for softmax, 0 for linear."""
    return 1 if Method(method) is Method.SOFTMAX else 0


def apply_msda_method(attention_weights: Tensor, method: str | Method) -> Tensor:
    """Normalize raw weights per ``method``; softmax runs over the joint ``L * P`` axis."""
    method = Method(method)
    if method is Method.LINEAR:
        return attention_weights
    if attention_weights.ndim == 5:  # noqa: PLR2004
        flat = attention_weights.flatten(-2)
        return torch.softmax(flat, -1).unflatten(-1, attention_weights.shape[-2:])
    if attention_weights.ndim != 4:  # noqa: PLR2004
        msg = (
            f"attention weights must be (B, Q, G, L * K) or (B, Q, G, L, K); "
            f"got {attention_weights.ndim} dimensions."
        )
        raise ValueError(msg)
    return torch.softmax(attention_weights, -1)


def resolve_msda_attn(attention_weights: Tensor, method: str | Method) -> tuple[Tensor, int]:
    """``(weights, aggregate)``: softmax stays raw for an in-kernel softmax (code 1)."""
    aggregate = msda_method_to_aggregate(method)
    if aggregate == 1:
        return attention_weights, 1
    return apply_msda_method(attention_weights, method), 0


def select_backend(context: MSDAContext) -> list[Backend | tuple[Backend, dict[str, Any]]]:
    """Candidate backends for a ``backend=None`` call, in order.

    GPU tensors (torch device type ``"cuda"``, which is HIP on ROCm) run the HIP
    kernels, float64 included. CPU tensors ask for the eager backend, which this
    build does not ship, so they raise :class:`~deformops_amd.core.errors.NoBackendError`
    with that reason instead of silently running a CPU path.
    """
    if context.device.type != "cuda":
        return [Backend.EAGER]
    return [Backend.HIP]


#: Keywords a backend consumes besides method/softmax (reference registry/msda.py:216-218).
_CALL_OPTIONS: frozenset[str] = frozenset(
    {"chunk_step", "num_points", "channels_per_thread", "threads_per_block", "fp32acc"}
)


def _checked_arguments(
    level_start_index: Tensor | None,
    sampling_locations: Tensor | None,
    attention_weights: Tensor | None,
    options: dict[str, Any],
) -> tuple[Tensor, Tensor, Tensor]:
    if level_start_index is None or sampling_locations is None or attention_weights is None:
        msg = (
            "msda takes (values, spatial_shapes, level_start_index, "
            "sampling_locations, attention_weights) positionally"
        )
        raise TypeError(msg)
    unknown = set(options) - _CALL_OPTIONS
    if unknown:
        msg = f"msda got unexpected keyword argument(s): {', '.join(sorted(unknown))}"
        raise TypeError(msg)
    return level_start_index, sampling_locations, attention_weights


def _context_of(  # noqa: PLR0913
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor | None = None,
    sampling_locations: Tensor | None = None,
    attention_weights: Tensor | None = None,
    *,
    method: str | Method | None = None,
    softmax: bool = False,
    **options: Any,
) -> MSDAContext:
    level_start_index, sampling_locations, attention_weights = _checked_arguments(
        level_start_index, sampling_locations, attention_weights, options
    )
    check_msda_call(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    return MSDAContext.from_call(
        value,
        spatial_shapes,
        sampling_locations,
        attention_weights,
        resolve_method(method, softmax=softmax),
    )


def _msda_call(  # noqa: PLR0913
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
    /,
    *,
    method: str | Method | None = None,
    softmax: bool = False,
    chunk_step: int = 128,
    backend: Backend | None = None,
) -> Tensor:
    r"""Multi-scale deformable attention on the MI355X HIP kernels.

    Samples every level of a flattened feature pyramid bilinearly at per-query,
    per-head locations and returns the weighted sum. ``B`` batch, ``S`` positions
    over all levels, ``G`` heads, ``D`` channels per head, ``Q`` queries, ``L``
    levels, ``K`` points per level. The five tensors are positional-only and may
    have any memory layout.

    Parameters
    ----------
    value
        The flattened feature pyramid, shape ``(B, S, G, D)``.
    spatial_shapes
        One ``(height, width)`` row per level, shape ``(L, 2)``, integer.
    level_start_index
        Where each level starts on the ``S`` axis, shape ``(L,)``, integer.
    sampling_locations
        Normalized ``(x, y)`` in ``[0, 1]``, shape ``(B, Q, G, L, K, 2)``; float32
        or the dtype of ``value`` (other floating dtypes are widened to float32).
    attention_weights
        Per-point weights, shape ``(B, Q, G, L * K)`` or ``(B, Q, G, L, K)``, with
        the dtype of ``value``.
    method
        ``"linear"`` (default) uses the weights as given; ``"softmax"`` normalizes
        them over the ``L * K`` points inside the kernel. ``None`` defers to
        ``softmax``.
    softmax
        ``True`` means ``method="softmax"`` when ``method`` is ``None``.
    chunk_step
        Accepted for compatibility and ignored: the HIP kernels take the whole
        batch in one launch.
    backend
        A :class:`Backend` member, or ``None`` for the public operator
        ``torch.ops.deformops.msda`` (or ``msda_softmax``).

    Returns
    -------
    The attended features, shape ``(B, Q, G * D)``, in the dtype of ``value``.

    Raises
    ------
    TypeError
        If ``backend`` is a raw string, an operand is missing, or a keyword is
        unknown.
    ValueError
        If the operands disagree in rank, size, dtype or device.
    NoBackendError
        If no backend can run the call: CPU tensors, or a shape the kernels do not
        cover; the message gives the reason.
    KernelUnavailableError
        If the HIP library is not built.

    Notes
    -----
    float32, float16, bfloat16 and float64 values run on the GPU. ``grad_value`` is
    summed in fp32 (fp64 for float64) by the single owner of each element and
    stored once in the value dtype; the backward uses no memory beyond the three
    gradient tensors.
    """
    raise NotImplementedError


msda = Registry("msda", context_of=_context_of, select=select_backend, describe=_msda_call)

_PUBLIC_SCHEMA = (
    "(Tensor value, Tensor spatial_shapes, Tensor level_start_index, "
    "Tensor sampling_locations, Tensor attention_weights) -> Tensor"
)
_LEVEL_TABLE = "the spatial shapes and level start offsets"

#: Keywords that override the policy, so such a call negotiates in Python.
_OVERRIDE_OPTIONS: frozenset[str] = _CALL_OPTIONS - {"chunk_step"}


def _public_kernel(method: Method) -> Any:
    def kernel(
        value: Tensor,
        spatial_shapes: Tensor,
        level_start_index: Tensor,
        sampling_locations: Tensor,
        attention_weights: Tensor,
    ) -> Tensor:
        return msda.run_selected(
            value,
            spatial_shapes,
            level_start_index,
            sampling_locations,
            attention_weights,
            method=method,
        )

    return kernel


define_public_op("msda", _PUBLIC_SCHEMA, _public_kernel(Method.LINEAR), shared={1: _LEVEL_TABLE, 2: _LEVEL_TABLE})
define_public_op(
    "msda_softmax", _PUBLIC_SCHEMA, _public_kernel(Method.SOFTMAX), shared={1: _LEVEL_TABLE, 2: _LEVEL_TABLE}
)


def _route_selected(  # noqa: PLR0913
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor | None = None,
    sampling_locations: Tensor | None = None,
    attention_weights: Tensor | None = None,
    *,
    method: str | Method | None = None,
    softmax: bool = False,
    **options: Any,
) -> Tensor:
    """Run a ``backend=None`` call through ``deformops::msda[_softmax]``."""
    if any(name in options for name in _OVERRIDE_OPTIONS):
        return msda.run_selected(
            value,
            spatial_shapes,
            level_start_index,
            sampling_locations,
            attention_weights,
            method=method,
            softmax=softmax,
            **options,
        )
    level_start_index, sampling_locations, attention_weights = _checked_arguments(
        level_start_index, sampling_locations, attention_weights, options
    )
    use_softmax = resolve_method(method, softmax=softmax) is Method.SOFTMAX
    op = torch.ops.deformops.msda_softmax if use_softmax else torch.ops.deformops.msda
    return op(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)


msda.route_selected_calls(_route_selected)
