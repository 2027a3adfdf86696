r"""Multi-scale deformable attention (MSDA): call context, selection policy, entry points.

``msda`` is the entry every caller uses. Its call surface is the reference's
(sources/deformops/registry/msda.py:274-361): five positional tensors, the keywords
``method``, ``softmax``, ``chunk_step`` and ``backend``, and the backend options
``num_points``, ``channels_per_thread``, ``threads_per_block`` and ``fp32acc``,
which the HIP kernels accept and ignore. ``torch.ops.deformops.msda`` and
``msda_softmax`` are the public operators.

A ``backend=None`` call goes through the public operator, so that ``torch.compile``,
``torch.export``, vmap and fake tensors see it. A plain eager call (real tensors, no
tracing, no dispatch or function mode) would only re-enter this module through the
operator's composite kernel and validate its operands twice; it runs the selected
backend directly instead.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Protocol, runtime_checkable

import torch
from torch import Tensor

from ..core.runtime import Method, is_training_from, resolve_method, sm_version_for
from ..core.sanitize import check_msda_call
from ._dispatch import Backend, Registry
from ._public import define_public_op

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
    """What backend selection knows of a call (fields as the reference's,
    registry/msda.py:40-88). ``num_queries`` is left out of equality, and is 0 when
    symbolic; ``head_dim`` is 0 when unknown. ``num_positions`` (S, the value rows of
    one image; 0 when symbolic or unknown) is this build's own addition, also left out
    of equality: a backend's addressable image size depends on it."""

    device: torch.device
    num_levels: int
    num_heads: int
    num_points: int
    dtype: torch.dtype
    sm_version: tuple[int, int]
    is_training: bool
    num_queries: int = dataclasses.field(compare=False)
    method: Method = Method.LINEAR
    head_dim: int = 0
    num_positions: int = dataclasses.field(default=0, compare=False)

    @classmethod
    def from_call(cls, value: Tensor, spatial_shapes: Tensor, sampling_locations: Tensor,
                  attention_weights: Tensor, method: Method) -> MSDAContext:
        """The context of a call; the tensors may be fake, with symbolic sizes."""
        B, Q, H, L, P, _ = sampling_locations.shape
        return cls(
            device=value.device,
            num_levels=int(spatial_shapes.shape[0]),
            num_heads=int(H),
            num_points=int(P),
            dtype=value.dtype,
            sm_version=sm_version_for(value.device),
            is_training=is_training_from(value, sampling_locations, attention_weights),
            num_queries=Q if isinstance(Q, int) else 0,
            method=method,
            head_dim=int(value.shape[3]),
            num_positions=value.shape[1] if isinstance(value.shape[1], int) else 0,
        )


@runtime_checkable
class MSDABackend(Protocol):
    """An adapter a layer can call directly (reference registry/msda.py:91-146)."""

    @property
    def name(self) -> str: ...

    def supports(self, context: MSDAContext) -> bool: ...

    def forward(self, value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor,
                sampling_locations: Tensor, attention_weights: Tensor, chunk_step: int,
                method: Method) -> Tensor: ...


def msda_method_to_aggregate(method: str | Method) -> int:
    """The kernels' integer code of a method: 1 for softmax, 0 for linear."""
    return int(Method(method) is Method.SOFTMAX)


def apply_msda_method(attention_weights: Tensor, method: str | Method) -> Tensor:
    """The weights ``method`` makes of raw ``attention_weights``: as given (linear), or a
    softmax over each (b, q, h)'s ``L * P`` points, flat ``(B, Q, H, L * P)`` or split
    ``(B, Q, H, L, P)``."""
    if Method(method) is Method.LINEAR:
        return attention_weights
    if attention_weights.ndim not in (4, 5):
        raise ValueError(
            f"attention weights are (B, Q, H, L * P) or (B, Q, H, L, P); got {attention_weights.ndim} "
            f"dimensions"
        )
    flat = attention_weights.reshape(*attention_weights.shape[:3], -1)
    return torch.softmax(flat, -1).reshape(attention_weights.shape)


def resolve_msda_attn(attention_weights: Tensor, method: str | Method) -> tuple[Tensor, int]:
    """``(weights, aggregate)`` for a kernel: softmax weights stay raw (the kernel applies
    it, code 1); linear ones pass as given (code 0)."""
    if msda_method_to_aggregate(method):
        return attention_weights, 1
    return apply_msda_method(attention_weights, method), 0


def select_backend(context: MSDAContext) -> list[Backend]:
    """The policy for ``backend=None``: GPU tensors (device type ``"cuda"``, HIP on
    ROCm) run the HIP kernels in every dtype, float64 included, and nothing else: a
    GPU call that the kernels cannot take raises ``NoBackendError``. CPU tensors run
    the eager backend, as in the reference (registry/msda.py:204-205)."""
    return [Backend.HIP] if context.device.type == "cuda" else [Backend.EAGER]


#: Keywords a backend consumes besides method / softmax (reference registry/msda.py:216-218).
_OPTIONS = frozenset({"chunk_step", "num_points", "channels_per_thread", "threads_per_block", "fp32acc"})
#: Of those, the ones that configure a particular backend: such a call skips the
#: public operator, whose schema cannot carry them.
_BACKEND_OPTIONS = _OPTIONS - {"chunk_step"}


def _operands(args: tuple[Any, ...], options: dict[str, Any]) -> tuple[Tensor, ...]:
    """The five positional tensors of a call; ``TypeError`` for a short call or an
    unknown keyword."""
    if len(args) != 5 or any(a is None for a in args):
        raise TypeError("msda takes (value, spatial_shapes, level_start_index, sampling_locations, "
                        f"attention_weights) positionally; got {len(args)} of them")
    unknown = sorted(name for name in options if name not in _OPTIONS)
    if unknown:
        raise TypeError(f"msda got unexpected keyword argument(s): {', '.join(unknown)}")
    return args


def _context_of(*args: Any, method: str | Method | None = None, softmax: bool = False,
                **options: Any) -> MSDAContext:
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = _operands(args, options)
    check_msda_call(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    return MSDAContext.from_call(value, spatial_shapes, sampling_locations, attention_weights,
                                 resolve_method(method, softmax=softmax))


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
        If no backend can run the call (a GPU shape the kernels do not cover, or a
        tensor on another device type); the message gives the reason.
    KernelUnavailableError
        If the HIP library is not built.

    Notes
    -----
    float32, float16, bfloat16 and float64 values run on the GPU, with fp32
    attention * bilinear weights (fp64 for float64). ``grad_value`` is summed in
    fp32 (fp64 for float64) by the single owner of each element and stored once;
    the backward uses no memory beyond the three gradient tensors. Valid levels
    that share positions of ``S`` sum their contributions into the shared
    ``grad_value`` elements. CPU tensors run torch operators in float32 (float64
    for float64 values), with the backward by autograd.
    """
    raise NotImplementedError


msda = Registry("msda", context_of=_context_of, select=select_backend, describe=_msda_call)

_SCHEMA = ("(Tensor value, Tensor spatial_shapes, Tensor level_start_index, "
           "Tensor sampling_locations, Tensor attention_weights) -> Tensor")
_TABLES = {1: "spatial_shapes", 2: "level_start_index"}


def _public_kernel(method: Method) -> Any:
    def kernel(value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor, sampling_locations: Tensor,
               attention_weights: Tensor) -> Tensor:
        return msda.run_selected(value, spatial_shapes, level_start_index, sampling_locations,
                                 attention_weights, method=method)

    return kernel


_PUBLIC = {
    Method.LINEAR: define_public_op("msda", _SCHEMA, _public_kernel(Method.LINEAR), fixed=_TABLES),
    Method.SOFTMAX: define_public_op("msda_softmax", _SCHEMA, _public_kernel(Method.SOFTMAX), fixed=_TABLES),
}


def _plain_eager(tensors: tuple[Tensor, ...]) -> bool:
    """Whether nothing would observe the public operator: not compiling or tracing, no
    dispatch or function mode (fake tensors, export), and real tensors that no
    functorch transform (vmap, grad) wraps."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack():  # noqa: SLF001
        return False
    if torch._C._is_torch_function_mode_enabled():  # noqa: SLF001
        return False
    wrapped = torch._C._functorch.is_functorch_wrapped_tensor  # noqa: SLF001
    return all(type(t) in (Tensor, torch.nn.Parameter) and not wrapped(t) for t in tensors)


def _route_selected(*args: Any, method: str | Method | None = None, softmax: bool = False,
                    **options: Any) -> Tensor:
    """A ``backend=None`` call: the public operator, or the same work directly when
    plain eager; backend options go to the selected backend."""
    if any(name in _BACKEND_OPTIONS for name in options):
        return msda.run_selected(*args, method=method, softmax=softmax, **options)
    tensors = _operands(args, options)
    chosen = resolve_method(method, softmax=softmax)
    if _plain_eager(tensors):
        return msda.run_selected(*tensors, method=chosen, **options)
    return _PUBLIC[chosen](*tensors)


msda.route_selected_calls(_route_selected)
