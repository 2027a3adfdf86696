"""Operand validation for the MSDA entry points.

Restates the MSDA part of the reference's sources/deformops/core/sanitize.py:
structural checks (rank, axis sizes, dtype, device; :276-392) run on every call
and read metadata only; the level-table checks (:395-436) read the table back to
the host, so they run only when ``DEFORMOPS_VALIDATE`` is set. Every failure is a
``ValueError`` naming the operand, raised before any kernel launches.

The HIP kernels additionally treat a level whose table entry does not fit inside
the value tensor as empty, so a malformed table yields zeros instead of an
out-of-bounds access even when the value checks are off.
"""

from __future__ import annotations

import os
from collections.abc import Sequence
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from torch import Tensor

__all__ = [
    "VALIDATE_ENV_VAR",
    "check_2power",
    "check_divisible",
    "check_msda_call",
    "check_msda_params",
    "check_positive",
    "value_checks_enabled",
]

#: Enables the level-table checks; any value but a falsy spelling turns them on.
VALIDATE_ENV_VAR = "DEFORMOPS_VALIDATE"

_FALSY = frozenset({"0", "false", "no", "off", ""})


def value_checks_enabled() -> bool:
    """Whether to run the checks that read the level table back to the host.

    Off by default: the readback synchronizes the stream and breaks graph capture.
    """
    return os.getenv(VALIDATE_ENV_VAR, "0").strip().lower() not in _FALSY


def check_positive(n: int, name: str) -> None:
    """Raise ``ValueError`` unless ``n`` is a positive integer."""
    if n <= 0:
        msg = f"Expected {name} to be a positive integer, got: {n}"
        raise ValueError(msg)


def check_divisible(a: int, b: int) -> None:
    """Raise ``ValueError`` unless ``b`` is non-zero and divides ``a``."""
    if b == 0:
        msg = "Expected a non-zero divisor, got: 0"
        raise ValueError(msg)
    if a % b != 0:
        msg = f"Expected {a} to be divisible by {b}"
        raise ValueError(msg)


def check_2power(n: int) -> None:
    """Raise ``ValueError`` unless ``n`` is a positive power of two (reference
    ``core/sanitize.py:56-74``)."""
    if n <= 0:
        msg = f"Expected a positive integer, got: {n}"
        raise ValueError(msg)
    if n & (n - 1):
        msg = f"Expected a power of 2, got: {n}"
        raise ValueError(msg)


def check_msda_params(dim: int, num_heads: int, num_levels: int, num_points: int) -> None:
    """Check the integers that size an MSDA layer (reference ``core/sanitize.py:120-146``)."""
    check_positive(dim, "dim")
    check_positive(num_heads, "num_heads")
    check_positive(num_levels, "num_levels")
    check_positive(num_points, "num_points")
    check_divisible(dim, num_heads)


def _rank(name: str, tensor: Tensor, allowed: tuple[int, ...]) -> None:
    if tensor.dim() not in allowed:
        wanted = " or ".join(str(a) for a in allowed)
        msg = (
            f"{name} must be {wanted}-dimensional, got {tensor.dim()} dimensions "
            f"with shape {tuple(tensor.shape)}"
        )
        raise ValueError(msg)


def _axis(name: str, tensor: Tensor, axis: int, expected: int, why: str) -> None:
    actual = tensor.size(axis)
    if actual != expected:
        msg = (
            f"{name} has size {actual} on axis {axis}, expected {expected} ({why}). "
            f"Full shape: {tuple(tensor.shape)}"
        )
        raise ValueError(msg)


def _floating(name: str, tensor: Tensor) -> None:
    if not tensor.is_floating_point():
        msg = f"{name} must be a floating-point tensor, got dtype {tensor.dtype}"
        raise ValueError(msg)


def _integral(name: str, tensor: Tensor) -> None:
    if tensor.is_floating_point() or tensor.is_complex():
        msg = (
            f"{name} must be an integer tensor (it indexes the value tensor), "
            f"got dtype {tensor.dtype}"
        )
        raise ValueError(msg)


def _same_device(named: Sequence[tuple[str, Tensor]]) -> None:
    first_name, first = named[0]
    for name, tensor in named[1:]:
        if tensor.device != first.device:
            msg = (
                f"{name} is on {tensor.device} but {first_name} is on {first.device}; "
                f"all operands must share one device"
            )
            raise ValueError(msg)


def check_msda_call(
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
) -> None:
    """Validate the five MSDA operands; raise ``ValueError`` on the first mismatch.

    Shapes: value ``(B, S, H, D)``, spatial_shapes ``(L, 2)`` integer,
    level_start_index ``(L,)`` integer, sampling_locations ``(B, Q, H, L, P, 2)``
    floating, attention_weights ``(B, Q, H, L * P)`` or ``(B, Q, H, L, P)`` in the
    dtype of value. All on one device.
    """
    _rank("value", value, (4,))
    _rank("spatial_shapes", spatial_shapes, (2,))
    _rank("level_start_index", level_start_index, (1,))
    _rank("sampling_locations", sampling_locations, (6,))
    _rank("attention_weights", attention_weights, (4, 5))

    _axis("spatial_shapes", spatial_shapes, 1, 2, "each row is (height, width)")
    _axis(
        "sampling_locations",
        sampling_locations,
        5,
        2,
        "each location is a normalized (x, y) pair",
    )

    batch, _, heads, _ = value.shape
    levels = spatial_shapes.size(0)
    _, queries, _, loc_levels, points, _ = sampling_locations.shape

    _axis("level_start_index", level_start_index, 0, levels, "one entry per level")
    _axis("sampling_locations", sampling_locations, 0, batch, "batch of value")
    _axis("sampling_locations", sampling_locations, 2, heads, "heads of value")
    _axis("sampling_locations", sampling_locations, 3, levels, "rows of spatial_shapes")
    _axis("attention_weights", attention_weights, 0, batch, "batch of value")
    _axis("attention_weights", attention_weights, 1, queries, "queries of locations")
    _axis("attention_weights", attention_weights, 2, heads, "heads of value")
    if attention_weights.dim() == 4:
        _axis(
            "attention_weights",
            attention_weights,
            3,
            loc_levels * points,
            "levels x points of sampling_locations",
        )
    else:
        _axis("attention_weights", attention_weights, 3, loc_levels, "levels of sampling_locations")
        _axis("attention_weights", attention_weights, 4, points, "points of sampling_locations")

    _integral("spatial_shapes", spatial_shapes)
    _integral("level_start_index", level_start_index)
    _floating("value", value)
    _floating("attention_weights", attention_weights)
    if attention_weights.dtype != value.dtype:
        msg = (
            f"attention_weights has dtype {attention_weights.dtype} but value has "
            f"{value.dtype}; mixed input dtypes are not supported. Cast the operands "
            f"to a common dtype, or wrap the call in autocast"
        )
        raise ValueError(msg)
    _floating("sampling_locations", sampling_locations)
    _same_device(
        [
            ("value", value),
            ("spatial_shapes", spatial_shapes),
            ("level_start_index", level_start_index),
            ("sampling_locations", sampling_locations),
            ("attention_weights", attention_weights),
        ]
    )

    if value_checks_enabled() and _has_values(spatial_shapes, level_start_index):
        _check_level_layout(value, spatial_shapes, level_start_index)


def _has_values(*tensors: Tensor) -> bool:
    """Whether the tensors hold readable data: not fake and not being traced."""
    import torch  # noqa: PLC0415
    from torch._subclasses.fake_tensor import is_fake  # noqa: PLC0415

    if torch.compiler.is_compiling():
        return False
    return not any(is_fake(t) or t.device.type == "meta" for t in tensors)


def _check_level_layout(value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor) -> None:
    """The levels must be non-empty, start at the running offset and tile value."""
    shapes = spatial_shapes.detach().cpu().tolist()
    starts = level_start_index.detach().cpu().tolist()
    for level, (height, width) in enumerate(shapes):
        if height <= 0 or width <= 0:
            msg = (
                f"spatial_shapes row {level} is ({height}, {width}); every level "
                f"must have a positive height and width"
            )
            raise ValueError(msg)
    expected, running = [], 0
    for height, width in shapes:
        expected.append(running)
        running += height * width
    if starts != expected:
        msg = (
            f"level_start_index {starts} is not the exclusive prefix sum of the level "
            f"sizes {[h * w for h, w in shapes]}; expected {expected}"
        )
        raise ValueError(msg)
    if running != value.size(1):
        msg = (
            f"spatial_shapes describes {running} positions but value has "
            f"{value.size(1)} on its spatial axis; the levels must tile the value "
            f"tensor exactly"
        )
        raise ValueError(msg)
