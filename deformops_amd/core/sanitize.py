"""Operand validation for the MSDA entry points.

The contract is the reference's (sources/deformops/core/sanitize.py:56-146 for the
layer sizes, :276-436 for a call): a malformed call raises ``ValueError`` naming
the operand at fault, before any kernel launches, and reads tensor metadata only;
the level-table contents are read back to the host only when ``DEFORMOPS_VALIDATE``
is set, since that synchronizes the stream and breaks graph capture.

The structural check here is one pass of shape unification. Each operand has a
pattern over the symbols B (batch), S (positions), H (heads), D (channels), Q
(queries), L (levels) and P (points); a symbol is bound by the first operand that
has it and every later occurrence must agree. The HIP kernels treat a level whose
table entry does not fit the value tensor as empty, so a malformed table yields
zeros, never an out-of-bounds access, when the value checks are off.
"""

from __future__ import annotations

import os
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


def value_checks_enabled() -> bool:
    """Whether the checks that read the level table back to the host run (off by default)."""
    return os.getenv(VALIDATE_ENV_VAR, "0").strip().lower() not in {"", "0", "false", "no", "off"}


# Layer sizes.


def check_positive(n: int, name: str) -> None:
    """``ValueError`` unless ``n`` is a positive integer."""
    if not n > 0:
        raise ValueError(f"{name} must be a positive integer; got {n}")


def check_divisible(a: int, b: int) -> None:
    """``ValueError`` unless ``b`` is non-zero and divides ``a``."""
    if b == 0 or a % b:
        raise ValueError(f"{a} is not divisible by {b}")


def check_2power(n: int) -> None:
    """``ValueError`` unless ``n`` is a positive power of 2."""
    if n <= 0 or n & (n - 1):
        raise ValueError(f"expected a positive power of 2; got {n}")


def check_msda_params(dim: int, num_heads: int, num_levels: int, num_points: int) -> None:
    """The integers that size an MSDA layer: all positive, ``dim`` split evenly over heads."""
    for name, n in (("dim", dim), ("num_heads", num_heads), ("num_levels", num_levels),
                    ("num_points", num_points)):
        check_positive(n, name)
    check_divisible(dim, num_heads)


# One call.

#: Axis patterns of the five operands: symbols bind on first sight, integers are
#: fixed sizes. attention_weights takes either pattern.
_PATTERNS: tuple[tuple[str, tuple[tuple[str | int, ...], ...]], ...] = (
    ("value", (("B", "S", "H", "D"),)),
    ("spatial_shapes", (("L", 2),)),
    ("level_start_index", (("L",),)),
    ("sampling_locations", (("B", "Q", "H", "L", "P", 2),)),
    ("attention_weights", (("B", "Q", "H", "LP"), ("B", "Q", "H", "L", "P"))),
)

_MEANING = {
    "B": "the batch of value",
    "H": "the heads of value",
    "L": "the levels (rows of spatial_shapes)",
    "Q": "the queries of sampling_locations",
    "P": "the points of sampling_locations",
    "LP": "levels x points of sampling_locations",
}


def _unify(name: str, shape: tuple[int, ...], patterns: tuple[tuple[str | int, ...], ...],
           bound: dict[str, int]) -> None:
    """Match ``shape`` to the pattern of its rank; bind new symbols, check old ones."""
    pattern = next((p for p in patterns if len(p) == len(shape)), None)
    if pattern is None:
        ranks = " or ".join(str(len(p)) for p in patterns)
        raise ValueError(f"{name} must have {ranks} dimensions; got shape {tuple(shape)}")
    for axis, (symbol, size) in enumerate(zip(pattern, shape)):
        if isinstance(symbol, int):
            want, why = symbol, "its fixed size"
        elif symbol in bound:
            want, why = bound[symbol], _MEANING.get(symbol, symbol)
        else:
            bound[symbol] = size
            continue
        if size != want:
            raise ValueError(
                f"{name} has {size} entries on axis {axis} where {want} are expected "
                f"({why}); its shape is {tuple(shape)}"
            )


def check_msda_call(
    value: Tensor,
    spatial_shapes: Tensor,
    level_start_index: Tensor,
    sampling_locations: Tensor,
    attention_weights: Tensor,
) -> None:
    """Validate the five MSDA operands; ``ValueError`` names the first operand at fault.

    value ``(B, S, H, D)`` floating; spatial_shapes ``(L, 2)`` and level_start_index
    ``(L,)`` integer; sampling_locations ``(B, Q, H, L, P, 2)`` floating;
    attention_weights ``(B, Q, H, L * P)`` or ``(B, Q, H, L, P)`` in value's dtype;
    one device for all.
    """
    operands = (value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    bound: dict[str, int] = {}
    for (name, patterns), tensor in zip(_PATTERNS, operands):
        if name == "attention_weights" and "L" in bound and "P" in bound:
            bound["LP"] = bound["L"] * bound["P"]
        _unify(name, tuple(tensor.shape), patterns, bound)

    for (name, _), tensor in zip(_PATTERNS, operands):
        integral = name in ("spatial_shapes", "level_start_index")
        if integral and (tensor.is_floating_point() or tensor.is_complex()):
            raise ValueError(f"{name} indexes the value tensor and must be integer; got {tensor.dtype}")
        if not integral and not tensor.is_floating_point():
            raise ValueError(f"{name} must be floating point; got {tensor.dtype}")
    if attention_weights.dtype != value.dtype:
        raise ValueError(
            f"attention_weights is {attention_weights.dtype} while value is {value.dtype}; "
            f"give both one dtype (or run the call under autocast)"
        )
    devices = {tensor.device for tensor in operands}
    if len(devices) > 1:
        where = ", ".join(f"{name} on {t.device}" for (name, _), t in zip(_PATTERNS, operands))
        raise ValueError(f"the operands must share one device; got {where}")

    if value_checks_enabled() and _readable(spatial_shapes, level_start_index):
        _check_level_table(value, spatial_shapes, level_start_index)


def _readable(*tensors: Tensor) -> bool:
    """Whether the tensors hold data the host can read: not traced, fake or meta."""
    import torch  # noqa: PLC0415
    from torch._subclasses.fake_tensor import is_fake  # noqa: PLC0415

    if torch.compiler.is_compiling():
        return False
    return all(t.device.type != "meta" and not is_fake(t) for t in tensors)


def _check_level_table(value: Tensor, spatial_shapes: Tensor, level_start_index: Tensor) -> None:
    """The levels are non-empty, laid end to end from 0, and exactly fill value's S axis."""
    sizes = [(int(h), int(w)) for h, w in spatial_shapes.detach().cpu().tolist()]
    starts = [int(s) for s in level_start_index.detach().cpu().tolist()]
    empty = [i for i, (h, w) in enumerate(sizes) if h <= 0 or w <= 0]
    if empty:
        raise ValueError(f"spatial_shapes has an empty level at row {empty[0]}: {sizes[empty[0]]}")
    offsets = [0]
    for h, w in sizes:
        offsets.append(offsets[-1] + h * w)
    if starts != offsets[:-1]:
        raise ValueError(
            f"level_start_index is {starts}, but levels of sizes {[h * w for h, w in sizes]} laid end "
            f"to end start at {offsets[:-1]}"
        )
    if offsets[-1] != value.shape[1]:
        raise ValueError(
            f"spatial_shapes covers {offsets[-1]} positions but value has {value.shape[1]} on its "
            f"spatial axis"
        )
