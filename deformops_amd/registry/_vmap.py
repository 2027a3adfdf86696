"""vmap rule of the public operators: fold the vmapped axis into the batch axis.

Same contract as the reference (sources/deformops/registry/_vmap.py:39-82): a
vmapped call becomes one call over ``size * B`` samples, and batching an argument
that describes the batch (the level tables) raises ``RuntimeError``.
"""

from __future__ import annotations

import functools
from collections.abc import Callable, Mapping
from typing import Any

from torch import Tensor

__all__ = ["fold_into_batch", "make_vmap_rule", "unfold_from_batch"]


def fold_into_batch(tensor: Tensor, batch_dim: int | None, size: int) -> Tensor:
    """Merge the vmap axis into dim 0; an unbatched argument is expanded (copied)."""
    if batch_dim is None:
        return tensor.unsqueeze(0).expand(size, *tensor.shape).flatten(0, 1)
    return tensor.movedim(batch_dim, 0).flatten(0, 1)


def unfold_from_batch(tensor: Tensor, size: int) -> Tensor:
    """Split dim 0 back into ``(size, B)``; an empty placeholder becomes ``(size, 0)``."""
    if tensor.numel() == 0 and tensor.dim() <= 1:
        return tensor.new_empty((size, 0))
    return tensor.unflatten(0, (size, -1))


def _rule(
    info: Any,
    in_dims: tuple[int | None, ...],
    *args: Any,
    op: Callable[..., Any],
    shared: Mapping[int, str],
    **kwargs: Any,
) -> tuple[Any, Any]:
    for position, description in shared.items():
        if position < len(in_dims) and in_dims[position] is not None:
            msg = (
                f"vmap over {description} is not supported: it describes the batch "
                f"rather than varying across it. Pass it with in_dims=None."
            )
            raise RuntimeError(msg)
    size = info.batch_size
    folded = [
        fold_into_batch(arg, in_dims[i], size)
        if isinstance(arg, Tensor) and i not in shared
        else arg
        for i, arg in enumerate(args)
    ]
    result = op(*folded, **kwargs)
    if isinstance(result, Tensor):
        return unfold_from_batch(result, size), 0
    parts = tuple(unfold_from_batch(r, size) for r in result)
    return parts, tuple(0 for _ in parts)


def make_vmap_rule(
    op: Callable[..., Any], *, shared: Mapping[int, str] | None = None
) -> Callable[..., tuple[Any, Any]]:
    """The vmap rule of ``op``; ``shared`` maps batch-describing positions to names."""
    return functools.partial(_rule, op=op, shared=shared or {})
