"""The public ``deformops::`` operators and their vmap rule.

``torch.ops.deformops.msda`` and ``msda_softmax`` keep the reference's names and
schema (sources/deformops/registry/msda.py:365-412), so code and exported graphs
that name them work unchanged. Each has one ``CompositeImplicitAutograd`` kernel,
which runs the registry's choice: a traced graph records the public operator,
autograd and the fake kernels come from the backend's private operator beneath it.

vmap (reference contract: sources/deformops/registry/_vmap.py:19-82) folds the
mapped axis into the batch axis, so a vmapped call is one kernel launch over
``size * B`` images. The level tables describe every image of a batch alike; a
mapped table would need a different pyramid per image and is refused with
``RuntimeError``.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from typing import Any

import torch
import torch.library
from torch import Tensor

__all__ = ["NAMESPACE", "define_public_op"]

NAMESPACE = "deformops"

#: Held for the life of the process: a collected Library unregisters its operators.
_LIBRARY = torch.library.Library(NAMESPACE, "FRAGMENT")


class _FoldVmap:
    """vmap rule: every mapped tensor argument becomes batch-major over ``size * B``;
    unmapped ones are repeated ``size`` times; ``fixed`` positions must be unmapped."""

    def __init__(self, op: Callable[..., Any], fixed: Mapping[int, str]) -> None:
        self.op = op
        self.fixed = dict(fixed)

    def __call__(self, info: Any, in_dims: tuple[int | None, ...], *args: Any, **kwargs: Any) -> tuple[Any, Any]:
        size = info.batch_size
        folded = []
        for position, (arg, dim) in enumerate(zip(args, in_dims)):
            if position in self.fixed:
                if dim is not None:
                    raise RuntimeError(
                        f"{self.fixed[position]} cannot be mapped by vmap: one pyramid describes every "
                        f"image of the batch. Pass it with in_dims=None."
                    )
                folded.append(arg)
            elif not isinstance(arg, Tensor):
                folded.append(arg)
            elif dim is None:
                folded.append(arg.expand(size, *arg.shape).reshape(size * arg.shape[0], *arg.shape[1:]))
            else:
                moved = arg.movedim(dim, 0)
                folded.append(moved.reshape(size * moved.shape[1], *moved.shape[2:]))
        result = self.op(*folded, **kwargs)
        if isinstance(result, Tensor):
            return self._split(result, size), 0
        parts = tuple(self._split(r, size) for r in result)
        return parts, (0,) * len(parts)

    @staticmethod
    def _split(result: Tensor, size: int) -> Tensor:
        if result.dim() <= 1 and result.numel() == 0:  # an empty placeholder
            return result.new_empty((size, 0))
        return result.reshape(size, result.shape[0] // size, *result.shape[1:])


def define_public_op(name: str, schema: str, kernel: Callable[..., Any], *,
                     fixed: Mapping[int, str] | None = None) -> Any:
    """Define ``deformops::<name>`` with ``kernel`` as its composite implementation and
    the batch-folding vmap rule (``fixed``: positions vmap may not map, with their
    names). A name that already exists is returned as it is."""
    namespace = getattr(torch.ops, NAMESPACE)
    if hasattr(namespace, name):
        return getattr(namespace, name)
    _LIBRARY.define(name + schema)
    _LIBRARY.impl(name, kernel, "CompositeImplicitAutograd")
    op = getattr(namespace, name)
    torch.library.register_vmap(f"{NAMESPACE}::{name}", _FoldVmap(op, fixed or {}), lib=_LIBRARY)
    return op
