"""Public ``deformops::`` operators whose single kernel runs the registry.

As in the reference (sources/deformops/registry/_public_ops.py:28-67), each public
operator has one ``CompositeImplicitAutograd`` kernel that selects a backend and
calls that backend's private operator, which carries the autograd, fake and
device kernels. The namespace is the reference's own, ``deformops``, so
``torch.ops.deformops.msda`` is the same call in both.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from typing import Any

import torch
import torch.library

from ._vmap import make_vmap_rule

__all__ = ["NAMESPACE", "define_public_op"]

NAMESPACE = "deformops"

#: Held for the life of the process: a collected Library unregisters its operators.
_LIBRARY = torch.library.Library(NAMESPACE, "FRAGMENT")


def define_public_op(
    name: str,
    schema: str,
    kernel: Callable[..., Any],
    *,
    shared: Mapping[int, str] | None = None,
) -> Any:
    """Define ``deformops::<name>`` with ``kernel`` and the batch-folding vmap rule.

    Idempotent: an operator that already exists is returned unchanged.
    """
    namespace = getattr(torch.ops, NAMESPACE)
    if hasattr(namespace, name):
        return getattr(namespace, name)
    _LIBRARY.define(f"{name}{schema}")
    _LIBRARY.impl(name, kernel, "CompositeImplicitAutograd")
    op = getattr(namespace, name)
    torch.library.register_vmap(f"{NAMESPACE}::{name}", make_vmap_rule(op, shared=shared), lib=_LIBRARY)
    return op
