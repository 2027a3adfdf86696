"""Operator dispatch: the MSDA registry, its call context and the public operators.

Import through this package, as with the reference::

    from deformops_amd.registry import Backend, msda
"""

from __future__ import annotations

from ..core.runtime import resolve_method
from ._dispatch import Backend, LoadedBackend, Registry, Resolution
from .msda import (
    MSDABackend,
    MSDAContext,
    MSDAMethod,
    apply_msda_method,
    msda,
    msda_method_to_aggregate,
    resolve_msda_attn,
    select_backend,
)

__all__ = [
    "Backend",
    "LoadedBackend",
    "MSDABackend",
    "MSDAContext",
    "MSDAMethod",
    "Registry",
    "Resolution",
    "apply_msda_method",
    "msda",
    "msda_method_to_aggregate",
    "resolve_method",
    "resolve_msda_attn",
    "select_backend",
]
