"""Layers over the MSDA operator (reference ``sources/deformops/nn/__init__.py``)."""

from __future__ import annotations

from .msda import MSDAMethod, MultiScaleDeformAttn2d

__all__ = ["MSDAMethod", "MultiScaleDeformAttn2d"]
