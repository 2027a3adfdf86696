"""The aggregation-method enum and call-context helpers.

Restates sources/deformops/core/runtime.py:17-91: an explicit ``method`` wins,
``softmax=True`` selects SOFTMAX otherwise, and LINEAR is the default.
"""

from __future__ import annotations

import enum
import functools
from typing import TYPE_CHECKING

import torch

if TYPE_CHECKING:
    from torch import Tensor

__all__ = ["Method", "arch_for", "is_training_from", "resolve_method", "sm_version_for"]


class Method(str, enum.Enum):
    """How the operator normalizes its attention weights.

    ``"linear"`` uses the weights as given; ``"softmax"`` normalizes them jointly
    over the ``L * P`` points of each (batch, query, head). Every ``method``
    argument takes the member or its string value.
    """

    LINEAR = "linear"
    SOFTMAX = "softmax"

    def __str__(self) -> str:
        return self.value


def resolve_method(method: str | Method | None, *, softmax: bool = False) -> Method:
    """Resolve the aggregation method of one call.

    Raises
    ------
    ValueError
        If ``method`` names no method.
    """
    if method is not None:
        return Method(method)
    return Method.SOFTMAX if softmax else Method.LINEAR


@functools.cache
def sm_version_for(device: torch.device) -> tuple[int, int]:
    """The ``(major, minor)`` compute capability torch reports; ``(0, 0)`` off GPU.

    On ROCm torch reports the gfx target as a capability (gfx950 is ``(9, 5)``).
    """
    if device.type != "cuda" or not torch.cuda.is_available():
        return (0, 0)
    return torch.cuda.get_device_capability(device)


@functools.cache
def arch_for(device: torch.device) -> str:
    """The gfx architecture name of ``device`` (``"gfx950"`` on MI355X), or ``""``."""
    if device.type != "cuda" or not torch.cuda.is_available():
        return ""
    name = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
    return name.split(":")[0]


def is_training_from(*tensors: Tensor) -> bool:
    """Whether a backward pass could follow: grad mode on and an input requiring grad."""
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
