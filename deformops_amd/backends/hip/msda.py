r"""Registry adapter of the HIP MSDA kernels (reference: backends/cuda/msda.py:14-51)."""

from __future__ import annotations

from typing import Any

import torch

from ...core.runtime import Method, resolve_method
from ...registry import Backend, msda
from . import _lib
from ._bridge import forward, supports_context


def msda_hip(
    value: Any,
    spatial_shapes: Any,
    level_start_index: Any,
    sampling_locations: Any,
    attention_weights: Any,
    *,
    chunk_step: int = 128,
    num_points: int | None = None,
    channels_per_thread: int = 0,
    threads_per_block: int = 0,
    method: Any = None,
    softmax: bool = False,
    **kwargs: Any,  # noqa: ARG001 - backend options of other builds (fp32acc)
) -> Any:
    """Run MSDA on the gfx950 HIP kernels."""
    use_softmax = resolve_method(method, softmax=softmax) is Method.SOFTMAX
    return forward(
        value,
        spatial_shapes,
        level_start_index,
        sampling_locations,
        attention_weights,
        chunk_step,
        num_points=num_points,
        channels_per_thread=channels_per_thread,
        threads_per_block=threads_per_block,
        softmax=use_softmax,
    )


def load(*, download: bool | None = None, compile: bool | str | None = None) -> str:  # noqa: A002
    """Load libdeformops_amd.so and return its path."""
    return str(_lib.load(download=download, compile=compile).path)


if torch.cuda.is_available() and torch.version.hip is not None:
    msda.register(Backend.HIP, msda_hip, supports=supports_context, load=load)
else:
    msda.mark_unavailable(Backend.HIP, "no ROCm GPU is available to this process")
