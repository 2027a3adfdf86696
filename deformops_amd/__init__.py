"""MI355X-native multi-scale deformable attention (MSDA).

A drop-in for deformops' MSDA operator on AMD Instinct MI355X (gfx950): the
``registry.msda`` call and the ``torch.ops.deformops.msda`` / ``msda_softmax``
operators, backed by hand-written HIP kernels: a forward, and a backward that
writes every element of ``grad_value`` once from fp32 registers (owner-computes,
no atomics on the gradient and no buffer beyond the three gradients).
"""

from __future__ import annotations

from .version import __version__

__all__ = ["__version__", "nn", "registry"]


def __getattr__(name: str):
    if name in ("registry", "core", "nn"):
        import importlib  # noqa: PLC0415

        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
