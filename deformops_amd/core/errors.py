"""Exceptions and warnings raised when the MSDA operator cannot run.

Same taxonomy as the reference (sources/deformops/core/errors.py:15-47), so code
written against deformops catches the same classes.
"""

from __future__ import annotations

__all__ = [
    "BackendFallbackWarning",
    "KernelBuildError",
    "KernelDownloadError",
    "KernelNotProvidedError",
    "KernelUnavailableError",
    "NoBackendError",
]


class KernelUnavailableError(RuntimeError):
    """The compiled kernel library could not be made available."""


class KernelNotProvidedError(KernelUnavailableError):
    """The library is not built, and building it was not allowed.

    ``backend=None`` selection treats this as "backend unavailable"; an explicit
    backend request raises it.
    """


class KernelDownloadError(KernelUnavailableError):
    """Kept for interface parity; this build never downloads kernels."""


class KernelBuildError(KernelUnavailableError):
    """Compiling the library with hipcc was allowed and failed."""


class NoBackendError(RuntimeError):
    """No backend can run an operator call."""


class BackendFallbackWarning(UserWarning):
    """``backend=None`` ran a backend other than its first choice.

    Set ``DEFORMOPS_FALLBACK_WARNINGS=0`` to silence it.
    """
