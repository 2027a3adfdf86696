"""Operator-agnostic pieces: method enum, errors and operand validation."""

from .errors import (
    BackendFallbackWarning,
    KernelBuildError,
    KernelDownloadError,
    KernelNotProvidedError,
    KernelUnavailableError,
    NoBackendError,
)
from .runtime import Method, is_training_from, resolve_method

__all__ = [
    "BackendFallbackWarning",
    "KernelBuildError",
    "KernelDownloadError",
    "KernelNotProvidedError",
    "KernelUnavailableError",
    "Method",
    "NoBackendError",
    "is_training_from",
    "resolve_method",
]
