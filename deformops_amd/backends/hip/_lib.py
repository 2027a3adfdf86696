"""ctypes binding of libdeformops_amd.so (the C ABI declared in include/deformops_amd.h).

The library is loaded once per process, on first use. A missing library raises
:class:`~deformops_amd.core.errors.KernelNotProvidedError` (or is built first when
the caller allows compiling); there is no fallback path.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from collections.abc import Iterator
from pathlib import Path

import torch

from ...core.errors import KernelBuildError, KernelNotProvidedError, KernelUnavailableError

__all__ = [
    "ABI_VERSION",
    "DTYPE_CODES",
    "FLAG_ACCUMULATE_GRAD_VALUE",
    "FLAG_GRAD_VALUE_ATOMIC",
    "FLAG_SOFTMAX",
    "PATH_ATOMIC_SORT",
    "PATH_NO_MFMA",
    "PATH_TILE8",
    "INDEX_CODES",
    "EXPORTED_SYMBOLS",
    "Library",
    "library_path",
    "load",
    "path_override",
]

#: MSDA_ABI_VERSION this binding was written for.
ABI_VERSION = 4

#: enum msda_dtype.
DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float64: 3,
}
#: enum msda_index_dtype.
INDEX_CODES: dict[torch.dtype, int] = {torch.int64: 0, torch.int32: 1}
#: enum msda_flags.
FLAG_SOFTMAX = 1
FLAG_ACCUMULATE_GRAD_VALUE = 2
FLAG_GRAD_VALUE_ATOMIC = 4
#: enum msda_path_bits.
PATH_NO_MFMA = 1
PATH_ATOMIC_SORT = 2
PATH_TILE8 = 4

#: Every function the header declares.
EXPORTED_SYMBOLS = (
    "msda_forward",
    "msda_backward",
    "msda_backward_workspace",
    "msda_backward_workspace_size",
    "msda_backward_no_alloc",
    "msda_last_error",
    "msda_abi_version",
    "msda_launch_geometry",
    "msda_set_path_override",
    "msda_set_phase_events",
)

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64


def library_path() -> Path:
    """Where the library is looked for: ``$DEFORMOPS_AMD_LIBRARY`` or the in-tree build."""
    override = os.environ.get("DEFORMOPS_AMD_LIBRARY")
    if override:
        return Path(override)
    return Path(__file__).resolve().parents[2] / "lib" / "libdeformops_amd.so"


class Library:
    """The loaded library with typed entry points."""

    def __init__(self, path: Path) -> None:
        self.path = path
        self.cdll = ctypes.CDLL(str(path))
        lib = self.cdll
        lib.msda_forward.argtypes = [_P, _I, _P, _P, _I, _P, _I, _P, _P, *([_L] * 7), _I, _P]
        lib.msda_forward.restype = _I
        lib.msda_backward.argtypes = [_P, _I, _P, _P, _I, _P, _I, _P, _P, _P, _P, _P, *([_L] * 7), _I, _P]
        lib.msda_backward.restype = _I
        lib.msda_backward_workspace.argtypes = [_P, _I, _P, _P, _I, _P, _I, _P, _P, _P, _P, _P, *([_L] * 7), _I, _P,
                                                _L, _P]
        lib.msda_backward_workspace.restype = _I
        lib.msda_backward_workspace_size.argtypes = [_I, *([_L] * 7), _I, ctypes.POINTER(_L)]
        lib.msda_backward_workspace_size.restype = _I
        lib.msda_backward_no_alloc.argtypes = lib.msda_backward.argtypes
        lib.msda_backward_no_alloc.restype = _I
        lib.msda_last_error.argtypes = []
        lib.msda_last_error.restype = ctypes.c_char_p
        lib.msda_abi_version.argtypes = []
        lib.msda_abi_version.restype = _I
        lib.msda_launch_geometry.argtypes = [
            _I, *([_L] * 7), _I,
            ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_L),
        ]
        lib.msda_launch_geometry.restype = _I
        lib.msda_set_path_override.argtypes = [_I]
        lib.msda_set_path_override.restype = _I
        lib.msda_set_phase_events.argtypes = [ctypes.POINTER(_P), _I]
        lib.msda_set_phase_events.restype = _I
        self.forward = lib.msda_forward
        self.backward = lib.msda_backward
        self.backward_workspace = lib.msda_backward_workspace
        self.backward_no_alloc = lib.msda_backward_no_alloc

    def workspace_size(self, dtype: torch.dtype, batch: int, spatial: int, heads: int, channels: int,
                       queries: int, levels: int, points: int, flags: int = 0) -> int:
        """Bytes of workspace ``backward_workspace`` takes for these sizes (host only)."""
        out = _L()
        self.check(self.cdll.msda_backward_workspace_size(
            DTYPE_CODES[dtype], batch, spatial, heads, channels, queries, levels, points, flags, ctypes.byref(out)))
        return int(out.value)

    def set_path_override(self, paths: int) -> int:
        """Force kernel paths (``PATH_*`` bits, 0 for the library's choice); returns the previous bits."""
        return int(self.cdll.msda_set_path_override(paths))

    def set_phase_events(self, events: list[int] | None) -> None:
        """Record these four raw HIP events between the phases of later backward calls
        on this thread (sort, grad_value, grad_sample); ``None`` stops it."""
        if not events:
            self.check(self.cdll.msda_set_phase_events(None, 0))
            return
        array = (_P * len(events))(*events)
        self.check(self.cdll.msda_set_phase_events(array, len(events)))

    def abi_version(self) -> int:
        return int(self.cdll.msda_abi_version())

    def last_error(self) -> str:
        raw = self.cdll.msda_last_error()
        return raw.decode() if raw else ""

    def check(self, status: int) -> None:
        """Raise ``RuntimeError`` with the library's message for a non-zero status."""
        if status != 0:
            msg = self.last_error() or f"msda call failed with status {status}"
            raise RuntimeError(msg)

    def launch_geometry(
        self, dtype: torch.dtype, batch: int, spatial: int, heads: int, channels: int,
        queries: int, levels: int, points: int, *, backward: bool = False,
    ) -> dict[str, int]:
        """The launch layout of a call with these sizes (host only, no GPU needed)."""
        cv, lh, waves, blocks = _I(), _I(), _I(), _L()
        status = self.cdll.msda_launch_geometry(
            DTYPE_CODES[dtype], batch, spatial, heads, channels, queries, levels, points,
            int(backward), ctypes.byref(cv), ctypes.byref(lh), ctypes.byref(waves), ctypes.byref(blocks),
        )
        self.check(status)
        return {
            "channels_per_lane": cv.value,
            "lanes_per_unit": lh.value,
            "waves_per_block": waves.value,
            "num_blocks": blocks.value,
        }


_lock = threading.Lock()
_loaded: Library | None = None


def load(*, download: bool | None = None, compile: bool | str | None = None) -> Library:  # noqa: A002, ARG001
    """Load the library once. With ``compile`` truthy a missing library is built first.

    Raises
    ------
    KernelNotProvidedError
        If the library is missing and compiling was not allowed.
    KernelBuildError
        If compiling was allowed and hipcc failed.
    KernelUnavailableError
        If the library loads but speaks another ABI version.
    """
    global _loaded  # noqa: PLW0603
    if _loaded is not None:
        return _loaded
    with _lock:
        if _loaded is not None:
            return _loaded
        path = library_path()
        if not path.exists():
            allow = compile if compile is not None else os.environ.get("DEFORMOPS_COMPILE", "0")
            if str(allow).strip().lower() in {"1", "true", "yes", "on", "always"}:
                from ... import _build  # noqa: PLC0415

                try:
                    path = _build.build()
                except Exception as error:
                    msg = f"building {path.name} with hipcc failed: {error}"
                    raise KernelBuildError(msg) from error
            else:
                msg = (
                    f"the HIP kernel library {path} is not built; run "
                    f"`python -m deformops_amd._build` (or set DEFORMOPS_COMPILE=1)"
                )
                raise KernelNotProvidedError(msg)
        library = Library(path)
        if library.abi_version() != ABI_VERSION:
            msg = f"{path} has ABI version {library.abi_version()}, this binding needs {ABI_VERSION}"
            raise KernelUnavailableError(msg)
        _loaded = library
        return library


@contextlib.contextmanager
def path_override(paths: int) -> Iterator[None]:
    """Run the enclosed calls on the kernel paths ``paths`` forces (tests of every path)."""
    library = load()
    previous = library.set_path_override(paths)
    try:
        yield
    finally:
        library.set_path_override(previous)
