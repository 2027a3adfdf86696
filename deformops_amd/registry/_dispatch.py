"""Backend registry: one per operator, mapping :class:`Backend` members to callables.

Behaviour follows the reference's ``Registry`` (sources/deformops/registry/_dispatch.py:
122-454): an explicit ``backend=`` runs that backend or raises
:class:`NoBackendError`; ``backend=None`` runs the first candidate of the
operator's selection policy that is registered, supports the call and can load
its kernel, memoized per call context; raw strings are rejected with
``TypeError``.

This build registers a single backend, ``Backend.HIP`` (``Backend.CUDA`` is an
alias of it, so code written for the reference's CUDA backend runs the HIP
kernels). ``TRITON`` and ``EAGER`` exist so such code still imports; asking for
them raises ``NoBackendError`` with the reason.
"""

from __future__ import annotations

import dataclasses
import importlib
import inspect
import logging
import os
import threading
import warnings
from collections.abc import Callable, Mapping, Sequence
from enum import Enum
from typing import Any

from ..core.errors import BackendFallbackWarning, KernelNotProvidedError, NoBackendError

__all__ = ["Backend", "LoadedBackend", "Registry", "Resolution"]

logger = logging.getLogger(__name__)

#: Set to a falsy value to silence :class:`BackendFallbackWarning`.
FALLBACK_WARNINGS_ENV_VAR = "DEFORMOPS_FALLBACK_WARNINGS"

_FALSY = frozenset({"0", "false", "no", "off"})


class Backend(str, Enum):
    """Compute backends. ``CUDA`` is an alias of ``HIP`` (torch's ROCm device type is
    ``"cuda"``); ``TRITON`` and ``EAGER`` are never registered in this build."""

    HIP = "hip"
    CUDA = "hip"
    TRITON = "triton"
    EAGER = "eager"

    @classmethod
    def _missing_(cls, value: object) -> Backend | None:
        if value == "cuda":
            return cls.HIP
        return None

    def __str__(self) -> str:
        return self.value


#: Where the adapter of each registered backend lives.
_ADAPTER_MODULES: dict[Backend, str] = {Backend.HIP: "deformops_amd.backends.hip"}

#: Why the other backends are absent.
_ABSENT_REASON = (
    "it is not part of this build, which runs MSDA only on AMD GPUs through its "
    "HIP kernels (Backend.HIP)"
)

Candidate = Backend | tuple[Backend, Mapping[str, Any]]


@dataclasses.dataclass(frozen=True)
class Resolution:
    """The backend a call runs on, its options, and the candidates passed over."""

    backend: Backend
    options: dict[str, Any]
    rejected: tuple[tuple[Backend, str], ...] = ()


@dataclasses.dataclass(frozen=True)
class LoadedBackend:
    """What :meth:`Registry.load` made ready: operator, backend and library path."""

    operator: str
    backend: Backend
    library: str | None


def _normalize(selected: Candidate | Sequence[Candidate]) -> list[tuple[Backend, dict[str, Any]]]:
    items: Sequence[Candidate]
    if isinstance(selected, Backend):
        items = [selected]
    elif isinstance(selected, tuple) and len(selected) == 2 and isinstance(selected[0], Backend):  # noqa: PLR2004
        items = [selected]  # type: ignore[list-item]
    else:
        items = selected  # type: ignore[assignment]
    out: list[tuple[Backend, dict[str, Any]]] = []
    for item in items:
        if isinstance(item, Backend):
            out.append((item, {}))
        else:
            out.append((item[0], dict(item[1])))
    return out


class Registry:
    """Backends of one operator, with a selection policy for ``backend=None``."""

    def __init__(
        self,
        name: str,
        *,
        context_of: Callable[..., Any],
        select: Callable[[Any], Candidate | Sequence[Candidate]],
        describe: Callable[..., Any] | None = None,
    ) -> None:
        self.name = name
        if describe is not None:
            self.__doc__ = describe.__doc__
            self.__signature__ = inspect.signature(describe)
        self._handlers: dict[Backend, Callable[..., Any]] = {}
        self._supports: dict[Backend, Callable[[Any], bool]] = {}
        self._loaders: dict[Backend, Callable[..., Any]] = {}
        self._absent: dict[Backend, str] = {}
        self._context_of = context_of
        self._select = select
        self._memo: dict[Any, Resolution] = {}
        self._imported = False
        self._lock = threading.RLock()
        self._route: Callable[..., Any] | None = None

    # Registration.

    def register(
        self,
        backend: Backend,
        op_handle: Callable[..., Any],
        *,
        supports: Callable[[Any], bool] | None = None,
        load: Callable[..., Any] | None = None,
    ) -> None:
        """File ``op_handle`` under ``backend``; ``supports`` and ``load`` are optional."""
        if not isinstance(backend, Backend):
            msg = (
                f"backend must be a Backend member, got {type(backend).__name__!r}. "
                f"Raw strings are not permitted."
            )
            raise TypeError(msg)
        self._handlers[backend] = op_handle
        self._absent.pop(backend, None)
        if supports is not None:
            self._supports[backend] = supports
        if load is not None:
            self._loaders[backend] = load
        self._memo.clear()

    def mark_unavailable(self, backend: Backend, reason: str) -> None:
        """Record why ``backend`` is not registered, for error messages."""
        if backend not in self._handlers:
            self._absent[backend] = reason

    def route_selected_calls(self, route: Callable[..., Any]) -> None:
        """Send every ``backend=None`` call through ``route`` (a public operator)."""
        self._route = route

    def _import_adapters(self) -> None:
        if self._imported:
            return
        with self._lock:
            if self._imported:
                return
            for backend in Backend:
                module = _ADAPTER_MODULES.get(backend)
                if module is None:
                    self.mark_unavailable(backend, _ABSENT_REASON)
                    continue
                try:
                    importlib.import_module(f"{module}.{self.name}")
                except Exception as error:  # noqa: BLE001
                    logger.debug("Failed to import %s.%s", module, self.name, exc_info=True)
                    reason = f"its adapter failed to import ({type(error).__name__}: {error})"
                    self.mark_unavailable(backend, reason)
                    warnings.warn(
                        f"The {backend.value!r} backend for {self.name!r} is unavailable: {reason}",
                        RuntimeWarning,
                        stacklevel=3,
                    )
            self._imported = True

    # Queries.

    def is_registered(self, backend: Backend) -> bool:
        self._import_adapters()
        return backend in self._handlers

    def get(self, backend: Backend) -> Callable[..., Any] | None:
        self._import_adapters()
        return self._handlers.get(backend)

    def available(self) -> list[str]:
        self._import_adapters()
        return sorted({b.value for b in self._handlers})

    def unavailable_reason(self, backend: Backend) -> str:
        return self._absent.get(backend, "it is not registered on this host")

    def load(
        self,
        backend: Backend,
        *,
        download: bool | None = None,
        compile: bool | str | None = None,  # noqa: A002
    ) -> LoadedBackend:
        """Make ``backend`` ready before the first call and report its library."""
        if not isinstance(backend, Backend):
            msg = f"backend must be a Backend member, got {type(backend).__name__!r}"
            raise TypeError(msg)
        if not self.is_registered(backend):
            msg = (
                f"The {backend.value!r} backend for {self.name} is unavailable: "
                f"{self.unavailable_reason(backend)}."
            )
            raise NoBackendError(msg)
        loader = self._loaders.get(backend)
        library = None
        if loader is not None:
            library = str(loader(download=download, compile=compile))
        return LoadedBackend(self.name, backend, library)

    # Selection.

    def _supports_call(self, backend: Backend, context: Any) -> bool:
        predicate = self._supports.get(backend)
        return predicate is None or bool(predicate(context))

    def _negotiate(self, context: Any) -> Resolution:
        rejected: list[tuple[Backend, str]] = []
        for backend, options in _normalize(self._select(context)):
            if backend not in self._handlers:
                rejected.append((backend, self.unavailable_reason(backend)))
                continue
            if not self._supports_call(backend, context):
                rejected.append((backend, "it does not support this call"))
                continue
            loader = self._loaders.get(backend)
            if loader is not None:
                try:
                    loader()
                except KernelNotProvidedError as error:
                    rejected.append((backend, str(error)))
                    continue
            if rejected and os.getenv(FALLBACK_WARNINGS_ENV_VAR, "").strip().lower() not in _FALSY:
                warnings.warn(
                    f"{self.name}: running the {backend.value!r} backend because "
                    + "; ".join(f"{b.value!r} was passed over: {r}" for b, r in rejected)
                    + f". Set {FALLBACK_WARNINGS_ENV_VAR}=0 to silence this warning.",
                    BackendFallbackWarning,
                    stacklevel=4,
                )
            return Resolution(backend, options, tuple(rejected))
        details = "; ".join(f"{b.value!r}: {r}" for b, r in rejected)
        msg = (
            f"No backend can run this {self.name} call ({context!r}). "
            f"Candidates in order of preference: {details or 'none'}."
        )
        raise NoBackendError(msg)

    def _resolved(self, context: Any) -> Resolution:
        hit = self._memo.get(context)
        if hit is None:
            hit = self._negotiate(context)
            self._memo[context] = hit
        return hit

    @staticmethod
    def _check_backend_argument(backend: object) -> None:
        if backend is not None and not isinstance(backend, Backend):
            msg = (
                f"backend argument must be a Backend member or None, got "
                f"{type(backend).__name__!r}. Raw strings are not permitted."
            )
            raise TypeError(msg)

    def _explicit(self, backend: Backend, context: Any) -> Callable[..., Any]:
        handler = self._handlers.get(backend)
        if handler is None:
            msg = (
                f"The {backend.value!r} backend for {self.name} is unavailable: "
                f"{self.unavailable_reason(backend)}. Registered backends: {self.available()}."
            )
            raise NoBackendError(msg)
        if not self._supports_call(backend, context):
            msg = f"The {backend.value!r} backend does not support this {self.name} call: {context!r}"
            raise NoBackendError(msg)
        return handler

    def resolve(self, *args: Any, backend: Backend | None = None, **kwargs: Any) -> Resolution:
        """Report which backend a call with these arguments would run on."""
        self._check_backend_argument(backend)
        self._import_adapters()
        context = self._context_of(*args, **kwargs)
        if backend is not None:
            self._explicit(backend, context)
            loader = self._loaders.get(backend)
            if loader is not None:
                loader()
            return Resolution(backend, {})
        return self._resolved(context)

    def run_selected(self, *args: Any, **kwargs: Any) -> Any:
        """Run a call on the policy's backend, bypassing any route."""
        self._import_adapters()
        context = self._context_of(*args, **kwargs)
        resolution = self._resolved(context)
        return self._handlers[resolution.backend](*args, **{**resolution.options, **kwargs})

    def __call__(self, *args: Any, backend: Backend | None = None, **kwargs: Any) -> Any:
        """Run the operator on the requested backend, or the selected one."""
        self._check_backend_argument(backend)
        if backend is not None:
            self._import_adapters()
            context = self._context_of(*args, **kwargs)
            return self._explicit(backend, context)(*args, **kwargs)
        if self._route is not None:
            return self._route(*args, **kwargs)
        return self.run_selected(*args, **kwargs)

    apply = __call__
