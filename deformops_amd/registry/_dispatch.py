"""The backend table of one operator.

Interface of the reference's registry (sources/deformops/registry/_dispatch.py:
35-454): the ``Backend`` enum, ``Resolution`` and ``LoadedBackend`` records, and a
``Registry`` whose ``register``, ``load``, ``resolve``, ``run_selected`` and
``__call__`` behave as there. An explicit ``backend=`` runs that backend or raises
``NoBackendError``; ``backend=None`` runs the first candidate of the operator's
policy that is registered, supports the call and loads its kernels; a raw string
for ``backend`` is a ``TypeError``.

This build ships two backends: the HIP kernels for GPU tensors and, for CPU
tensors only, torch operators (``EAGER``). So the table is small and the choice
needs little: a policy names one candidate, and checking it is a dictionary
lookup, a predicate on the call's context and an already-loaded library.
``Backend.CUDA`` is an alias of ``Backend.HIP``, so code written for the
reference's CUDA backend runs the HIP kernels; ``TRITON`` exists so that such code
imports, and asking for it says why it is absent.
"""

from __future__ import annotations

import dataclasses
import importlib
import inspect
import os
import threading
import warnings
from collections.abc import Callable, Iterable, Mapping
from enum import Enum
from typing import Any

from ..core.errors import BackendFallbackWarning, KernelNotProvidedError, NoBackendError

__all__ = ["Backend", "LoadedBackend", "Registry", "Resolution"]

#: Set to a falsy value to silence :class:`BackendFallbackWarning`.
FALLBACK_WARNINGS_ENV_VAR = "DEFORMOPS_FALLBACK_WARNINGS"


class Backend(str, Enum):
    """Compute backends. ``CUDA`` is an alias of ``HIP`` (torch's device type on ROCm is
    ``"cuda"``, and ``Backend("cuda")`` is ``HIP``); ``EAGER`` takes CPU tensors only,
    and ``TRITON`` is never registered in this build."""

    HIP = "hip"
    CUDA = "hip"
    TRITON = "triton"
    EAGER = "eager"

    @classmethod
    def _missing_(cls, value: object) -> Backend | None:
        return cls.HIP if value == "cuda" else None

    def __str__(self) -> str:
        return self.value


@dataclasses.dataclass(frozen=True)
class Resolution:
    """The backend a call runs on, the options the policy gives it, and the
    ``(backend, reason)`` of every candidate it preferred that could not run."""

    backend: Backend
    options: dict[str, Any]
    rejected: tuple[tuple[Backend, str], ...] = ()


@dataclasses.dataclass(frozen=True)
class LoadedBackend:
    """What :meth:`Registry.load` made ready: the operator, the backend and the path of
    its kernel library (``None`` for a backend without one)."""

    operator: str
    backend: Backend
    library: str | None


@dataclasses.dataclass
class _Entry:
    run: Callable[..., Any]
    supports: Callable[[Any], bool] | None = None
    load: Callable[..., Any] | None = None


#: Packages that hold each backend's adapter module (``<package>.<operator>``).
_ADAPTERS: dict[Backend, str] = {
    Backend.HIP: "deformops_amd.backends.hip",
    Backend.EAGER: "deformops_amd.backends.eager",
}

_NOT_BUILT = (
    "it is not part of this build, which runs MSDA on AMD GPUs through its HIP kernels "
    "(Backend.HIP) and on CPU tensors in torch operators (Backend.EAGER)"
)


def _candidates(picked: Any) -> Iterable[tuple[Backend, dict[str, Any]]]:
    """A policy's answer as ``(backend, options)`` pairs: it may name one backend, one
    ``(backend, options)`` pair, or a sequence of either."""
    if isinstance(picked, Backend) or (isinstance(picked, tuple) and picked and isinstance(picked[0], Backend)
                                       and len(picked) == 2 and isinstance(picked[1], Mapping)):
        picked = [picked]
    for item in picked:
        if isinstance(item, Backend):
            yield item, {}
        else:
            yield item[0], dict(item[1])


def _require_backend(backend: object, *, allow_none: bool) -> None:
    if backend is None and allow_none:
        return
    if not isinstance(backend, Backend):
        raise TypeError(
            f"backend must be a Backend member{' or None' if allow_none else ''}, not "
            f"{type(backend).__name__} (raw strings are not accepted)"
        )


class Registry:
    """The backends of one operator and the policy that picks one for ``backend=None``.

    Parameters
    ----------
    name
        The operator's name, also the adapter module name under each backend package.
    context_of
        Builds the selection context from a call's arguments, validating them.
    select
        The policy: context to candidate backends, best first.
    describe
        A function whose docstring and signature document the operator.
    """

    def __init__(
        self,
        name: str,
        *,
        context_of: Callable[..., Any],
        select: Callable[[Any], Any],
        describe: Callable[..., Any] | None = None,
    ) -> None:
        self.name = name
        self._context_of = context_of
        self._select = select
        self._entries: dict[Backend, _Entry] = {}
        self._absent: dict[Backend, str] = {}
        self._route: Callable[..., Any] | None = None
        self._adapters_ready = False
        self._lock = threading.Lock()
        # Choices that passed over no backend, per context: a repeated call skips the
        # policy and the support predicates. Emptied whenever the table changes.
        self._chosen: dict[Any, Resolution] = {}
        if describe is not None:
            self.__doc__ = describe.__doc__
            self.__signature__ = inspect.signature(describe)

    # The table.

    def register(
        self,
        backend: Backend,
        op_handle: Callable[..., Any],
        *,
        supports: Callable[[Any], bool] | None = None,
        load: Callable[..., Any] | None = None,
    ) -> None:
        """File ``op_handle`` as ``backend``'s implementation, with an optional
        ``supports(context)`` predicate and ``load(download=, compile=)`` hook."""
        _require_backend(backend, allow_none=False)
        self._entries[backend] = _Entry(op_handle, supports, load)
        self._absent.pop(backend, None)
        self._chosen.clear()

    def mark_unavailable(self, backend: Backend, reason: str) -> None:
        """Record why ``backend`` is not registered; error messages quote it."""
        if backend not in self._entries:
            self._absent[backend] = reason
            self._chosen.clear()

    def route_selected_calls(self, route: Callable[..., Any]) -> None:
        """Send ``backend=None`` calls through ``route`` (the public operator)."""
        self._route = route

    def _import_adapters(self) -> None:
        if self._adapters_ready:
            return
        with self._lock:
            if self._adapters_ready:
                return
            for backend in (Backend.HIP, Backend.TRITON, Backend.EAGER):
                package = _ADAPTERS.get(backend)
                if package is None:
                    self.mark_unavailable(backend, _NOT_BUILT)
                    continue
                try:
                    importlib.import_module(f"{package}.{self.name}")
                except Exception as error:  # noqa: BLE001 - reported, and the backend marked absent
                    reason = f"its adapter failed to import ({type(error).__name__}: {error})"
                    self.mark_unavailable(backend, reason)
                    warnings.warn(f"{self.name}: the {backend.value!r} backend is unavailable: {reason}",
                                  RuntimeWarning, stacklevel=3)
            self._adapters_ready = True

    # Queries.

    def is_registered(self, backend: Backend) -> bool:
        self._import_adapters()
        return backend in self._entries

    def get(self, backend: Backend) -> Callable[..., Any] | None:
        self._import_adapters()
        entry = self._entries.get(backend)
        return None if entry is None else entry.run

    def available(self) -> list[str]:
        self._import_adapters()
        return sorted({backend.value for backend in self._entries})

    def unavailable_reason(self, backend: Backend) -> str:
        return self._absent.get(backend, "it is not registered on this host")

    def load(self, backend: Backend, *, download: bool | None = None,
             compile: bool | str | None = None) -> LoadedBackend:  # noqa: A002
        """Make ``backend`` ready before its first call; report its library."""
        _require_backend(backend, allow_none=False)
        self._import_adapters()
        entry = self._entries.get(backend)
        if entry is None:
            raise NoBackendError(f"{self.name}: the {backend.value!r} backend is unavailable: "
                                 f"{self.unavailable_reason(backend)}.")
        library = None if entry.load is None else str(entry.load(download=download, compile=compile))
        return LoadedBackend(self.name, backend, library)

    # Choosing.

    def _refusal(self, backend: Backend, context: Any) -> str | None:
        """Why ``backend`` cannot run a call with ``context``, or ``None`` when it can
        (its kernels then are loaded)."""
        entry = self._entries.get(backend)
        if entry is None:
            return self.unavailable_reason(backend)
        if entry.supports is not None and not entry.supports(context):
            return "it does not support this call"
        if entry.load is not None:
            try:
                entry.load()
            except KernelNotProvidedError as error:
                return str(error)
        return None

    def _choose(self, context: Any) -> Resolution:
        known = self._chosen.get(context)
        if known is not None:
            return known
        rejected: list[tuple[Backend, str]] = []
        for backend, options in _candidates(self._select(context)):
            reason = self._refusal(backend, context)
            if reason is not None:
                rejected.append((backend, reason))
                continue
            if rejected and os.getenv(FALLBACK_WARNINGS_ENV_VAR, "1").strip().lower() not in {"0", "false", "no", "off"}:
                passed = "; ".join(f"{b.value!r}: {why}" for b, why in rejected)
                warnings.warn(f"{self.name} runs on {backend.value!r}, passing over {passed}. Set "
                              f"{FALLBACK_WARNINGS_ENV_VAR}=0 to silence this.", BackendFallbackWarning,
                              stacklevel=4)
            resolution = Resolution(backend, options, tuple(rejected))
            if not rejected:
                self._chosen[context] = resolution
            return resolution
        tried = "; ".join(f"{b.value!r}: {why}" for b, why in rejected) or "none"
        raise NoBackendError(f"No backend can run this {self.name} call ({context!r}). Candidates: {tried}.")

    def _explicit(self, backend: Backend, context: Any) -> _Entry:
        entry = self._entries.get(backend)
        if entry is None:
            raise NoBackendError(
                f"{self.name}: the {backend.value!r} backend is unavailable: {self.unavailable_reason(backend)}. "
                f"Registered: {self.available()}."
            )
        if entry.supports is not None and not entry.supports(context):
            raise NoBackendError(f"{self.name}: the {backend.value!r} backend does not support this call: "
                                 f"{context!r}")
        return entry

    def resolve(self, *args: Any, backend: Backend | None = None, **kwargs: Any) -> Resolution:
        """The backend a call with these arguments would run on, without running it."""
        _require_backend(backend, allow_none=True)
        self._import_adapters()
        context = self._context_of(*args, **kwargs)
        if backend is None:
            return self._choose(context)
        entry = self._explicit(backend, context)
        if entry.load is not None:
            entry.load()
        return Resolution(backend, {})

    def run_selected(self, *args: Any, **kwargs: Any) -> Any:
        """Run a call on the policy's choice, never through the route."""
        self._import_adapters()
        choice = self._choose(self._context_of(*args, **kwargs))
        return self._entries[choice.backend].run(*args, **{**choice.options, **kwargs})

    def __call__(self, *args: Any, backend: Backend | None = None, **kwargs: Any) -> Any:
        """Run the operator on ``backend``, or on the policy's choice for ``None``."""
        _require_backend(backend, allow_none=True)
        if backend is None:
            if self._route is not None:
                return self._route(*args, **kwargs)
            return self.run_selected(*args, **kwargs)
        self._import_adapters()
        return self._explicit(backend, self._context_of(*args, **kwargs)).run(*args, **kwargs)

    apply = __call__
