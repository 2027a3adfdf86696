"""Replacing a model's modules in place (reference ``integrations/_patch.py:17-103``)."""

from __future__ import annotations

from collections.abc import Callable, Sequence
from typing import Any

from torch import nn

__all__ = ["ModuleFactory", "patch_modules", "replace_module_recursively"]

#: Builds the replacement of one matched module from that module.
ModuleFactory = Callable[[Any], nn.Module]


def patch_modules(
    module: nn.Module,
    replacements: Sequence[tuple[type[Any], ModuleFactory]],
    *,
    strict: bool = True,
) -> nn.Module:
    """Swap every descendant that is an instance of a listed class, in one walk.

    A child is matched against ``replacements`` in order; the first class it is
    an instance of wins, and ``factory(child)`` takes its attribute. The
    replacement's own children are walked too, so a listed class nested inside
    another is found. Each module is replaced once: a replacement may keep the
    module it replaces as a child, and a module shared by several parents is
    replaced by one shared replacement. The root itself is never replaced.

    Parameters
    ----------
    module
        The model or subtree; changed in place.
    replacements
        ``(class, factory)`` pairs.
    strict
        Raise when nothing was replaced: usually the installed library renamed
        the class and the model still runs its own implementation.

    Returns
    -------
    ``module``.

    Raises
    ------
    RuntimeError
        If ``strict`` and no module matched.
    """
    # original id -> (original, replacement); the original is held so that no id is
    # reused during the walk.
    replaced: dict[int, tuple[nn.Module, nn.Module]] = {}
    # (module, ids of the originals whose replacements contain it)
    pending: list[tuple[nn.Module, frozenset[int]]] = [(module, frozenset())]
    while pending:
        parent, inside = pending.pop()
        for name, child in list(parent.named_children()):
            key = id(child)
            if key in replaced:
                if key not in inside:  # the same module shared elsewhere: share its replacement
                    setattr(parent, name, replaced[key][1])
                    continue
                pending.append((child, inside))  # kept inside its own replacement
                continue
            factory = next((f for cls, f in replacements if isinstance(child, cls)), None)
            if factory is None:
                pending.append((child, inside))
                continue
            new = factory(child)
            replaced[key] = (child, new)
            setattr(parent, name, new)
            pending.append((new, inside | {key}))
    if strict and not replaced:
        wanted = ", ".join(f"{cls.__module__}.{cls.__qualname__}" for cls, _ in replacements)
        msg = (
            f"nothing in {type(module).__name__} is an instance of {wanted}; the installed "
            f"library may name these modules differently, and the model would keep its own "
            f"implementation. Pass strict=False to allow a model without them."
        )
        raise RuntimeError(msg)
    return module


def replace_module_recursively(
    module: nn.Module,
    old_class: type[Any],
    factory: ModuleFactory,
    *,
    strict: bool = True,
) -> nn.Module:
    """:func:`patch_modules` with one class."""
    return patch_modules(module, [(old_class, factory)], strict=strict)
