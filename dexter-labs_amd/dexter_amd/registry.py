"""Kernel registry: many implementations per op, one picked per call.

Same contract as dexter's registry (``python/dexter/registry.py:34-173``), so
an implementation package written against one registers into the other:

* ``Priority`` bands REFERENCE=0 < PORTABLE=4 < PERFORMANT=8 < SPECIALISED=12;
  higher wins.
* The capability gate is checked first; a spec whose gate fails is invisible.
* ``DEXTER_KERNEL=<family/mode>:<name>[,...]`` pins one implementation; a pin
  naming an implementation this platform cannot run raises ``LookupError``.
* Otherwise the first viable spec whose optional ``accepts(*args, **kwargs)``
  predicate holds is returned; if none, ``LookupError``.
* ``register`` rejects a duplicate name within one ``family/mode`` with
  ``ValueError``.

This package registers no torch fallback: on a platform without a HIP kernel
for the call, selection raises instead of quietly running something else.
"""

from __future__ import annotations

import os
from collections import defaultdict
from dataclasses import dataclass, field
from enum import IntEnum
from typing import Callable, Iterator

from .platform import Capability, PlatformInfo, current_platform

__all__ = ["Priority", "KernelSpec", "register", "select", "select_spec",
           "candidates", "explain", "unregister"]


class Priority(IntEnum):
    """How specialised an implementation is; higher is preferred."""

    REFERENCE = 0
    PORTABLE = 4
    PERFORMANT = 8
    SPECIALISED = 12


@dataclass(frozen=True)
class KernelSpec:
    name: str
    family: str
    mode: str
    impl: Callable
    capability: Capability = field(default_factory=Capability)
    priority: Priority | int = Priority.PERFORMANT
    accepts: Callable[..., bool] | None = None

    @property
    def key(self) -> str:
        return f"{self.family}/{self.mode}"

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return f"<KernelSpec {self.key}:{self.name} pri={int(self.priority)}>"


# family/mode -> specs, kept sorted best-first so selection is a scan.
_REGISTRY: dict[str, list[KernelSpec]] = defaultdict(list)


def register(
    family: str,
    mode: str,
    *,
    name: str,
    capability: Capability | None = None,
    priority: Priority | int = Priority.PERFORMANT,
    accepts: Callable[..., bool] | None = None,
) -> Callable[[Callable], Callable]:
    """Decorator: add ``fn`` as an implementation of ``family/mode``."""

    def wrap(fn: Callable) -> Callable:
        spec = KernelSpec(name=name, family=family, mode=mode, impl=fn,
                          capability=capability or Capability(),
                          priority=priority, accepts=accepts)
        bucket = _REGISTRY[spec.key]
        if any(s.name == name for s in bucket):
            raise ValueError(f"duplicate kernel {spec.key}:{name}")
        bucket.append(spec)
        bucket.sort(key=lambda s: int(s.priority), reverse=True)  # stable
        fn.dexter_spec = spec  # type: ignore[attr-defined]
        return fn

    return wrap


def unregister(family: str, mode: str, name: str) -> None:
    """Remove one spec (tests register throwaway specs and clean up)."""
    bucket = _REGISTRY[f"{family}/{mode}"]
    bucket[:] = [s for s in bucket if s.name != name]


def candidates(family: str, mode: str,
               platform: PlatformInfo | None = None) -> Iterator[KernelSpec]:
    """Specs for ``family/mode`` whose gate this platform passes, best first."""
    platform = platform or current_platform()
    for spec in _REGISTRY[f"{family}/{mode}"]:
        if spec.capability.satisfied_by(platform):
            yield spec


def _pinned(key: str) -> str | None:
    for entry in os.environ.get("DEXTER_KERNEL", "").split(","):
        entry = entry.strip()
        if not entry:
            continue
        pin_key, _, pin_name = entry.partition(":")
        if pin_key == key:
            return pin_name
    return None


def select_spec(family: str, mode: str, *args, **kwargs) -> KernelSpec:
    """Like :func:`select` but returns the whole spec (name, priority, ...)."""
    key = f"{family}/{mode}"
    pin = _pinned(key)
    viable = list(candidates(family, mode))
    if pin is not None:
        for spec in viable:
            if spec.name == pin:
                return spec
        raise LookupError(f"DEXTER_KERNEL pinned {key}:{pin}, which is not available here")
    for spec in viable:
        if spec.accepts is None or spec.accepts(*args, **kwargs):
            return spec
    raise LookupError(
        f"no kernel for {key} on {current_platform().describe()}. "
        f"Registered: {[s.name for s in _REGISTRY[key]] or 'none'}"
    )


def select(family: str, mode: str, *args, **kwargs) -> Callable:
    """Best implementation of ``family/mode`` for this platform and call.

    ``args``/``kwargs`` go only to ``accepts`` predicates, never to the impl.
    """
    return select_spec(family, mode, *args, **kwargs).impl


def explain(family: str, mode: str, *args, **kwargs) -> str:
    """Why each registered spec was or was not picked, one line per spec."""
    key = f"{family}/{mode}"
    platform = current_platform()
    lines = [f"{key} on {platform.describe()}"]
    chosen = None
    for spec in _REGISTRY[key]:
        if not spec.capability.satisfied_by(platform):
            missing = sorted(spec.capability.features - platform.features)
            reason = f"needs {missing}" if missing else "arch gate"
            lines.append(f"  - {spec.name:<28} skipped ({reason})")
        elif spec.accepts is not None and not spec.accepts(*args, **kwargs):
            lines.append(f"  - {spec.name:<28} skipped (shape not accepted)")
        elif chosen is None:
            chosen = spec
            lines.append(f"  * {spec.name:<28} SELECTED (pri={int(spec.priority)})")
        else:
            lines.append(f"  - {spec.name:<28} viable (pri={int(spec.priority)})")
    return "\n".join(lines)
