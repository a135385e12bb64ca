"""Kernel registry: many implementations per op, one picked per call.

The interface matches dexter's registry (``python/dexter/registry.py:34-152``)
so an implementation package written against one registers into the other:

* ``Priority`` bands REFERENCE=0 < PORTABLE=4 < PERFORMANT=8 < SPECIALISED=12;
  higher wins, and equal priorities keep registration order.
* The capability gate comes first: a spec whose gate the platform fails is
  never a candidate, whatever its priority.
* ``DEXTER_KERNEL=<family/mode>:<name>[,...]`` pins one implementation; a pin
  naming an implementation this platform cannot run raises ``LookupError``.
* Otherwise the best candidate whose optional ``accepts(*args, **kwargs)``
  predicate holds is returned; if none, ``LookupError``.
* ``register`` rejects a second spec of the same name for one ``family/mode``
  with ``ValueError``.

Internally every decision is one pass, :func:`_rulings`, that classifies each
registered spec for a call (gated, declined, eligible); :func:`select_spec`
takes the first eligible one and :func:`explain` prints the whole pass. This
package registers no torch fallback: on a platform without a HIP kernel for the
call, selection raises instead of quietly running something else.
"""

from __future__ import annotations

import bisect
import functools
import itertools
import os
from dataclasses import dataclass, field
from enum import IntEnum
from typing import Callable, Iterator

from .platform import Capability, PlatformInfo, current_platform

__all__ = ["Priority", "KernelSpec", "register", "select", "select_spec", "candidates",
           "explain", "registered", "unregister"]

PIN_ENV = "DEXTER_KERNEL"


class Priority(IntEnum):
    """How specialised an implementation is; higher is preferred."""

    REFERENCE = 0
    PORTABLE = 4
    PERFORMANT = 8
    SPECIALISED = 12


@dataclass(frozen=True)
class KernelSpec:
    """One implementation of an op, with its gate and shape predicate."""

    name: str
    family: str
    mode: str
    impl: Callable
    capability: Capability = field(default_factory=Capability)
    priority: Priority | int = Priority.PERFORMANT
    accepts: Callable[..., bool] | None = None

    @property
    def key(self) -> str:
        return op_key(self.family, self.mode)


def op_key(family: str, mode: str) -> str:
    return f"{family}/{mode}"


class _Catalogue:
    """Specs per op key in selection order: priority descending, then age.

    Each entry carries a sort key ``(-priority, serial)``, so inserting with
    ``bisect`` keeps the order without re-sorting, and a spec registered later
    at the same priority lands behind the earlier ones.
    """

    def __init__(self) -> None:
        self._entries: dict[str, list[tuple[tuple[int, int], KernelSpec]]] = {}
        self._serial = itertools.count()

    def add(self, spec: KernelSpec) -> None:
        entries = self._entries.setdefault(spec.key, [])
        if any(s.name == spec.name for _, s in entries):
            raise ValueError(f"duplicate kernel {spec.key}:{spec.name}")
        order = (-int(spec.priority), next(self._serial))
        bisect.insort(entries, (order, spec), key=lambda e: e[0])

    def remove(self, key: str, name: str) -> None:
        entries = self._entries.get(key, [])
        entries[:] = [e for e in entries if e[1].name != name]

    def specs(self, key: str) -> tuple[KernelSpec, ...]:
        return tuple(s for _, s in self._entries.get(key, ()))


_CATALOGUE = _Catalogue()


def register(
    family: str,
    mode: str,
    *,
    name: str,
    capability: Capability | None = None,
    priority: Priority | int = Priority.PERFORMANT,
    accepts: Callable[..., bool] | None = None,
) -> Callable[[Callable], Callable]:
    """Decorator: add the decorated function as an implementation of ``family/mode``.

    The function comes back unchanged apart from a ``dexter_spec`` attribute
    holding its :class:`KernelSpec`.
    """
    gate = capability if capability is not None else Capability()

    def add(fn: Callable) -> Callable:
        spec = KernelSpec(name, family, mode, fn, gate, priority, accepts)
        _CATALOGUE.add(spec)
        fn.dexter_spec = spec  # type: ignore[attr-defined]
        return fn

    return add


def unregister(family: str, mode: str, name: str) -> None:
    """Remove one spec (tests register throwaway specs and clean up)."""
    _CATALOGUE.remove(op_key(family, mode), name)


def registered(family: str, mode: str) -> tuple[KernelSpec, ...]:
    """Every spec of ``family/mode`` in selection order, runnable here or not."""
    return _CATALOGUE.specs(op_key(family, mode))


def candidates(family: str, mode: str,
               platform: PlatformInfo | None = None) -> Iterator[KernelSpec]:
    """Specs of ``family/mode`` whose gate ``platform`` (default: this one) passes."""
    where = platform if platform is not None else current_platform()
    return (s for s in registered(family, mode) if s.capability.satisfied_by(where))


@functools.lru_cache(maxsize=16)
def _pins(raw: str) -> dict[str, str]:
    """``DEXTER_KERNEL`` as ``{op key: pinned name}``; the first entry for a key wins.

    An entry without ``:`` pins the empty name, which no spec has, so selection
    for that op raises.
    """
    table: dict[str, str] = {}
    for item in raw.split(","):
        key, _, name = item.strip().partition(":")
        if key:
            table.setdefault(key, name)
    return table


def _pin_for(key: str) -> str | None:
    return _pins(os.environ.get(PIN_ENV, "")).get(key)


# Ruling of one spec for one call, in the order selection considers them.
GATED, DECLINED, ELIGIBLE = "gated", "declined", "eligible"


@dataclass(frozen=True)
class Ruling:
    spec: KernelSpec
    status: str          # GATED, DECLINED or ELIGIBLE
    detail: str = ""     # why a spec was gated


def _gate_detail(spec: KernelSpec, platform: PlatformInfo) -> str:
    missing = sorted(spec.capability.features - platform.features)
    if missing:
        return f"platform lacks {missing}"
    return f"vendor/arch outside the gate ({platform.vendor} {platform.arch})"


def _rulings(key: str, platform: PlatformInfo, args: tuple, kwargs: dict) -> list[Ruling]:
    """Classify every spec of ``key`` for this call (predicates only for runnable specs)."""
    out = []
    for spec in _CATALOGUE.specs(key):
        if not spec.capability.satisfied_by(platform):
            out.append(Ruling(spec, GATED, _gate_detail(spec, platform)))
        elif spec.accepts is not None and not spec.accepts(*args, **kwargs):
            out.append(Ruling(spec, DECLINED))
        else:
            out.append(Ruling(spec, ELIGIBLE))
    return out


def select_spec(family: str, mode: str, *args, **kwargs) -> KernelSpec:
    """Like :func:`select` but returns the whole spec (name, priority, ...)."""
    key = op_key(family, mode)
    platform = current_platform()
    pin = _pin_for(key)
    if pin is not None:
        # A pin overrides the predicates, not the gate.
        for spec in candidates(family, mode, platform):
            if spec.name == pin:
                return spec
        raise LookupError(f"{PIN_ENV} pinned {key}:{pin}, which is not available here")
    for ruling in _rulings(key, platform, args, kwargs):
        if ruling.status == ELIGIBLE:
            return ruling.spec
    names = [s.name for s in _CATALOGUE.specs(key)]
    raise LookupError(f"no kernel for {key} on {platform.describe()}. "
                      f"Registered: {names or 'none'}")


def select(family: str, mode: str, *args, **kwargs) -> Callable:
    """Best implementation of ``family/mode`` for this platform and call.

    ``args``/``kwargs`` go only to ``accepts`` predicates, never to the impl.
    """
    return select_spec(family, mode, *args, **kwargs).impl


def explain(family: str, mode: str, *args, **kwargs) -> str:
    """The selection pass for one call as text: a header, then one row per spec.

    Rows are in selection order; the chosen spec is marked ``chosen``, other
    runnable ones ``eligible``, and the rest say why they were passed over.
    """
    key = op_key(family, mode)
    platform = current_platform()
    pin = _pin_for(key)
    rows = _rulings(key, platform, args, kwargs)
    try:
        chosen = select_spec(family, mode, *args, **kwargs).name
    except LookupError as err:
        chosen, failure = None, str(err)
    width = max((len(r.spec.name) for r in rows), default=0)
    text = [f"{key} on {platform.describe()}" + (f" [pin: {pin}]" if pin is not None else "")]
    for r in rows:
        tag = "chosen" if r.spec.name == chosen and r.status != GATED else r.status
        why = {GATED: f": {r.detail}", DECLINED: ": accepts() declined these arguments"}
        text.append(f"  {tag:<8} {r.spec.name:<{width}}  priority {int(r.spec.priority):>2}"
                    f"{why.get(r.status, '')}")
    if chosen is None:
        text.append(f"  no selection: {failure}")
    return "\n".join(text)
