"""Device description that kernel gates are checked against.

Mirrors the interface of dexter's ``platform`` module
(``python/dexter/platform.py:38-278``): ``ArchVersion``, ``PlatformInfo``,
``Capability``, ``current_platform`` and ``override_platform`` keep their
names, fields and meaning, so a kernel gate written for one works unchanged
against the other.

What differs is the table of known parts. The reference knows RDNA3/3.5
(wave32, WMMA, 64 KB LDS) and raises on anything else
(``platform.py:201-208``); this module knows CDNA4 (gfx950, MI355X): wave64,
MFMA matrix cores with bf16/f16/fp8/int8 inputs, 160 KB of LDS per CU, HBM3E,
and ``global_load_lds`` (direct global→LDS copies). An unknown AMD part still
raises ``RuntimeError`` (naming the part and the architectures this table
knows), because a kernel picked on a guessed platform is worse than no kernel.
"""

from __future__ import annotations

import functools
import os
from dataclasses import dataclass, field

__all__ = [
    "ArchVersion",
    "AmdArch",
    "PlatformInfo",
    "Capability",
    "current_platform",
    "override_platform",
    "cdna4_platform",
]


@dataclass(frozen=True, order=True)
class ArchVersion:
    """GPU generation as (major, minor); ordered so gates can use ``<``/``>``.

    gfx950 is (9, 5). RDNA3 parts are (11, x), so a gate with
    ``min_arch=(11, 0)`` never admits a CDNA part and vice versa with
    ``max_arch=(9, 5)``.
    """

    major: int
    minor: int

    def __str__(self) -> str:
        return f"{self.major}.{self.minor}"


@dataclass(frozen=True)
class AmdArch:
    """Fixed facts about one AMD ISA."""

    version: ArchVersion
    family: str
    wavefront: int
    lds_bytes: int
    cus_per_group: int  # CUs behind one torch "multiprocessor"
    features: frozenset[str]
    peak_bandwidth: float  # GB/s, datasheet
    peak_bf16_tflops: float  # dense, datasheet


# Feature strings follow dexter's vocabulary (``platform.py:61-65``):
#   matrix:<dtype>  the matrix unit takes this input type natively
#   mma:<family>    which matrix instruction family exists (mfma here)
#   memory:<kind>   data movement a kernel may assume
# plus "memory:hbm" for discrete HBM parts.
_AMD_ARCHS: dict[str, AmdArch] = {
    "gfx950": AmdArch(  # CDNA4, Instinct MI355X / MI350X
        version=ArchVersion(9, 5),
        family="CDNA4",
        wavefront=64,
        lds_bytes=160 * 1024,
        # CDNA reports CUs directly as torch multiprocessors.
        cus_per_group=1,
        features=frozenset(
            {
                "matrix:f16",
                "matrix:bf16",
                "matrix:int8",
                "matrix:fp8",
                "mma:mfma",
                "memory:hbm",
                "memory:async_copy",
            }
        ),
        peak_bandwidth=8000.0,
        # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP per clock per CU.
        peak_bf16_tflops=2516.6,
    ),
}


@dataclass(frozen=True)
class PlatformInfo:
    """All that kernel selection may depend on (same fields as dexter's)."""

    vendor: str  # "amd" | "nvidia" | "cpu"
    arch: str  # "gfx950", ...
    arch_version: ArchVersion
    family: str  # "CDNA4", ...
    device_name: str
    compute_units: int
    wavefront: int
    lds_bytes: int
    total_memory: int  # bytes
    memory_bandwidth: float  # GB/s
    features: frozenset[str] = field(default_factory=frozenset)

    @property
    def is_amd(self) -> bool:
        return self.vendor == "amd"

    @property
    def is_rdna3_plus(self) -> bool:
        return self.is_amd and self.arch_version >= ArchVersion(11, 0)

    @property
    def is_cdna4(self) -> bool:
        return self.is_amd and self.family == "CDNA4"

    @property
    def has_unified_memory(self) -> bool:
        return "memory:unified" in self.features

    def supports(self, *features: str) -> bool:
        return all(f in self.features for f in features)

    def describe(self) -> str:
        """One line for error messages and ``explain``: arch first, then the device."""
        mem = f"{self.total_memory / 2**30:.0f} GiB" if self.total_memory else "no device memory"
        return (f"{self.arch}/{self.family} ({self.device_name}; {self.compute_units} CUs, "
                f"{self.wavefront}-lane waves, {mem}, {self.memory_bandwidth / 1e3:.2f} TB/s)")


@dataclass(frozen=True)
class Capability:
    """What a kernel needs from the platform (same semantics as dexter's)."""

    vendors: frozenset[str] | None = None
    min_arch: ArchVersion | None = None
    max_arch: ArchVersion | None = None
    features: frozenset[str] = field(default_factory=frozenset)

    def satisfied_by(self, platform: PlatformInfo) -> bool:
        if self.vendors is not None and platform.vendor not in self.vendors:
            return False
        if self.min_arch is not None and platform.arch_version < self.min_arch:
            return False
        if self.max_arch is not None and platform.arch_version > self.max_arch:
            return False
        return self.features <= platform.features


def _from_arch(arch: str, device_name: str, multiprocessors: int,
               total_memory: int) -> PlatformInfo:
    known = _AMD_ARCHS.get(arch)
    if known is None:
        rows = ", ".join(sorted(_AMD_ARCHS))
        raise RuntimeError(f"unsupported AMD architecture {arch!r}: no platform row for it "
                           f"(rows exist for {rows})")
    return PlatformInfo(
        vendor="amd",
        arch=arch,
        arch_version=known.version,
        family=known.family,
        device_name=device_name,
        compute_units=multiprocessors * known.cus_per_group,
        wavefront=known.wavefront,
        lds_bytes=known.lds_bytes,
        total_memory=total_memory,
        memory_bandwidth=known.peak_bandwidth,
        features=known.features,
    )


def cdna4_platform(compute_units: int = 256, total_memory: int = 288 * 10**9) -> PlatformInfo:
    """A gfx950 ``PlatformInfo`` without touching a device (tests, gate checks)."""
    return _from_arch("gfx950", "AMD Instinct MI355X", compute_units, total_memory)


def _cpu_platform() -> PlatformInfo:
    """No GPU: a platform no GPU kernel's gate admits."""
    return PlatformInfo(
        vendor="cpu",
        arch="cpu",
        arch_version=ArchVersion(0, 0),
        family="CPU",
        device_name="cpu",
        compute_units=os.cpu_count() or 1,
        wavefront=1,
        lds_bytes=0,
        total_memory=0,
        memory_bandwidth=0.0,
        features=frozenset(),
    )


@functools.lru_cache(maxsize=1)
def _detect() -> PlatformInfo:
    import torch

    if not torch.cuda.is_available():
        return _cpu_platform()
    props = torch.cuda.get_device_properties(torch.cuda.current_device())
    if not getattr(torch.version, "hip", None):
        raise RuntimeError("dexter_amd runs on ROCm builds of torch only")
    arch = props.gcnArchName.split(":")[0]  # drop ":sramecc+:xnack-"
    return _from_arch(arch, props.name, props.multi_processor_count, props.total_memory)


_override: PlatformInfo | None = None


def current_platform() -> PlatformInfo:
    """The detected platform (cached per process) unless overridden."""
    return _override if _override is not None else _detect()


def override_platform(platform: PlatformInfo | None) -> None:
    """Force a platform for tests and cross-arch gate checks; ``None`` undoes it."""
    global _override
    _override = platform


def peak_bf16_tflops(platform: PlatformInfo | None = None) -> float:
    """Datasheet dense bf16 MFMA peak of the platform's arch, 0 if unknown."""
    platform = platform or current_platform()
    known = _AMD_ARCHS.get(platform.arch)
    return known.peak_bf16_tflops if known else 0.0
