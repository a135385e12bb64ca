"""Registry and platform semantics (no GPU): the drop-in boundary.

Mirrors the rules of dexter's registry (``python/dexter/registry.py:34-173``)
and platform gates (``python/dexter/platform.py:169-185``), using fake
``PlatformInfo`` values for gfx950, an RDNA3.5 part and the CPU.
"""

from __future__ import annotations

import dataclasses
import re

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd import platform as plat
from dexter_amd import registry as reg
from dexter_amd.ops.gfx950._common import CDNA4


@pytest.fixture
def cdna4():
    plat.override_platform(plat.cdna4_platform())
    yield plat.current_platform()
    plat.override_platform(None)


@pytest.fixture
def cpu():
    plat.override_platform(plat._cpu_platform())
    yield plat.current_platform()
    plat.override_platform(None)


def rdna35() -> plat.PlatformInfo:
    return plat.PlatformInfo(
        vendor="amd", arch="gfx1151", arch_version=plat.ArchVersion(11, 5), family="RDNA3.5",
        device_name="Strix Halo", compute_units=40, wavefront=32, lds_bytes=64 * 1024,
        total_memory=0, memory_bandwidth=256.0,
        features=frozenset({"matrix:bf16", "mma:wmma", "memory:unified"}))


RDNA3_GATE = plat.Capability(vendors=frozenset({"amd"}), min_arch=plat.ArchVersion(11, 0),
                             features=frozenset({"mma:wmma", "matrix:bf16"}))


def test_cdna4_platform_row():
    p = plat.cdna4_platform()
    assert p.is_amd and p.arch == "gfx950" and p.family == "CDNA4" and p.is_cdna4
    assert p.wavefront == 64 and p.lds_bytes == 160 * 1024 and p.compute_units == 256
    assert p.supports("mma:mfma", "matrix:bf16", "matrix:fp8")
    assert not p.supports("mma:wmma") and not p.is_rdna3_plus
    assert "gfx950" in p.describe() and "CDNA4" in p.describe()


def test_unknown_amd_arch_raises():
    with pytest.raises(RuntimeError, match="unsupported AMD architecture 'gfx1234'"):
        plat._from_arch("gfx1234", "x", 1, 0)


def test_gates_do_not_cross():
    assert CDNA4.satisfied_by(plat.cdna4_platform())
    assert not CDNA4.satisfied_by(rdna35())
    assert not CDNA4.satisfied_by(plat._cpu_platform())
    assert RDNA3_GATE.satisfied_by(rdna35())
    assert not RDNA3_GATE.satisfied_by(plat.cdna4_platform())  # (9,5) < (11,0)


@pytest.mark.parametrize("key,name", [
    ("attention/blockwise_causal", "hip_blockwise_causal_gfx950"),
    ("rope/qk_norm_rope", "hip_qk_norm_rope_gfx950"),
    ("cache/append", "hip_kv_append_gfx950"),
    ("rope/qk_norm_rope_append", "hip_qk_norm_rope_append_gfx950"),
    ("attention/blockwise_causal_varlen", "hip_blockwise_causal_varlen_gfx950"),
    ("rope/qkv_norm_rope", "hip_qkv_norm_rope_gfx950"),
    ("norm/adaln", "hip_adaln_gfx950"),
    ("norm/gated_residual", "hip_gated_residual_gfx950"),
])
def test_hip_kernels_registered_specialised(key, name):
    specs = reg.registered(*key.split("/"))
    spec = next(s for s in specs if s.name == name)
    assert int(spec.priority) == int(reg.Priority.SPECIALISED)
    assert spec.capability == CDNA4


def test_selection_on_cdna4_picks_hip(cdna4):
    fam, mode = "attention", "blockwise_causal"
    spec = next(reg.candidates(fam, mode))
    assert spec.name == "hip_blockwise_causal_gfx950"
    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)  # CPU tensor: declined by accepts
    text = reg.explain(fam, mode, q, q, q)
    assert "gfx950" in text and "hip_blockwise_causal_gfx950" in text
    assert "declined" in text and "no selection" in text


def test_no_fallback_on_cpu(cpu):
    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(LookupError, match="no kernel for attention/blockwise_causal"):
        ops.blockwise_causal_attention(q, q, q)
    with pytest.raises(LookupError, match="no kernel for rope/qk_norm_rope"):
        w = torch.ones(128)
        ops.qk_norm_rope(q, q, w, w, torch.ones(4, 32), torch.zeros(4, 32))
    with pytest.raises(LookupError, match="no kernel for cache/append"):
        ops.kv_cache_append(torch.zeros(2, 1, 8, 2, 64, dtype=torch.bfloat16), q, q, 0)
    x = torch.zeros(1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(LookupError, match="no kernel for norm/adaln"):
        ops.adaln_modulate(x, x[:, :1], x[:, :1])
    with pytest.raises(LookupError, match="no kernel for norm/gated_residual"):
        ops.gated_residual(x, x, x[:, :1])


def test_accepts_declines_shapes_the_kernel_does_not_cover(cdna4):
    # accepts() needs .is_cuda; a CPU tensor on a faked gfx950 is declined.
    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(LookupError):
        reg.select("attention", "blockwise_causal", q, q, q)


# ---------------------------------------------- generic registry rules -----

@pytest.fixture
def scratch_family():
    fam, mode = "test", "probe"
    yield fam, mode
    for s in reg.registered(fam, mode):
        reg.unregister(fam, mode, s.name)


def test_priority_order_and_reference_never_wins(cdna4, scratch_family):
    fam, mode = scratch_family
    reg.register(fam, mode, name="ref", priority=reg.Priority.REFERENCE)(lambda: "ref")
    reg.register(fam, mode, name="fast", priority=reg.Priority.PERFORMANT)(lambda: "fast")
    reg.register(fam, mode, name="best", priority=reg.Priority.SPECIALISED,
                 capability=CDNA4)(lambda: "best")
    assert reg.select(fam, mode)() == "best"
    plat.override_platform(rdna35())
    assert reg.select(fam, mode)() == "fast"


def test_capability_checked_before_priority(scratch_family):
    fam, mode = scratch_family
    plat.override_platform(rdna35())
    try:
        reg.register(fam, mode, name="cdna_only", priority=99, capability=CDNA4)(lambda: 1)
        reg.register(fam, mode, name="generic", priority=1)(lambda: 2)
        assert reg.select(fam, mode)() == 2
    finally:
        plat.override_platform(None)


def test_accepts_predicate_and_args_not_forwarded(cdna4, scratch_family):
    fam, mode = scratch_family
    seen = []

    def small_only(x):
        seen.append(x)
        return x < 10

    reg.register(fam, mode, name="small", priority=12, accepts=small_only)(lambda: "small")
    reg.register(fam, mode, name="any", priority=4)(lambda: "any")
    assert reg.select(fam, mode, 3)() == "small"
    assert reg.select(fam, mode, 30)() == "any"
    assert seen == [3, 30]
    text = reg.explain(fam, mode, 30)
    assert re.search(r"declined +small", text) and re.search(r"chosen +any", text)


def test_pin_wins_and_bad_pin_raises(cdna4, scratch_family, monkeypatch):
    fam, mode = scratch_family
    reg.register(fam, mode, name="a", priority=12)(lambda: "a")
    reg.register(fam, mode, name="b", priority=4)(lambda: "b")
    monkeypatch.setenv("DEXTER_KERNEL", f"other/x:zzz, {fam}/{mode}:b")
    assert reg.select(fam, mode)() == "b"
    monkeypatch.setenv("DEXTER_KERNEL", f"{fam}/{mode}:missing")
    with pytest.raises(LookupError, match="pinned test/probe:missing"):
        reg.select(fam, mode)


def test_duplicate_name_rejected(scratch_family):
    fam, mode = scratch_family
    reg.register(fam, mode, name="dup")(lambda: 1)
    with pytest.raises(ValueError, match="duplicate kernel test/probe:dup"):
        reg.register(fam, mode, name="dup")(lambda: 2)


def test_no_viable_kernel_message(cpu, scratch_family):
    fam, mode = scratch_family
    reg.register(fam, mode, name="gpu_only", capability=CDNA4)(lambda: 1)
    with pytest.raises(LookupError, match=r"Registered: \['gpu_only'\]"):
        reg.select(fam, mode)


def test_platform_info_is_frozen():
    p = plat.cdna4_platform()
    with pytest.raises(dataclasses.FrozenInstanceError):
        p.arch = "x"  # type: ignore[misc]


def test_equal_priority_keeps_registration_order(cdna4, scratch_family):
    fam, mode = scratch_family
    for name in ("first", "second", "third"):
        reg.register(fam, mode, name=name, priority=8)(lambda n=name: n)
    reg.register(fam, mode, name="top", priority=12, accepts=lambda: False)(lambda: "top")
    assert [s.name for s in reg.registered(fam, mode)] == ["top", "first", "second", "third"]
    assert reg.select(fam, mode)() == "first"
    reg.unregister(fam, mode, "first")
    assert reg.select(fam, mode)() == "second"


def test_pin_overrides_accepts_but_not_gate(cdna4, scratch_family, monkeypatch):
    fam, mode = scratch_family
    reg.register(fam, mode, name="picky", priority=12, accepts=lambda: False)(lambda: "picky")
    reg.register(fam, mode, name="gated", priority=12,
                 capability=plat.Capability(vendors=frozenset({"nvidia"})))(lambda: "gated")
    monkeypatch.setenv("DEXTER_KERNEL", f"{fam}/{mode}:picky")
    assert reg.select(fam, mode)() == "picky"
    monkeypatch.setenv("DEXTER_KERNEL", f"{fam}/{mode}:gated")
    with pytest.raises(LookupError, match="not available here"):
        reg.select(fam, mode)
    # An entry without ':' pins the empty name: nothing matches.
    monkeypatch.setenv("DEXTER_KERNEL", f"{fam}/{mode}")
    with pytest.raises(LookupError, match=f"pinned {fam}/{mode}:,"):
        reg.select(fam, mode)
    # The first entry for a key wins.
    monkeypatch.setenv("DEXTER_KERNEL", f"{fam}/{mode}:picky,{fam}/{mode}:gated")
    assert reg.select(fam, mode)() == "picky"


def test_explain_rows(cdna4, scratch_family):
    fam, mode = scratch_family
    reg.register(fam, mode, name="wmma", priority=12,
                 capability=plat.Capability(features=frozenset({"mma:wmma"})))(lambda: 0)
    reg.register(fam, mode, name="small", priority=8, accepts=lambda x: x < 10)(lambda: 1)
    reg.register(fam, mode, name="any", priority=4)(lambda: 2)
    rows = reg.explain(fam, mode, 30).splitlines()
    assert rows[0].startswith(f"{fam}/{mode} on ") and "gfx950" in rows[0]
    assert re.match(r"  gated +wmma +priority 12: platform lacks \['mma:wmma'\]", rows[1])
    assert re.match(r"  declined +small +priority  8: accepts\(\) declined", rows[2])
    assert re.match(r"  chosen +any +priority  4$", rows[3])
    rows = reg.explain(fam, mode, 3).splitlines()
    assert re.match(r"  chosen +small", rows[2]) and re.match(r"  eligible +any", rows[3])
