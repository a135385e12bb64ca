"""The C-ABI library: it loads and exports every symbol the header declares.

No device work happens here: only calls that fail argument validation before
touching the HIP runtime, and the version query.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from dexter_amd.ops.gfx950 import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "dexter_gfx950.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_functions()
    for want in ("dx_qk_norm_rope", "dx_qk_norm_rope_append", "dx_kv_append",
                 "dx_blockwise_causal_attention", "dx_blockwise_causal_attention_varlen",
                 "dx_attention_workspace_bytes", "dx_last_error", "dx_abi_version",
                 "dx_adaln_modulate", "dx_gated_residual"):
        assert want in names


def test_library_exports_every_declared_symbol(built_lib):
    lib = ctypes.CDLL(str(built_lib))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_library_resolves_all_of_its_own_symbols(built_lib):
    """No kernel or stub of the library's own namespace is left undefined (a
    dropped template instantiation links, then fails at load on the GPU box)."""
    import shutil
    import subprocess
    if shutil.which("nm") is None:
        pytest.skip("nm not available")
    out = subprocess.run(["nm", "-D", "--undefined-only", str(built_lib)], capture_output=True,
                         text=True, check=True).stdout
    own = [line.split()[-1] for line in out.splitlines() if "_ZN2dx" in line]
    assert not own, f"undefined: {own}"


def test_product_library_carries_no_phase_stamps(built_lib):
    """The timeline build's readers (and so its stamp code) exist only in the measurement
    library that `build.py --timeline` writes beside this one."""
    lib = ctypes.CDLL(str(built_lib))
    stamped = [n for n in ("dx_timeline_words", "dx_timeline_read", "dx_timeline_clear")
               if hasattr(lib, n)]
    assert not stamped, f"product library exports {stamped}"


def test_loader_binds_exactly_the_header(built_lib):
    assert sorted(_lib.exported_symbols()) == declared_functions()


def test_abi_version(built_lib):
    lib = _lib.load()
    assert lib.dx_abi_version() == _lib.ABI_VERSION
    header_version = int(re.search(r"#define DX_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert header_version == _lib.ABI_VERSION


def test_overflow_is_reported_before_any_launch(built_lib):
    lib = _lib.load()
    rc = lib.dx_kv_append(16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, 0,
                          _lib.DX_BF16, 1, 5, 2, 64, 8, 4, None)
    assert rc == _lib.DX_EFULL
    assert lib.dx_last_error().decode() == "KV cache full: 4 + 5 > 8"
    with pytest.raises(RuntimeError, match="KV cache full: 4 \\+ 5 > 8"):
        _lib.check(rc, "kv_append")


def test_bad_arguments_are_rejected(built_lib):
    lib = _lib.load()
    rc = lib.dx_kv_append(16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, 0,
                          99, 1, 1, 2, 64, 8, 0, None)
    assert rc == _lib.DX_EINVAL and "dtype" in lib.dx_last_error().decode()
    args = [16, 0, 0, 0] * 3 + [None, 0, 0, 0, 0] + [16, 0, 0, 0]
    # (dtype, B, Lq, Lk, H, Hkv, D, cache_len, starts, starts dtype, n_blocks, causal, scale,
    #  workspace, bytes, stream)
    rc = lib.dx_blockwise_causal_attention(*args, _lib.DX_BF16, 1, 8, 8, 2, 2, 96, 0, None,
                                           _lib.DX_I32, 0, 0, 1.0, None, 0, None)
    assert rc == _lib.DX_EINVAL and "head_dim 96" in lib.dx_last_error().decode()
    # Lk != Lq is cross-attention, defined only without a causal or block mask.
    rc = lib.dx_blockwise_causal_attention(*args, _lib.DX_BF16, 1, 8, 9, 2, 2, 128, 0, None,
                                           _lib.DX_I32, 0, 1, 1.0, None, 0, None)
    assert rc == _lib.DX_EINVAL and "must equal q length" in lib.dx_last_error().decode()
    with pytest.raises(ValueError, match="must equal q length"):
        _lib.check(rc, "attention")
    rc = lib.dx_blockwise_causal_attention(*args, _lib.DX_BF16, 1, 8, 8, 6, 4, 128, 0, None,
                                           _lib.DX_I32, 0, 0, 1.0, None, 0, None)
    assert rc == _lib.DX_EINVAL and "not a multiple" in lib.dx_last_error().decode()
    rc = lib.dx_blockwise_causal_attention(*args, _lib.DX_BF16, 1, 8, 0, 2, 2, 128, 0, None,
                                           _lib.DX_I32, 0, 0, 1.0, None, 0, None)
    assert rc == _lib.DX_EINVAL and "no keys" in lib.dx_last_error().decode()


def test_norm_entry_points_validate_before_any_launch(built_lib):
    lib = _lib.load()
    bf, f32 = _lib.DX_BF16, _lib.DX_F32
    # Empty rows: success, nothing launched (null pointers are never touched).
    assert lib.dx_adaln_modulate(None, 0, 0, bf, None, 0, 0, None, 0, 0, bf,
                                 None, 0, 0, bf, 1, 0, 3072, 1e-6, None) == _lib.DX_OK
    assert lib.dx_gated_residual(None, 0, 0, None, 0, 0, bf, None, 0, 0, bf,
                                 None, 0, 0, bf, 0, 5, 3072, None) == _lib.DX_OK
    rc = lib.dx_adaln_modulate(None, 0, 0, 7, None, 0, 0, None, 0, 0, bf,
                               None, 0, 0, bf, 1, 1, 64, 1e-6, None)
    assert rc == _lib.DX_EINVAL and "dtype codes" in lib.dx_last_error().decode()
    rc = lib.dx_adaln_modulate(None, 0, 0, bf, None, 0, 0, None, 0, 0, f32,
                               None, 0, 0, bf, 1, 1, 64, 1e-6, None)
    assert rc == _lib.DX_EINVAL and "promotion" in lib.dx_last_error().decode()
    rc = lib.dx_gated_residual(None, 0, 0, None, 0, 0, bf, None, 0, 0, bf,
                               None, 0, 0, bf, 1, 1, 1 << 20, None)
    assert rc == _lib.DX_EINVAL and "exceeds" in lib.dx_last_error().decode()
    rc = lib.dx_gated_residual(None, 0, 0, None, 0, 0, bf, None, 0, 0, bf,
                               None, 0, 0, bf, 70000, 1, 64, None)
    assert rc == _lib.DX_EINVAL and "grid limits" in lib.dx_last_error().decode()
    with pytest.raises(ValueError, match="grid limits"):
        _lib.check(rc, "gated_residual")


def test_noalloc_refuses_a_call_beyond_its_scratch_before_any_launch(built_lib):
    """The no-allocation entry point plans first and refuses a call whose
    workspace exceeds the static scratch (64 MiB) without touching memory:
    128 heads x 16 forced splits need ~71 MB of partials."""
    lib = _lib.load()
    h, d, lq, c = 128, 128, 128, 4096
    row = h * d  # [B, L, H, D] contiguous: strides (L*H*D, H*D, D)
    qkv = [16, lq * row, row, d] * 3
    cache = [16, (c + lq) * row, (c + lq) * row, row, d]
    out = [16, lq * row, row, d]
    with _lib.tuning(_lib.TUNE_ATTN_SPLITS, 16):
        need = lib.dx_attention_workspace_bytes(1, lq, lq, h, d, c, None)
        rc = lib.dx_blockwise_causal_attention_noalloc(
            *qkv, *cache, *out, _lib.DX_BF16, 1, lq, lq, h, h, d, c, None, _lib.DX_I32, 0, 0,
            0.088, None)
    assert need > (64 << 20)
    assert rc == _lib.DX_EWORKSPACE
    assert "static scratch" in lib.dx_last_error().decode()


def test_planner_choices_at_the_measured_shapes(built_lib):
    """The launch plans at the benchmark shapes, read back through the workspace
    size (256 KiB of arrival counters, then per partial `rows` f16 values of D
    and a 16-byte record per row). Each split count was chosen by measurement:
    C1 8 splits of 128-row items, C3 3 splits of 256-row items, the C4 ragged
    batch 1/1/2/6 by length, cross-attention onto 257 image keys 5 splits of one
    tile and onto 512 text keys 4 of two; C2 (768 items) has none. Runs without
    a GPU, where the planner assumes MI355X's 256 CUs."""
    lib = _lib.load()
    counters, d = 256 << 10, 128

    def ws(partials, rows):
        return counters + partials * rows * (2 * d + 16)

    assert lib.dx_attention_workspace_bytes(1, 83, 83, 24, d, 1245, None) == ws(24 * 8, 128)
    assert lib.dx_attention_workspace_bytes(1, 8192, 8192, 24, d, 0, None) == 0
    assert lib.dx_attention_workspace_bytes(1, 913, 913, 40, d, 7304, None) == ws(40 * 4 * 3, 256)
    lens = (ctypes.c_int64 * 4)(0, 332, 1245, 3237)
    assert lib.dx_attention_workspace_bytes(4, 99, 99, 24, d, 0, lens) == ws(24 * (1 + 1 + 2 + 6), 128)
    assert lib.dx_attention_workspace_bytes(1, 83, 257, 24, d, 0, None) == ws(24 * 5, 128)
    assert lib.dx_attention_workspace_bytes(1, 83, 512, 24, d, 0, None) == ws(24 * 4, 128)


def test_general_kernel_plan(built_lib):
    """fp32 inputs and head dims 16, 32, 256 run on the general kernel, whose
    workspace is the counter region (never written by it) and then, per split
    of each 64-query item, 64 rows of D fp32 values and an 8-byte {m, l}
    record. About two items per CU (256 CUs without a GPU), at least two
    32-key tiles per split; none when the items alone fill the chip. The
    workspace query takes no dtype: at head dims 64 and 128 it reports the
    16-bit kernels' bytes, within which fp32 calls lower their split count."""
    lib = _lib.load()
    counters = 256 << 10

    def ws(items, d):
        return counters + items * 64 * (4 * d + 8)

    # 83 queries x 24 heads: 48 items, 512 // 48 = 10 splits over 42 tiles.
    assert lib.dx_attention_workspace_bytes(1, 83, 83, 24, 256, 1245, None) == ws(48 * 10, 256)
    assert lib.dx_attention_workspace_bytes(1, 83, 83, 24, 32, 1245, None) == ws(48 * 10, 32)
    # Few keys: at most one split per two tiles (40 keys: 2 tiles, 1 split).
    assert lib.dx_attention_workspace_bytes(1, 20, 20, 2, 16, 20, None) == 0
    # 3,072 items: no split.
    assert lib.dx_attention_workspace_bytes(1, 8192, 8192, 24, 32, 0, None) == 0
    lens = (ctypes.c_int64 * 2)(100, 3000)
    assert lib.dx_attention_workspace_bytes(2, 16, 16, 4, 256, 0, lens) == ws(8 * 16, 256)
    assert lib.dx_attention_workspace_bytes(1, 8, 8, 2, 96, 0, None) < 0
    # Dtype codes other than bf16, f16 and f32 are refused before any launch.
    args = [16, 0, 0, 0] * 3 + [None, 0, 0, 0, 0] + [16, 0, 0, 0]
    rc = lib.dx_blockwise_causal_attention(*args, 7, 1, 8, 8, 2, 2, 64, 0, None,
                                           _lib.DX_I32, 0, 0, 1.0, None, 0, None)
    assert rc == _lib.DX_EINVAL and "dtype code 7" in lib.dx_last_error().decode()
