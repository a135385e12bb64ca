"""ctypes binding of libdexter_gfx950.so (declarations: include/dexter_gfx950.h).

The library is loaded once per process, behind a lock, from the package
directory where ``csrc/build.py`` puts it. There is no fallback: if the
library is missing or was built for another ABI revision, loading raises, and
so does every op that needs it.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_NAME = "libdexter_gfx950.so"
LIB_PATH = Path(__file__).resolve().parents[2] / LIB_NAME
ABI_VERSION = 10

DX_OK, DX_EINVAL, DX_ELAUNCH, DX_EFULL, DX_EWORKSPACE = 0, 1, 2, 3, 4
DX_BF16, DX_F16, DX_F32, DX_I32, DX_I64 = 0, 1, 2, 3, 4
# dx_set_tuning keys (launch-schedule overrides for measurement and tests).
(TUNE_ATTN_SPLITS, TUNE_ATTN_KERNEL, TUNE_NORM_WAVES, TUNE_QKV_SPLITS, TUNE_QKV_WAVES,
 TUNE_ATTN_MERGE, TUNE_ATTN_PMERGE) = range(7)

_DTYPE_CODE = {torch.bfloat16: DX_BF16, torch.float16: DX_F16, torch.float32: DX_F32,
               torch.int32: DX_I32, torch.int64: DX_I64}

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_f = ctypes.c_float

# Argument lists, in the header's order.
_SIGNATURES: dict[str, tuple[type, list]] = {
    "dx_last_error": (ctypes.c_char_p, []),
    "dx_abi_version": (_i, []),
    "dx_set_tuning": (_i, [_i, _i]),
    "dx_qk_norm_rope": (_i, [
        _p, _l, _l, _l,            # q, strides
        _p, _l, _l, _l,            # k, strides
        _i,                        # io dtype
        _p, _p, _i,                # q_weight, k_weight, weight dtype
        _p, _l, _p, _l, _i,        # cos, cos_sl, sin, sin_sl, table dtype
        _p, _p,                    # q_out, k_out
        _l, _l, _l, _l,            # B, L, H, D
        _f, _i, _p]),              # eps, interleaved, stream
    "dx_qk_norm_rope_append": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,            # v, strides
        _i,
        _p, _p, _i,
        _p, _l, _p, _l, _i,
        _p, _p,
        _p, _l, _l, _l, _l, _l, _l,  # cache, plane, sb, ss, sh, capacity, start
        _l, _l, _l, _l,
        _f, _i, _p]),
    "dx_kv_append": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l, _l,        # cache, plane, sb, ss, sh
        _i, _l, _l, _l, _l,        # dtype, B, n, H, D
        _l, _l, _p]),              # capacity, start, stream
    "dx_blockwise_causal_attention": (_i, [
        _p, _l, _l, _l,            # q
        _p, _l, _l, _l,            # k
        _p, _l, _l, _l,            # v
        _p, _l, _l, _l, _l,        # cache, plane, sb, ss, sh
        _p, _l, _l, _l,            # out
        _i, _l, _l, _l, _l, _l, _l,  # dtype, B, Lq, Lk, H, Hkv, D
        _l, _p, _i, _l,            # cache_len, starts, starts dtype, n_blocks
        _i, _f,                    # causal, scale
        _p, _l, _p]),              # workspace, bytes, stream
    "dx_qk_norm_rope_attention": (_i, [
        _p, _l, _l, _l,            # q (pre-norm)
        _p, _l, _l, _l,            # k (pre-norm)
        _p, _l, _l, _l,            # v
        _i,                        # io dtype
        _p, _p, _i,                # q_weight, k_weight, weight dtype
        _p, _l, _p, _l, _i,        # cos, cos_sl, sin, sin_sl, table dtype
        _f, _i,                    # eps, interleaved
        _p, _p,                    # q_out, k_out
        _p, _l, _l, _l, _l,        # cache, plane, sb, ss, sh
        _l, _l, _i,                # capacity, cache_len, append
        _p, _l, _l, _l,            # out
        _l, _l, _l, _l,            # B, L, H, D
        _p, _i, _l,                # starts, starts dtype, n_blocks
        _i, _f,                    # causal, scale
        _p, _l, _p]),              # workspace, bytes, stream
    "dx_blockwise_causal_attention_noalloc": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _l, _l, _l, _l, _l, _l,
        _l, _p, _i, _l,
        _i, _f,
        _p]),                      # stream (no workspace)
    "dx_blockwise_causal_attention_varlen": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _l, _l, _l, _l, _l, _l,
        ctypes.POINTER(ctypes.c_int64), _p, _i, _l,
        _i, _f,
        _p, _l, _p]),
    "dx_blockwise_causal_attention_dev": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _l, _l, _l, _l, _l, _l,
        _p, _l,                    # device cache length (int32), cache capacity
        _p, _i, _l,
        _i, _f,
        _p, _l, _p]),
    "dx_kv_append_dev": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l, _l,
        _i, _l, _l, _l, _l,
        _l, _p, _p, _p]),          # capacity, device start (int32), status, stream
    "dx_qk_norm_rope_append_dev": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _i,
        _p, _p, _i,
        _p, _l, _p, _l, _i,
        _p, _p,
        _p, _l, _l, _l, _l, _l, _p, _p,  # cache, plane, sb, ss, sh, capacity, start, status
        _l, _l, _l, _l,
        _f, _i, _p]),
    "dx_attention_workspace_bytes": (_l, [_l, _l, _l, _l, _l, _l,
                                          ctypes.POINTER(ctypes.c_int64)]),
    "dx_qkv_norm_rope": (_i, [
        _p, _l, _l, _i,            # x, sb, sl, io dtype
        _p, _p, _p, _l,            # wq, wk, wv, weight row stride
        _p, _p, _p,                # bq, bk, bv (may be null)
        _p, _p, _i,                # q/k norm weights, dtype
        _p, _l, _p, _l, _i,        # cos, cos_sl, sin, sin_sl, table dtype
        _p, _p, _p,                # q_out, k_out, v_out
        _p, _l, _l, _l, _l,        # cache (may be null), plane, sb, ss, sh
        _l, _l, _p, _p,            # capacity, start, device start, status
        _l, _l, _l, _l, _l,        # B, L, C, H, D
        _f, _i,                    # eps, interleaved
        _p, _l, _p]),              # workspace, bytes, stream
    "dx_qkv_workspace_bytes": (_l, [_l, _l, _l, _l, _l]),
    "dx_adaln_modulate": (_i, [
        _p, _l, _l, _i,            # x, sb, sl, x dtype
        _p, _l, _l,                # scale, sb, sl
        _p, _l, _l, _i,            # shift, sb, sl, modulation dtype
        _p, _l, _l, _i,            # out, sb, sl, out dtype
        _l, _l, _l, _f, _p]),      # B, L, C, eps, stream
    "dx_gated_residual": (_i, [
        _p, _l, _l,                # x, sb, sl
        _p, _l, _l, _i,            # y, sb, sl, x/y dtype
        _p, _l, _l, _i,            # gate, sb, sl, gate dtype
        _p, _l, _l, _i,            # out, sb, sl, out dtype
        _l, _l, _l, _p]),          # B, L, C, stream
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    """Every function name the header declares (and the loader binds)."""
    return list(_SIGNATURES)


def load() -> ctypes.CDLL:
    """The loaded library, with argument/return types set. Raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_NAME} is not built ({LIB_PATH}); run "
                    "`python dexter-labs_amd/csrc/build.py` (or __graft_entry__.build())")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            got = lib.dx_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_NAME} ABI {got}, expected {ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Turn a DX_E* return code into the matching Python exception."""
    if rc == DX_OK:
        return
    msg = load().dx_last_error().decode(errors="replace")
    if rc == DX_EFULL:
        raise RuntimeError(msg)  # "KV cache full: ..." as the reference raises
    if rc == DX_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[t]
    except KeyError:
        raise ValueError(f"dtype {t} has no kernel") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_tuning_values: dict[int, int] = {}


def set_tuning(key: int, value: int) -> None:
    """Process-wide launch-schedule override (0 restores the library's choice)."""
    check(load().dx_set_tuning(int(key), int(value)), "set_tuning")
    _tuning_values[int(key)] = int(value)


def get_tuning(key: int) -> int:
    """The override last set through ``set_tuning`` for ``key`` (0: none)."""
    return _tuning_values.get(int(key), 0)


class tuning:
    """Context manager for launch-schedule overrides, e.g.
    ``with tuning(TUNE_ATTN_SPLITS, 4): ...``; on exit the key gets back the
    value it had on entry, so nested contexts and an outer ``set_tuning``
    survive an inner context."""

    def __init__(self, key: int, value: int) -> None:
        self.key, self.value = key, value
        self.saved = 0

    def __enter__(self) -> "tuning":
        self.saved = get_tuning(self.key)
        set_tuning(self.key, self.value)
        return self

    def __exit__(self, *exc) -> None:
        set_tuning(self.key, self.saved)


_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Outgrown workspaces, never released: a graph captured while one was current
# replays with its address, so its memory must not go back to the allocator.
# Growth doubles, so these hold less than the current buffers do.
_retired: list[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A zero-initialised scratch buffer of at least ``nbytes`` for the current stream.

    One buffer per (device, stream), kept between calls and grown when needed.
    The attention kernels keep arrival counters in it that must be zero when a
    call starts and that every call leaves at zero, so the buffer is zeroed
    once, when it is allocated. Calls on one stream are ordered, so they never
    share it concurrently. A buffer first needed under graph capture is
    allocated in the graph's memory pool and its zero fill is recorded (each
    replay clears it again, which is harmless): warm a captured call up on the
    capture stream (``runtime.capture`` and the bench do) to keep the fill out.
    """
    if nbytes <= 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           stream_handle(device))
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 2 * buf.numel() if buf is not None else 0)
            if buf is not None:
                _retired.append(buf)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _workspaces[key] = buf
    return buf
