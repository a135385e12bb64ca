"""QK-RMSNorm + rotary on gfx950 (HIP kernel ``dx_qk_norm_rope``).

Registered as ``rope/qk_norm_rope`` with the signature of dexter's
implementations (``ops/reference/rope.py:43-56``,
``ops/gfx1151/rope/qk_norm_rope.py:93-110``):
``(q, k, q_weight, k_weight, cos, sin, eps, interleaved=True) -> (q, k)``.
The norm spans the whole ``H*D`` plane of a token and the weight is ``H*D``
long (Wan's QK norm runs before the head split). One workgroup per token and
plane (q, k, and v when the cache append writes it).

``rope/qk_norm_rope_append`` is the same pass with the rotated k and the raw
v also written into rows ``[start, start+L)`` of a ``[2, B, S, H, D]`` cache
(the fused form of ``KVCache.append``, ``models/dreamzero/model.py:53-58``).
``start`` may be a device cursor (one int32 on the device,
``dx_qk_norm_rope_append_dev``), read when the kernel runs; a block that would
not fit is then not written to the cache and ``status`` (optional int32) is set
to 1, while q and k are still returned.
"""

from __future__ import annotations

import torch

from ...registry import Priority, register
from . import _lib
from ._common import CDNA4, MATRIX_DTYPES, as_rows, device_cursor, strides

_TABLE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_MAX_PLANE = 256 * 4 * 16


def _accepts(q, k, *args, **kwargs) -> bool:
    return (q.is_cuda and k.is_cuda and q.dtype in MATRIX_DTYPES and k.dtype == q.dtype
            and q.dim() == 4 and q.shape == k.shape and q.shape[-1] % 16 == 0
            and q.shape[2] * q.shape[3] <= _MAX_PLANE)


def _accepts_append(q, k, v, cache, *args, **kwargs) -> bool:
    return (_accepts(q, k) and v.shape == q.shape and v.dtype == q.dtype
            and cache.dtype == q.dtype and cache.is_cuda)


def _prepare(q, k, q_weight, k_weight, cos, sin):
    if q.shape != k.shape or q.dim() != 4:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} must both be [B, L, H, D]")
    b, seq, heads, dim = q.shape
    if q_weight.numel() != heads * dim or k_weight.numel() != heads * dim:
        raise ValueError(f"norm weights must have H*D = {heads * dim} elements")
    wdt = q_weight.dtype if q_weight.dtype in _TABLE_DTYPES else torch.float32
    qw = q_weight.reshape(-1).to(device=q.device, dtype=wdt).contiguous()
    kw = k_weight.reshape(-1).to(device=q.device, dtype=wdt).contiguous()
    tdt = cos.dtype if cos.dtype in _TABLE_DTYPES else torch.float32
    tables = []
    for t in (cos, sin):
        if t.dim() != 2 or t.shape[-1] != dim // 2 or t.shape[0] not in (seq, 1):
            raise ValueError(f"cos/sin must be [L, D/2] = [{seq}, {dim // 2}], got {tuple(t.shape)}")
        tables.append(as_rows(t.to(device=q.device, dtype=tdt)))
    return as_rows(q), as_rows(k), qw, kw, tables[0], tables[1], tdt


def _row_stride(t: torch.Tensor) -> int:
    return 0 if t.shape[0] == 1 else t.stride(0)


@register("rope", "qk_norm_rope", name="hip_qk_norm_rope_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts)
def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps, interleaved=True):
    q, k, qw, kw, c, s, tdt = _prepare(q, k, q_weight, k_weight, cos, sin)
    b, seq, heads, dim = q.shape
    q_out = torch.empty((b, seq, heads, dim), device=q.device, dtype=q.dtype)
    k_out = torch.empty_like(q_out)
    lib = _lib.load()
    rc = lib.dx_qk_norm_rope(
        q.data_ptr(), *strides(q, 3), k.data_ptr(), *strides(k, 3),
        _lib.dtype_code(q.dtype),
        qw.data_ptr(), kw.data_ptr(), _lib.dtype_code(qw.dtype),
        c.data_ptr(), _row_stride(c), s.data_ptr(), _row_stride(s), _lib.dtype_code(tdt),
        q_out.data_ptr(), k_out.data_ptr(), b, seq, heads, dim,
        float(eps), int(bool(interleaved)), _lib.stream_handle(q.device))
    _lib.check(rc, "qk_norm_rope")
    return q_out, k_out


@register("rope", "qk_norm_rope_append", name="hip_qk_norm_rope_append_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts_append)
def qk_norm_rope_append(q, k, v, q_weight, k_weight, cos, sin, cache, start, eps,
                        interleaved=True, status=None):
    q, k, qw, kw, c, s, tdt = _prepare(q, k, q_weight, k_weight, cos, sin)
    b, seq, heads, dim = q.shape
    if v.shape != q.shape or v.dtype != q.dtype:
        raise ValueError("v must match q in shape and dtype")
    if cache.dim() != 5 or cache.shape[0] != 2 or tuple(cache.shape[1:2]) != (b,) \
            or tuple(cache.shape[3:]) != (heads, dim) or cache.dtype != q.dtype:
        raise ValueError(f"cache must be [2, {b}, S, {heads}, {dim}] of {q.dtype}, "
                         f"got {tuple(cache.shape)} {cache.dtype}")
    if not (cache.stride(-1) == 1 and cache.data_ptr() % 16 == 0
            and all(x % 8 == 0 for x in cache.stride()[:-1])):
        raise ValueError("cache must have a contiguous, 16-byte aligned head_dim")
    v = as_rows(v)
    q_out = torch.empty((b, seq, heads, dim), device=q.device, dtype=q.dtype)
    k_out = torch.empty_like(q_out)
    lib = _lib.load()
    head = [q.data_ptr(), *strides(q, 3), k.data_ptr(), *strides(k, 3), v.data_ptr(),
            *strides(v, 3), _lib.dtype_code(q.dtype),
            qw.data_ptr(), kw.data_ptr(), _lib.dtype_code(qw.dtype),
            c.data_ptr(), _row_stride(c), s.data_ptr(), _row_stride(s), _lib.dtype_code(tdt),
            q_out.data_ptr(), k_out.data_ptr(),
            cache.data_ptr(), cache.stride(0), cache.stride(1), cache.stride(2),
            cache.stride(3), cache.shape[2]]
    tail = [b, seq, heads, dim, float(eps), int(bool(interleaved)), _lib.stream_handle(q.device)]
    if isinstance(start, torch.Tensor):
        start = device_cursor(start, q.device, "qk_norm_rope_append")
        if status is not None:
            status = device_cursor(status, q.device, "qk_norm_rope_append status")
        rc = lib.dx_qk_norm_rope_append_dev(*head, start.data_ptr(), _lib.ptr(status), *tail)
    else:
        rc = lib.dx_qk_norm_rope_append(*head, int(start), *tail)
    _lib.check(rc, "qk_norm_rope_append")
    return q_out, k_out
