"""KV-cache chunk append on gfx950 (HIP kernel ``dx_kv_append``).

Registered as ``cache/append``: ``(cache, k, v, start) -> None`` writes
``k``/``v`` ``[B, n, H, D]`` into rows ``[start, start+n)`` of planes 0/1 of
``cache`` ``[2, B, S, H, D]``, the work ``KVCache.append`` does with two
torch slice copies (``models/dreamzero/model.py:53-58``). The overflow check
runs on the host before any launch and raises the reference's
``RuntimeError("KV cache full: ...")``.

``start`` may also be a device cursor (one int32 on the cache's device,
``dx_kv_append_dev``): the kernel reads it when it runs, so a captured graph
appends at the cursor's current value on every replay. The host cannot check
it; a block that would not fit is then not written, and ``status`` (an int32
on the device, optional) is set to 1.
"""

from __future__ import annotations

import torch

from ...registry import Priority, register
from . import _lib
from ._common import CDNA4, as_rows, device_cursor, strides

_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _accepts(cache, k, v, *args, **kwargs) -> bool:
    return (cache.is_cuda and cache.dtype in _DTYPES and k.dtype == cache.dtype
            and v.dtype == cache.dtype and cache.dim() == 5 and k.dim() == 4
            and k.shape == v.shape
            and (k.shape[-1] * k.element_size()) % 16 == 0)


@register("cache", "append", name="hip_kv_append_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts)
def kv_cache_append(cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor, start,
                    status: torch.Tensor | None = None) -> None:
    if k.shape != v.shape or k.dim() != 4:
        raise ValueError("k and v must both be [B, n, H, D]")
    b, n, heads, dim = k.shape
    if cache.dim() != 5 or cache.shape[0] != 2 or cache.shape[1] != b \
            or tuple(cache.shape[3:]) != (heads, dim):
        raise ValueError(f"cache must be [2, {b}, S, {heads}, {dim}], got {tuple(cache.shape)}")
    capacity = cache.shape[2]
    on_device = isinstance(start, torch.Tensor)
    if on_device:
        start = device_cursor(start, cache.device, "kv_cache_append")
        if status is not None:
            status = device_cursor(status, cache.device, "kv_cache_append status")
    else:
        start = int(start)
        if start + n > capacity:
            raise RuntimeError(f"KV cache full: {start} + {n} > {capacity}")
    per16 = 16 // cache.element_size()
    if not (cache.stride(-1) == 1 and cache.data_ptr() % 16 == 0
            and all(x % per16 == 0 for x in cache.stride()[:-1])):
        raise ValueError("cache must have a contiguous, 16-byte aligned head_dim")
    k, v = as_rows(k), as_rows(v)
    lib = _lib.load()
    args = [k.data_ptr(), *strides(k, 3), v.data_ptr(), *strides(v, 3),
            cache.data_ptr(), cache.stride(0), cache.stride(1), cache.stride(2), cache.stride(3),
            _lib.dtype_code(cache.dtype), b, n, heads, dim, capacity]
    if on_device:
        rc = lib.dx_kv_append_dev(*args, start.data_ptr(), _lib.ptr(status),
                                  _lib.stream_handle(cache.device))
    else:
        rc = lib.dx_kv_append(*args, start, _lib.stream_handle(cache.device))
    _lib.check(rc, "kv_cache_append")
