"""SelfAttention's decode step in one call on gfx950 (HIP ``dx_qk_norm_rope_attention``).

Registered as ``attention/qk_norm_rope_blockwise_causal``. It computes what
``SelfAttention.forward`` does between the projections and the output
projection (``models/dreamzero/model.py:166-182``): ``ops.qk_norm_rope`` of
the pre-norm q and k, with ``append`` the cache write of the rotated k and v
at row ``cache_len`` (``KVCache.append``, ``:53-58``), and
``ops.blockwise_causal_attention`` of the rotated q over the cache's first
``cache_len`` rows and the rotated k, v.

One call instead of three dispatches: the prologue kernel (with the cache
write when appending), then the attention launch. q, k, the cache rows and the
output are the same bits as those ops give.
"""

from __future__ import annotations

import math

import torch

from ...registry import Priority, register
from . import _lib
from ._common import CDNA4, as_rows, strides
from .attention import _check_cache, _starts
from .rope import _accepts as _rope_accepts
from .rope import _prepare, _row_stride


def _accepts(q, k, v, *args, **kwargs) -> bool:
    return (_rope_accepts(q, k) and v.shape == q.shape and v.dtype == q.dtype
            and q.shape[-1] in (64, 128))


@register("attention", "qk_norm_rope_blockwise_causal", name="hip_qk_norm_rope_attention_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts)
def qk_norm_rope_attention(q, k, v, q_weight, k_weight, cos, sin, kv_cache, cache_len, append,
                           block_boundaries, softmax_scale, causal, eps, interleaved):
    if isinstance(cache_len, torch.Tensor):
        raise ValueError("qk_norm_rope_attention takes a host cache_len (a device cursor goes "
                         "through qk_norm_rope_append and blockwise_causal_attention)")
    q, k, qw, kw, c, s, tdt = _prepare(q, k, q_weight, k_weight, cos, sin)
    b, seq, heads, dim = q.shape
    if v.shape != q.shape or v.dtype != q.dtype:
        raise ValueError("v must match q in shape and dtype")
    cache_len = int(cache_len)
    if cache_len < 0:
        raise ValueError("cache_len must be >= 0")
    append = bool(append)
    if (cache_len > 0 or append) and kv_cache is None:
        raise ValueError("cache_len > 0 or append needs kv_cache")
    if kv_cache is not None:
        _check_cache(kv_cache, b, heads, dim, q.dtype, cache_len)
        cache_args = [kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1),
                      kv_cache.stride(2), kv_cache.stride(3), kv_cache.shape[2]]
    else:
        cache_args = [None, 0, 0, 0, 0, 0]
    v = as_rows(v)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(dim)
    q_out = torch.empty((b, seq, heads, dim), device=q.device, dtype=q.dtype)
    k_out = torch.empty_like(q_out)
    out = torch.empty_like(q_out)
    starts, starts_dt, n_blocks = _starts(block_boundaries, seq, q.device)
    lib = _lib.load()
    ws_bytes = lib.dx_attention_workspace_bytes(b, seq, seq, heads, dim, cache_len, None)
    if ws_bytes < 0:
        _lib.check(-ws_bytes, "attention workspace")
    ws = _lib.workspace(q.device, ws_bytes)
    rc = lib.dx_qk_norm_rope_attention(
        q.data_ptr(), *strides(q, 3), k.data_ptr(), *strides(k, 3), v.data_ptr(), *strides(v, 3),
        _lib.dtype_code(q.dtype), qw.data_ptr(), kw.data_ptr(), _lib.dtype_code(qw.dtype),
        c.data_ptr(), _row_stride(c), s.data_ptr(), _row_stride(s), _lib.dtype_code(tdt),
        float(eps), int(bool(interleaved)), q_out.data_ptr(), k_out.data_ptr(),
        *cache_args, cache_len, int(append), out.data_ptr(), *strides(out, 3),
        b, seq, heads, dim, _lib.ptr(starts), starts_dt, n_blocks, int(bool(causal)),
        float(scale), _lib.ptr(ws), ws_bytes, _lib.stream_handle(q.device))
    _lib.check(rc, "qk_norm_rope_attention")
    return out, q_out, k_out
