"""QKV projection fused with the QK-norm + rotary prologue (HIP ``dx_qkv_norm_rope``).

Registered as ``rope/qkv_norm_rope``: one call does what
``SelfAttention.forward`` (``models/dreamzero/model.py:162-175``) does with
three ``nn.Linear`` projections, ``ops.qk_norm_rope`` and ``KVCache.append``:

    q, k, v = x wq^T + bq, x wk^T + bk, x wv^T + bv      (rounded to x's dtype)
    q, k = qk_norm_rope(q, k, ...)                       (the prologue, bit for bit)
    cache[:, :, start:start+L] = (k, v)                  (when a cache is given)

For decode chunks (at most 128 tokens) the projection is a weight stream:
at the Wan-5B chunk the three weights are 57 MB against 0.5 MB of
activations. The HIP path is a split-K MFMA GEMM that reads each weight byte
once from every CU, then the prologue kernel summing its fp32 partials, so
the q/k/v projections never make a bf16 round trip through HBM before the
norm. ``start`` may be a device cursor, as for ``qk_norm_rope_append``.
"""

from __future__ import annotations

import torch

from ...registry import Priority, register
from . import _lib
from ._common import CDNA4, MATRIX_DTYPES, device_cursor, rows_ok

_TABLE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
MAX_TOKENS = 128


def _weight_ok(w, hd, c, dtype) -> bool:
    return (w.dim() == 2 and tuple(w.shape) == (hd, c) and w.dtype == dtype and w.is_cuda
            and w.stride(1) == 1 and w.data_ptr() % 16 == 0 and w.stride(0) % 8 == 0)


def _accepts(x, wq, bq, wk, bk, wv, bv, q_weight, k_weight, cos, sin, heads, *args,
             **kwargs) -> bool:
    if not (x.is_cuda and x.dtype in MATRIX_DTYPES and x.dim() == 3):
        return False
    b, seq, c = x.shape
    hd = wq.shape[0] if wq.dim() == 2 else -1
    return (0 < b * seq <= MAX_TOKENS and c % 512 == 0 and hd % 128 == 0 and hd <= 8192
            and hd % heads == 0 and (hd // heads) % 16 == 0
            and all(_weight_ok(w, hd, c, x.dtype) for w in (wq, wk, wv))
            and wq.stride(0) == wk.stride(0) == wv.stride(0))


def _bias(t, hd, dtype, device):
    if t is None:
        return None
    if t.numel() != hd:
        raise ValueError(f"bias must have {hd} elements, got {t.numel()}")
    return t.reshape(-1).to(device=device, dtype=dtype).contiguous()


@register("rope", "qkv_norm_rope", name="hip_qkv_norm_rope_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts)
def qkv_norm_rope(x, wq, bq, wk, bk, wv, bv, q_weight, k_weight, cos, sin, heads, eps,
                  interleaved=True, cache=None, start=0, status=None):
    b, seq, c = x.shape
    hd = wq.shape[0]
    dim = hd // heads
    if not rows_ok(x):
        x = x.contiguous()
    wdt = q_weight.dtype if q_weight.dtype in _TABLE_DTYPES else torch.float32
    qw = q_weight.reshape(-1).to(device=x.device, dtype=wdt).contiguous()
    kw = k_weight.reshape(-1).to(device=x.device, dtype=wdt).contiguous()
    if qw.numel() != hd or kw.numel() != hd:
        raise ValueError(f"norm weights must have H*D = {hd} elements")
    tdt = cos.dtype if cos.dtype in _TABLE_DTYPES else torch.float32
    tables = []
    for t in (cos, sin):
        if t.dim() != 2 or t.shape[-1] != dim // 2 or t.shape[0] not in (seq, 1):
            raise ValueError(f"cos/sin must be [L, D/2] = [{seq}, {dim // 2}], got {tuple(t.shape)}")
        t = t.to(device=x.device, dtype=tdt)
        tables.append(t if rows_ok(t) else t.contiguous())
    cs, sn = tables
    biases = [_bias(t, hd, x.dtype, x.device) for t in (bq, bk, bv)]
    q_out = torch.empty((b, seq, heads, dim), device=x.device, dtype=x.dtype)
    k_out = torch.empty_like(q_out)
    v_out = torch.empty_like(q_out)
    lib = _lib.load()
    ws_n = lib.dx_qkv_workspace_bytes(b, seq, c, heads, dim)
    if ws_n < 0:
        _lib.check(-ws_n, "qkv_norm_rope workspace")
    ws = torch.empty(max(ws_n, 16), dtype=torch.uint8, device=x.device)
    cache_args = [None, 0, 0, 0, 0, 0, 0, None, None]
    if cache is not None:
        if cache.dim() != 5 or cache.shape[0] != 2 or cache.shape[1] != b \
                or tuple(cache.shape[3:]) != (heads, dim) or cache.dtype != x.dtype:
            raise ValueError(f"cache must be [2, {b}, S, {heads}, {dim}] of {x.dtype}, "
                             f"got {tuple(cache.shape)} {cache.dtype}")
        if not (cache.stride(-1) == 1 and cache.data_ptr() % 16 == 0
                and all(s % 8 == 0 for s in cache.stride()[:-1])):
            raise ValueError("cache must have a contiguous, 16-byte aligned head_dim")
        dev_start = None
        if isinstance(start, torch.Tensor):
            dev_start = device_cursor(start, x.device, "qkv_norm_rope")
            if status is not None:
                status = device_cursor(status, x.device, "qkv_norm_rope status")
            start = 0
        cache_args = [cache.data_ptr(), *cache.stride()[:4], cache.shape[2], int(start),
                      _lib.ptr(dev_start), _lib.ptr(status)]
    rc = lib.dx_qkv_norm_rope(
        x.data_ptr(), x.stride(0), x.stride(1), _lib.dtype_code(x.dtype),
        wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), wq.stride(0),
        *[_lib.ptr(t) for t in biases],
        qw.data_ptr(), kw.data_ptr(), _lib.dtype_code(wdt),
        cs.data_ptr(), 0 if cs.shape[0] == 1 else cs.stride(0),
        sn.data_ptr(), 0 if sn.shape[0] == 1 else sn.stride(0), _lib.dtype_code(tdt),
        q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(),
        *cache_args, b, seq, c, heads, dim, float(eps), int(bool(interleaved)),
        ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device))
    _lib.check(rc, "qkv_norm_rope")
    return q_out, k_out, v_out
