"""Blockwise-causal flash attention on gfx950 (HIP kernel ``dx_blockwise_causal_attention``).

Registered as ``attention/blockwise_causal`` with the signature of dexter's
implementations (``ops/reference/attention.py:50-77``,
``ops/gfx1151/attention/blockwise_causal.py:146-173``):
``(q, k, v, kv_cache, cache_len, block_boundaries, softmax_scale, causal=False)``.

Differences from the Triton wrapper it replaces, none visible in results:

* The cached history is read where it lies: no ``torch.cat`` of
  ``kv_cache[:, :, :cache_len]`` with ``k``/``v`` per call
  (``blockwise_causal.py:153-156``); the kernel takes the cache and the new
  keys as two sources of one key sequence.
* Visibility limits are derived on the device from ``block_boundaries`` by the
  kernel itself (no ``searchsorted`` launches, no host sync).
* Whole key tiles past a workgroup's last visible key are never loaded.

Semantics follow the torch reference op (the correctness oracle): a query with
no visible key gives NaN (the reference's softmax of an all ``-inf`` row);
``block_boundaries`` rows before the first start see only the cache.

Two cases the reference op cannot take are defined as its callers use them:

* **Cross-attention.** ``k``/``v`` longer or shorter than ``q`` with no block
  boundaries and ``causal=False``: every key is visible. ``CrossAttention``
  calls the op so for the text and image conditioning
  (``models/dreamzero/model.py:234-241``); the reference's mask is
  ``[q_len, cache_len + q_len]`` (``ops/reference/attention.py:30``) and the
  Triton limits ignore keys past ``q_len`` (``blockwise_causal.py:134-135``).
* **Grouped-query attention.** ``k``/``v`` (and the cache) with ``Hkv`` heads,
  ``H`` a multiple of ``Hkv``: query head ``h`` reads K/V head ``h // (H // Hkv)``,
  what ``repeat_interleave(H // Hkv, dim=2)`` gives
  (``vla/groot/backbone.py:109-114``), without materialising the copy.

Inputs in bf16 or f16 at head dim 64 or 128 run on the bf16/f16 MFMA kernels;
fp32 inputs (any supported head dim) and bf16/f16 at head dims 16, 32 and 256
run on the general kernel (fp32 MFMA, fp32 softmax; ``csrc/attn_any.hip``), as
the reference op is dtype-generic (``ops/reference/attention.py:62-77``) and
the Triton kernel takes any power-of-two head dim
(``blockwise_causal.py:162-172``).

``cache_len`` may be a device cursor (one int32 on the device,
``dx_blockwise_causal_attention_dev``): the kernels read the cached row count
when they run, clamped to the cache capacity, and the launch is planned for the
whole capacity. A graph captured once then stays correct as the cache grows.
"""

from __future__ import annotations

import math

import torch

from ...registry import Priority, register
from . import _lib
from ._common import CDNA4, as_rows, device_cursor, strides

# Input dtypes and head dims the kernels are built for (the C ABI's own checks).
ATTN_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
ATTN_HEAD_DIMS = (16, 32, 64, 128, 256)


def _accepts(q, k, v, *args, **kwargs) -> bool:
    return (q.is_cuda and q.dtype in ATTN_DTYPES and q.dim() == 4
            and k.dtype == q.dtype and v.dtype == q.dtype
            and k.shape == v.shape and k.dim() == 4
            and q.shape[-1] in ATTN_HEAD_DIMS and k.shape[-1] == q.shape[-1]
            and k.shape[2] > 0 and q.shape[2] % k.shape[2] == 0)


def _starts(block_boundaries, q_len: int, device: torch.device):
    """(tensor, dtype code, count) of block starts on the device."""
    if block_boundaries is None:
        return None, _lib.DX_I32, 0
    bb = block_boundaries.reshape(-1)
    if bb.numel() == 0:
        # No block at all: no current key is visible to any query (the
        # reference's loop over an empty start list sets nothing).
        bb = torch.full((1,), q_len, dtype=torch.int32, device=device)
    if bb.device != device:
        bb = bb.to(device)
    if bb.dtype not in (torch.int32, torch.int64):
        bb = bb.to(torch.int64)
    return bb.contiguous(), _lib.dtype_code(bb.dtype), bb.numel()


def _check_cache(kv_cache, b, heads, dim, dtype, need_rows: int):
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2 or kv_cache.shape[1] != b \
            or tuple(kv_cache.shape[3:]) != (heads, dim):
        raise ValueError(f"kv_cache must be [2, {b}, S, {heads}, {dim}], got {tuple(kv_cache.shape)}")
    if kv_cache.dtype != dtype:
        raise ValueError(f"kv_cache dtype {kv_cache.dtype} differs from q's {dtype}")
    if kv_cache.shape[2] < need_rows:
        raise ValueError(f"cache_len {need_rows} exceeds the cache capacity {kv_cache.shape[2]}")
    per16 = 16 // kv_cache.element_size()
    if not (kv_cache.stride(-1) == 1 and kv_cache.data_ptr() % 16 == 0
            and all(x % per16 == 0 for x in kv_cache.stride()[:-1])):
        raise ValueError("kv_cache must have a contiguous, 16-byte aligned head_dim")


def _launch(q, k, v, kv_cache, cache_len, cache_lens, block_boundaries, softmax_scale,
            causal, cursor=None):
    if q.dim() != 4 or k.shape != v.shape or k.dim() != 4:
        raise ValueError("q, k, v must be [B, L, H, D] with k and v of one shape")
    b, q_len, heads, dim = q.shape
    kv_len, kv_heads = k.shape[1], k.shape[2]
    if k.shape[0] != b or k.shape[3] != dim or kv_heads == 0 or heads % kv_heads:
        raise ValueError(f"k/v {tuple(k.shape)} do not match q {tuple(q.shape)} (the k/v heads "
                         "must divide the query heads)")
    if kv_len != q_len and (block_boundaries is not None or causal):
        raise ValueError(
            f"k/v length {kv_len} must equal q length {q_len} with block_boundaries or causal: "
            f"the block mask is [q_len, cache_len + q_len] (ops/reference/attention.py:30)")
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(dim)
    q, k, v = as_rows(q), as_rows(k), as_rows(v)
    if cursor is not None:
        if kv_cache is None:
            raise ValueError("a device cache_len needs kv_cache")
        cursor = device_cursor(cursor, q.device, "blockwise_causal_attention cache_len")
        cache_len = kv_cache.shape[2]  # planned for the capacity; the kernel clamps the cursor
    max_cache = max(cache_lens) if cache_lens is not None else cache_len
    if max_cache > 0:
        if kv_cache is None:
            raise ValueError("cache_len > 0 needs kv_cache")
        _check_cache(kv_cache, b, kv_heads, dim, q.dtype, max_cache)
        cache_ptr = kv_cache.data_ptr()
        c_strides = [kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2),
                     kv_cache.stride(3)]
    else:
        cache_ptr, c_strides = None, [0, 0, 0, 0]
    out = torch.empty((b, q_len, heads, dim), device=q.device, dtype=q.dtype)
    starts, starts_dt, n_blocks = _starts(block_boundaries, q_len, q.device)
    lib = _lib.load()
    arr = None
    if cache_lens is not None:
        arr = (_lib.ctypes.c_int64 * b)(*[int(x) for x in cache_lens])
    if kv_len == 0 and max_cache == 0 and q_len > 0:
        raise ValueError("attention over no keys: k/v are empty and there is no cache")
    ws_bytes = lib.dx_attention_workspace_bytes(b, q_len, kv_len, heads, dim, int(cache_len), arr)
    if ws_bytes < 0:
        _lib.check(-ws_bytes, "attention workspace")
    ws = _lib.workspace(q.device, ws_bytes)
    common = [
        q.data_ptr(), *strides(q, 3), k.data_ptr(), *strides(k, 3), v.data_ptr(), *strides(v, 3),
        cache_ptr, *c_strides, out.data_ptr(), *strides(out, 3),
        _lib.dtype_code(q.dtype), b, q_len, kv_len, heads, kv_heads, dim,
    ]
    tail = [_lib.ptr(starts), starts_dt, n_blocks, int(bool(causal)), float(scale),
            _lib.ptr(ws), ws_bytes, _lib.stream_handle(q.device)]
    if cursor is not None:
        rc = lib.dx_blockwise_causal_attention_dev(*common, cursor.data_ptr(), int(cache_len),
                                                   *tail)
    elif cache_lens is None:
        rc = lib.dx_blockwise_causal_attention(*common, int(cache_len), *tail)
    else:
        rc = lib.dx_blockwise_causal_attention_varlen(*common, arr, *tail)
    _lib.check(rc, "blockwise_causal_attention")
    return out


@register("attention", "blockwise_causal", name="hip_blockwise_causal_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts)
def blockwise_causal_attention(q, k, v, kv_cache, cache_len, block_boundaries,
                               softmax_scale, causal=False):
    if isinstance(cache_len, torch.Tensor):
        return _launch(q, k, v, kv_cache, 0, None, block_boundaries, softmax_scale, causal,
                       cursor=cache_len)
    cache_len = int(cache_len)
    if cache_len < 0:
        raise ValueError("cache_len must be >= 0")
    if kv_cache is None:
        # The reference concatenates nothing without a cache; a positive
        # cache_len then only widens its mask, which cannot broadcast (raises).
        if cache_len > 0:
            raise ValueError("cache_len > 0 needs kv_cache")
    return _launch(q, k, v, kv_cache, cache_len, None, block_boundaries, softmax_scale, causal)


@register("attention", "blockwise_causal_varlen", name="hip_blockwise_causal_varlen_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts)
def blockwise_causal_attention_varlen(q, k, v, kv_cache, cache_lens, block_boundaries,
                                      softmax_scale, causal=False):
    cache_lens = [int(x) for x in cache_lens]
    if len(cache_lens) != q.shape[0]:
        raise ValueError(f"{len(cache_lens)} cache lengths for a batch of {q.shape[0]}")
    if any(x < 0 for x in cache_lens):
        raise ValueError("cache lengths must be >= 0")
    if len(cache_lens) > 64:
        raise ValueError("varlen attention takes at most 64 sequences per call")
    return _launch(q, k, v, kv_cache, 0, cache_lens, block_boundaries, softmax_scale, causal)
