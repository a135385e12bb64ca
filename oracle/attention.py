"""Torch fp32 restatement of dexter's reference blockwise-causal attention.

Follows ``python/dexter/ops/reference/attention.py``:

* mask (:22-47): ``[q_len, cache_len + q_len]``; the cached history is always
  visible (:31); ``causal`` is token-causal on the current keys (:33-37);
  ``block_boundaries is None`` makes every current key visible (:39-41);
  otherwise each pair ``(lo, hi)`` of consecutive entries of the starts plus a
  final ``q_len`` sets ``mask[lo:hi, cache_len : cache_len + hi]`` (:43-46),
  Python's slice rules included: rows ``[lo:hi]`` of ``q_len``, and current
  keys ``[0, pair_end(hi))``, where a stop ``cache_len + hi`` below zero
  counts from the end of the whole key axis.
* op (:50-77): default scale ``1/sqrt(D)`` (:63); cache rows ``[:cache_len]``
  in front of k/v (:65-67); fp32 logits (:71); ``-inf`` fill (:74); softmax
  then ``@ v`` in fp32 (:76); cast to q's dtype (:77).

Two extensions, where the reference op raises (its mask is
``[q_len, cache_len + q_len]``, :30) but its callers rely on a meaning:

* ``kv_len != q_len`` with no block boundaries and ``causal=False`` is
  cross-attention, every key visible (``models/dreamzero/model.py:237-238``:
  "Conditioning is fully visible: no mask, no cache offset");
* k/v with fewer heads than q (grouped-query attention) read head
  ``h // (H // Hkv)``: the expansion ``repeat_interleave(H // Hkv, dim=2)`` that
  GR00T's backbone applies before calling the op (``vla/groot/backbone.py:109-114``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math

import torch


def visible_end(q_len: int, cache_len: int, block_boundaries, causal: bool = False,
                kv_len: int | None = None) -> torch.Tensor:
    """Per query, one past the last visible key index (int64 ``[q_len]``, CPU).

    Each row of the reference mask is a prefix of the key axis, so it is fully
    described by where the prefix ends. ``kv_len`` (default ``q_len``) is the
    number of current keys; it may differ from ``q_len`` only without a mask.
    """
    kv_len = q_len if kv_len is None else kv_len
    if kv_len != q_len and (causal or block_boundaries is not None):
        raise ValueError(f"kv_len {kv_len} != q_len {q_len} needs no causal or block mask")
    rows = torch.arange(q_len, dtype=torch.int64)
    if causal:
        return cache_len + rows + 1
    if block_boundaries is None:
        return torch.full((q_len,), cache_len + kv_len, dtype=torch.int64)
    bounds = [int(x) for x in torch.as_tensor(block_boundaries).reshape(-1).tolist()] + [q_len]
    end = torch.zeros(q_len, dtype=torch.int64)
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        # Python slicing, as the reference's mask[lo:hi, ...] uses.
        seg = end[lo:hi]
        end[lo:hi] = torch.clamp(seg, min=pair_end(hi, cache_len, q_len))
    return cache_len + end


def pair_end(hi: int, cache_len: int, q_len: int) -> int:
    """Current keys ``[0, e)`` that the reference's column slice
    ``mask[..., cache_len : cache_len + hi]`` sets on a ``cache_len + q_len``
    key axis (``ops/reference/attention.py:45``), by Python's slice rules.

    ``hi >= 0``: the stop clamps at the axis end, ``e = min(hi, q_len)``.
    ``-cache_len <= hi < 0``: the stop lies before the start, nothing.
    ``hi < -cache_len``: the negative stop counts from the axis end,
    ``cache_len + q_len + hi`` in absolute columns, so the current keys up to
    ``cache_len + q_len + hi`` (at least 0) are set.
    """
    if hi >= 0:
        return min(hi, q_len)
    return max(cache_len + q_len + hi, 0) if cache_len + hi < 0 else 0


def block_causal_mask(q_len: int, cache_len: int, block_boundaries, device=None,
                      causal: bool = False, kv_len: int | None = None) -> torch.Tensor:
    """Bool ``[q_len, cache_len + kv_len]`` (``kv_len`` defaults to ``q_len``); True = may attend."""
    kv_len = q_len if kv_len is None else kv_len
    ends = visible_end(q_len, cache_len, block_boundaries, causal, kv_len)
    cols = torch.arange(cache_len + kv_len, dtype=torch.int64)
    mask = cols[None, :] < ends[:, None]
    return mask if device is None else mask.to(device)


def blockwise_causal_attention(q, k, v, kv_cache=None, cache_len: int = 0,
                               block_boundaries=None, softmax_scale=None, causal=False,
                               keep_fp32: bool = False) -> torch.Tensor:
    """q ``[B, Lq, H, D]``, k/v ``[B, Lk, Hkv, D]``; kv_cache ``[2, B, S, Hkv, D]``.
    CPU, fp32 math.

    Returns q's dtype like the reference, or the fp32 result before that cast
    when ``keep_fp32`` (the tolerance checks compare against this).
    """
    b, q_len, h, d = q.shape
    kv_len, h_kv = k.shape[1], k.shape[2]
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    keys, vals = k, v
    if kv_cache is not None and cache_len > 0:
        keys = torch.cat((kv_cache[0, :, :cache_len].to(k.device), k), dim=1)
        vals = torch.cat((kv_cache[1, :, :cache_len].to(v.device), v), dim=1)
    if h_kv != h:
        if h % h_kv:
            raise ValueError(f"{h} query heads are not a multiple of {h_kv} k/v heads")
        keys = keys.repeat_interleave(h // h_kv, dim=2)
        vals = vals.repeat_interleave(h // h_kv, dim=2)
    # Contiguous operands: batched products on transposed views are avoided.
    qf = q.float().permute(0, 2, 1, 3).contiguous()         # [B, H, Lq, D]
    kf = keys.float().permute(0, 2, 3, 1).contiguous()      # [B, H, D, Lk]
    vf = vals.float().permute(0, 2, 1, 3).contiguous()      # [B, H, Lk, D]
    logits = torch.matmul(qf, kf) * scale
    mask = block_causal_mask(q_len, cache_len, block_boundaries, logits.device, causal, kv_len)
    logits = logits.masked_fill(~mask, float("-inf"))
    out = torch.matmul(torch.softmax(logits, dim=-1).contiguous(), vf).permute(0, 2, 1, 3)
    return out if keep_fp32 else out.to(q.dtype)
