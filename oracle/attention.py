"""Torch fp32 restatement of dexter's reference blockwise-causal attention.

Follows ``python/dexter/ops/reference/attention.py``:

* mask (:22-47): ``[q_len, cache_len + q_len]``; the cached history is always
  visible (:31); ``causal`` is token-causal on the current keys (:33-37);
  ``block_boundaries is None`` makes every current key visible (:39-41);
  otherwise block ``[lo, hi)`` (starts plus a final ``q_len``) sees current
  keys ``[0, hi)`` (:43-46).
* op (:50-77): default scale ``1/sqrt(D)`` (:63); cache rows ``[:cache_len]``
  in front of k/v (:65-67); fp32 logits (:71); ``-inf`` fill (:74); softmax
  then ``@ v`` in fp32 (:76); cast to q's dtype (:77).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math

import torch


def visible_end(q_len: int, cache_len: int, block_boundaries, causal: bool = False) -> torch.Tensor:
    """Per query, one past the last visible key index (int64 ``[q_len]``, CPU).

    Each row of the reference mask is a prefix of the key axis, so it is fully
    described by where the prefix ends.
    """
    rows = torch.arange(q_len, dtype=torch.int64)
    if causal:
        return cache_len + rows + 1
    if block_boundaries is None:
        return torch.full((q_len,), cache_len + q_len, dtype=torch.int64)
    bounds = [int(x) for x in torch.as_tensor(block_boundaries).reshape(-1).tolist()] + [q_len]
    end = torch.zeros(q_len, dtype=torch.int64)
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        # Python slicing, as the reference's mask[lo:hi, ...] uses.
        seg = end[lo:hi]
        end[lo:hi] = torch.clamp(seg, min=min(hi, q_len))
    return cache_len + end


def block_causal_mask(q_len: int, cache_len: int, block_boundaries, device=None,
                      causal: bool = False) -> torch.Tensor:
    """Bool ``[q_len, cache_len + q_len]``; True = may attend."""
    ends = visible_end(q_len, cache_len, block_boundaries, causal)
    cols = torch.arange(cache_len + q_len, dtype=torch.int64)
    mask = cols[None, :] < ends[:, None]
    return mask if device is None else mask.to(device)


def blockwise_causal_attention(q, k, v, kv_cache=None, cache_len: int = 0,
                               block_boundaries=None, softmax_scale=None, causal=False,
                               keep_fp32: bool = False) -> torch.Tensor:
    """q, k, v ``[B, L, H, D]``; kv_cache ``[2, B, S, H, D]``. CPU, fp32 math.

    Returns q's dtype like the reference, or the fp32 result before that cast
    when ``keep_fp32`` (the tolerance checks compare against this).
    """
    b, q_len, h, d = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    keys, vals = k, v
    if kv_cache is not None and cache_len > 0:
        keys = torch.cat((kv_cache[0, :, :cache_len].to(k.device), k), dim=1)
        vals = torch.cat((kv_cache[1, :, :cache_len].to(v.device), v), dim=1)
    # Contiguous operands: batched products on transposed views are avoided.
    qf = q.float().permute(0, 2, 1, 3).contiguous()         # [B, H, Lq, D]
    kf = keys.float().permute(0, 2, 3, 1).contiguous()      # [B, H, D, Lk]
    vf = vals.float().permute(0, 2, 1, 3).contiguous()      # [B, H, Lk, D]
    logits = torch.matmul(qf, kf) * scale
    mask = block_causal_mask(q_len, cache_len, block_boundaries, logits.device, causal)
    logits = logits.masked_fill(~mask, float("-inf"))
    out = torch.matmul(torch.softmax(logits, dim=-1).contiguous(), vf).permute(0, 2, 1, 3)
    return out if keep_fp32 else out.to(q.dtype)
