"""fp64 brute force of the path, independent of the torch restatements.

Written from the definitions, not from the torch code: attention is an
explicit loop over (batch, head, query) with a stable softmax over exactly
the visible keys (decided per key by the rule of
``ops/reference/attention.py:22-47``); the prologue is numpy float64 with no
intermediate rounding (the reference's bf16 rounding after the norm,
``ops/reference/rope.py:40``, is applied only when ``round_to`` is given).
Meant for small inputs (config C0 and the like): it is slow on purpose.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math

import numpy as np


def key_visible(i: int, j: int, q_len: int, cache_len: int, starts, causal: bool) -> bool:
    """Whether query ``i`` may attend to key ``j`` (key 0 = first cached row).

    Block pairs follow the reference's ``mask[lo:hi, cache_len:cache_len + hi]``
    (``ops/reference/attention.py:43-46``) through membership in sliced
    ``range`` objects, which apply Python's slice rules (negative bounds count
    from the end, out-of-range bounds clamp) without restating them.
    """
    if j < cache_len:
        return True
    jj = j - cache_len
    if causal:
        return jj <= i
    if starts is None:
        return True
    bounds = list(starts) + [q_len]
    rows, cols = range(q_len), range(cache_len + q_len)
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        if i in rows[lo:hi] and j in cols[cache_len:cache_len + hi]:
            return True
    return False


def slice_mask(q_len: int, cache_len: int, starts, causal: bool = False):
    """The reference's mask as nested Python lists of bools, built with real
    slice assignment on each row list, step by step as
    ``ops/reference/attention.py:30-46`` builds its tensor."""
    n = cache_len + q_len
    mask = [[False] * n for _ in range(q_len)]
    for row in mask:
        row[:cache_len] = [True] * len(row[:cache_len])
    if causal:
        for r, row in enumerate(mask):
            for c in range(q_len):
                row[cache_len + c] = c <= r
        return mask
    if starts is None:
        for row in mask:
            row[cache_len:] = [True] * len(row[cache_len:])
        return mask
    bounds = list(starts) + [q_len]
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        for row in mask[lo:hi]:
            seg = row[cache_len:cache_len + hi]
            row[cache_len:cache_len + hi] = [True] * len(seg)
    return mask


def attention(q, k, v, cache_k=None, cache_v=None, cache_len=0, starts=None,
              causal=False, scale=None):
    """q ``[B, Lq, H, D]``, k/v ``[B, Lk, Hkv, D]``; cache_k/v ``[B, S, Hkv, D]``.
    Returns fp64 ``[B, Lq, H, D]``.

    A query with no visible key gives NaN (0/0), as a softmax over nothing.
    With ``Hkv < H`` query head ``hh`` reads k/v head ``hh // (H // Hkv)``.
    ``Lk != Lq`` is meant without a mask (every key visible).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, q_len, h, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if cache_len > 0:
        keys = np.concatenate([np.asarray(cache_k, np.float64)[:, :cache_len], k], axis=1)
        vals = np.concatenate([np.asarray(cache_v, np.float64)[:, :cache_len], v], axis=1)
    else:
        keys, vals = k, v
    n_keys = keys.shape[1]
    group = h // keys.shape[2]  # query heads per k/v head
    out = np.empty((b, q_len, h, d), dtype=np.float64)
    for i in range(q_len):
        vis = np.array([key_visible(i, j, q_len, cache_len, starts, causal) for j in range(n_keys)],
                       dtype=bool)
        for bb in range(b):
            for hh in range(h):
                if not vis.any():
                    out[bb, i, hh] = np.nan
                    continue
                kh = hh // group
                s = keys[bb, vis, kh] @ q[bb, i, hh] * scale
                w = np.exp(s - s.max())
                out[bb, i, hh] = (w[:, None] * vals[bb, vis, kh]).sum(0) / w.sum()
    return out


def qk_norm_rope(x, weight, cos, sin, eps=1e-6, interleaved=True, round_to=None):
    """One tensor ``[B, L, H, D]`` through plane-RMSNorm then rotary, in fp64.

    ``round_to`` (a callable float64 -> float64) models the reference's cast
    to the input dtype between norm and rotation.
    """
    x = np.asarray(x, dtype=np.float64)
    b, seq, h, d = x.shape
    plane = x.reshape(b, seq, h * d)
    rms = np.sqrt((plane ** 2).mean(-1, keepdims=True) + eps)
    y = (plane / rms * np.asarray(weight, np.float64).reshape(1, 1, -1)).reshape(b, seq, h, d)
    if round_to is not None:
        y = round_to(y)
    c = np.asarray(cos, np.float64)[None, :, None, :]
    s = np.asarray(sin, np.float64)[None, :, None, :]
    out = np.empty_like(y)
    if interleaved:
        lo, hi = y[..., 0::2], y[..., 1::2]
        out[..., 0::2] = lo * c - hi * s
        out[..., 1::2] = lo * s + hi * c
    else:
        half = d // 2
        lo, hi = y[..., :half], y[..., half:]
        out[..., :half] = lo * c - hi * s
        out[..., half:] = lo * s + hi * c
    return out


def adaln_modulate(x, scale, shift, eps=1e-6, round_to=None):
    """LayerNorm (no affine) of each row of ``x [..., C]`` then ``* (1 + scale) + shift``,
    in fp64 with explicit per-row loops.

    LayerNorm here is the textbook one: the row mean, the biased variance
    (divide by C), and ``(x - mean) / sqrt(var + eps)``. ``scale``/``shift``
    broadcast against ``x`` as numpy arrays do. ``round_to`` (a callable
    float64 -> float64) models the reference's rounding after each op:
    after the norm, after ``1 + scale``, after the product and after the sum.
    """
    x = np.asarray(x, dtype=np.float64)
    scale = np.asarray(scale, dtype=np.float64)
    shift = np.asarray(shift, dtype=np.float64)
    shape = np.broadcast_shapes(x.shape, scale.shape, shift.shape)
    rows = x.reshape(-1, x.shape[-1])
    normed = np.empty_like(rows)
    for r in range(rows.shape[0]):
        row = rows[r]
        n = row.shape[0]
        mean = sum(float(v) for v in row) / n
        var = sum((float(v) - mean) ** 2 for v in row) / n
        normed[r] = (row - mean) / math.sqrt(var + eps)
    normed = normed.reshape(x.shape)
    rnd = round_to if round_to is not None else (lambda a: a)
    gain = rnd(1.0 + scale)
    prod = rnd(np.broadcast_to(rnd(normed), shape) * gain)
    return rnd(prod + shift)


def gated_residual(x, y, gate, round_to=None):
    """``x + y * gate`` in fp64; ``round_to`` rounds the product and the sum."""
    x, y, gate = (np.asarray(t, dtype=np.float64) for t in (x, y, gate))
    rnd = round_to if round_to is not None else (lambda a: a)
    return rnd(x + rnd(y * gate))
