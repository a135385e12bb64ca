"""Public op surface for the blockwise-causal attention path.

Each function asks the registry for the best implementation on this platform
and calls it, exactly as dexter's dispatchers do (``python/dexter/ops/__init__.py``):

* ``qk_norm_rope``               -> ``select("rope", "qk_norm_rope", q, k)``
  (reference ``ops/__init__.py:66-86``; same arguments and defaults)
* ``blockwise_causal_attention`` -> ``select("attention", "blockwise_causal", q, k, v)``
  (reference ``ops/__init__.py:127-147``; same keyword-only arguments)
* ``kv_cache_append``            -> ``select("cache", "append", cache, k, v)``
  (no dispatcher in the reference: ``KVCache.append`` does two torch slice
  copies, ``models/dreamzero/model.py:53-58``; here it is a kernel too)
* ``qkv_norm_rope``              -> ``select("rope", "qkv_norm_rope", x, wq, ...)``
  (no dispatcher in the reference: ``SelfAttention.forward`` runs three
  ``nn.Linear`` and ``ops.qk_norm_rope``, ``models/dreamzero/model.py:162-175``;
  here one call for decode chunks)
* ``qk_norm_rope_attention``     -> ``select("attention", "qk_norm_rope_blockwise_causal", q, k, v)``
  (no dispatcher in the reference: ``SelfAttention.forward`` calls
  ``ops.qk_norm_rope``, ``KVCache.append`` and ``ops.blockwise_causal_attention``,
  ``models/dreamzero/model.py:166-182``; here one call)
* ``adaln_modulate``             -> ``select("norm", "adaln", x, scale, shift)``
  (reference ``ops/__init__.py:39-49``; same arguments and default eps)
* ``gated_residual``             -> ``select("norm", "gated_residual", x, y, gate)``
  (reference ``ops/__init__.py:52-54``)

Importing this module registers the gfx950 HIP kernels. Nothing else is
registered, so on a machine without an MI355X every call raises
``LookupError`` rather than running a slower stand-in.
"""

from __future__ import annotations

import torch

from ..registry import select

__all__ = ["qk_norm_rope", "blockwise_causal_attention", "kv_cache_append",
           "qk_norm_rope_append", "blockwise_causal_attention_varlen",
           "adaln_modulate", "gated_residual", "qkv_norm_rope", "qk_norm_rope_attention"]


def qkv_norm_rope(
    x: torch.Tensor,
    wq: torch.Tensor, bq: torch.Tensor | None,
    wk: torch.Tensor, bk: torch.Tensor | None,
    wv: torch.Tensor, bv: torch.Tensor | None,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float = 1e-6,
    interleaved: bool = True,
    cache: torch.Tensor | None = None,
    start: int | torch.Tensor = 0,
    status: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The q/k/v projections of a ``[B, L, C]`` chunk, QK-norm + rotary, and the cache write.

    Equals ``q, k, v = F.linear(x, wq, bq), F.linear(x, wk, bk), F.linear(x, wv, bv)``
    viewed as ``[B, L, heads, D]``, then ``qk_norm_rope(q, k, ...)``, and, with a
    ``cache``, ``kv_cache_append(cache, k_rotated, v, start, status)``. Returns the
    rotated ``q``, ``k`` and the projected ``v``.
    """
    return select("rope", "qkv_norm_rope", x, wq, bq, wk, bk, wv, bv, q_weight, k_weight, cos,
                  sin, heads)(x, wq, bq, wk, bk, wv, bv, q_weight, k_weight, cos, sin, heads,
                              eps, interleaved, cache, start, status)


def adaln_modulate(
    x: torch.Tensor,
    scale: torch.Tensor,
    shift: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Modulated LayerNorm of the DiT block: normalise each ``C``-row of ``x`` (no
    affine), multiply by ``1 + scale`` and add ``shift``; one kernel, one read of ``x``.

    ``x`` is ``[B, L, C]``. ``scale`` and ``shift`` broadcast against it: per row
    (``[B, L, C]``), per batch (``[B, 1, C]``, the Wan block's modulation) or one
    row for all (``[C]``). The result has torch's promoted dtype.
    """
    return select("norm", "adaln", x, scale, shift)(x, scale, shift, eps)


def gated_residual(x: torch.Tensor, y: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Residual add with a gate, ``x + y * gate``: the attention or FFN branch ``y``
    scaled by its per-channel gate and added to the stream ``x`` in one pass
    (``gate`` broadcasts like ``adaln_modulate``'s modulation)."""
    return select("norm", "gated_residual", x, y, gate)(x, y, gate)


def qk_norm_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float = 1e-6,
    interleaved: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm over the whole ``H*D`` plane of each token, then rotary, for q and k.

    ``q``/``k`` are ``[B, L, H, D]``; the weights are ``[H*D]``; ``cos``/``sin``
    are ``[L, D//2]``. ``interleaved`` pairs ``(2j, 2j+1)`` (Wan); otherwise
    ``(j, j + D/2)``. Returns new ``(q, k)`` tensors of the input dtype.
    """
    return select("rope", "qk_norm_rope", q, k)(
        q, k, q_weight, k_weight, cos, sin, eps, interleaved)


def blockwise_causal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    kv_cache: torch.Tensor | None = None,
    cache_len: int | torch.Tensor = 0,
    block_boundaries: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    causal: bool = False,
) -> torch.Tensor:
    """Softmax attention of ``q`` over ``[cache[:cache_len] | k]`` with block causality.

    A query in the block starting at ``block_boundaries[i]`` sees the whole
    cached history and every current key before the end of its own block.
    ``None`` is one block (all current keys visible); ``causal=True`` is
    token-causal on the current keys. ``kv_cache`` is ``[2, B, S, H, D]``;
    rows ``[0, cache_len)`` are read in place, never copied. ``cache_len`` may
    be a device cursor (a one-element int32 tensor) that the kernels read when
    they run, so a captured graph follows a growing cache. ``k``/``v`` of
    another length than ``q`` (no mask) is cross-attention; ``k``/``v`` with
    fewer heads is grouped-query attention.
    """
    return select("attention", "blockwise_causal", q, k, v)(
        q, k, v, kv_cache, cache_len, block_boundaries, softmax_scale, causal)


def qk_norm_rope_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    kv_cache: torch.Tensor | None = None,
    cache_len: int = 0,
    append: bool = False,
    block_boundaries: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    causal: bool = False,
    eps: float = 1e-6,
    interleaved: bool = True,
    return_qk: bool = False,
):
    """``qk_norm_rope``, the cache write of the rotated k and v (``append``), and
    ``blockwise_causal_attention``, as ``SelfAttention.forward`` chains them.

    Same results as ``qr, kr = qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps,
    interleaved)``, then (with ``append``) ``kv_cache_append(kv_cache, kr, v, cache_len)``,
    then ``blockwise_causal_attention(qr, kr, v, kv_cache=kv_cache, cache_len=cache_len,
    ...)``. Returns the attention output, and with ``return_qk`` also ``qr`` and ``kr``.
    ``cache_len`` is the row count before the append (the model reads it first).
    """
    out, qr, kr = select("attention", "qk_norm_rope_blockwise_causal", q, k, v)(
        q, k, v, q_weight, k_weight, cos, sin, kv_cache, cache_len, append, block_boundaries,
        softmax_scale, causal, eps, interleaved)
    return (out, qr, kr) if return_qk else out


def blockwise_causal_attention_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    kv_cache: torch.Tensor,
    cache_lens: list[int],
    block_boundaries: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    causal: bool = False,
) -> torch.Tensor:
    """``blockwise_causal_attention`` over a ragged batch in one launch.

    Sequence ``b`` attends to ``kv_cache[:, b, :cache_lens[b]]`` followed by
    its own ``k``/``v`` rows; results equal one ``blockwise_causal_attention``
    call per sequence with ``cache_len=cache_lens[b]``. (The reference takes a
    scalar ``cache_len`` only, so a ragged batch there is a loop of calls.)
    """
    return select("attention", "blockwise_causal_varlen", q, k, v)(
        q, k, v, kv_cache, cache_lens, block_boundaries, softmax_scale, causal)


def kv_cache_append(cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    start: int | torch.Tensor, status: torch.Tensor | None = None) -> None:
    """Write ``k``/``v`` ``[B, n, H, D]`` into rows ``[start, start+n)`` of both planes
    of ``cache`` ``[2, B, S, H, D]``. Raises ``RuntimeError("KV cache full ...")``
    when ``start + n > S``, before anything is launched.

    ``start`` may be a device cursor (a one-element int32 tensor), read by the
    kernel when it runs; a block that would not fit is then skipped and
    ``status`` (an int32 tensor, optional) set to 1.
    """
    return select("cache", "append", cache, k, v)(cache, k, v, start, status)


def qk_norm_rope_append(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    cache: torch.Tensor,
    start: int | torch.Tensor,
    eps: float = 1e-6,
    interleaved: bool = True,
    status: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``qk_norm_rope`` and ``kv_cache_append`` of the rotated k and raw v, in one pass.

    Same results as ``q, k = qk_norm_rope(...)`` followed by
    ``kv_cache_append(cache, k, v, start, status)``; ``start`` may be a device cursor.
    """
    return select("rope", "qk_norm_rope_append", q, k, v, cache)(
        q, k, v, q_weight, k_weight, cos, sin, cache, start, eps, interleaved, status)


# Importing the implementation package is what populates the registry.
from . import gfx950  # noqa: E402,F401
