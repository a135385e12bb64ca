"""A self-attention layer that calls the path the way DreamZero's DiT does.

Follows ``SelfAttention.forward`` (``models/dreamzero/model.py:158-183``):
project q/k/v, QK-RMSNorm + rotary through ``ops.qk_norm_rope``, read
``cache_len`` **before** appending, append k/v only when ``write``, attend
with ``ops.blockwise_causal_attention`` over the cache plus the new block,
project out. It exists to show the drop-in: nothing here names a kernel, the
registry picks the gfx950 implementations.

With ``write=True`` the prologue and the append run as one kernel
(``KVCache.append_fused``). For decode chunks (at most 128 tokens, ``dim`` a
multiple of 512) the q/k/v projections join them: ``ops.qkv_norm_rope`` runs
the projections, the prologue and the cache write in two kernels. Longer
chunks use ``torch.nn.functional.linear`` (hipBLASLt) for the projections and,
with a host cache length, ``ops.qk_norm_rope_attention`` for the prologue,
append and attention in one call.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import ops
from .kv_cache import KVCache


class SelfAttention(nn.Module):
    def __init__(self, dim: int, heads: int, eps: float = 1e-6,
                 dtype: torch.dtype = torch.bfloat16, device=None) -> None:
        super().__init__()
        if dim % heads:
            raise ValueError("dim must be a multiple of heads")
        self.heads, self.head_dim, self.eps = heads, dim // heads, eps
        kw = dict(dtype=dtype, device=device)
        self.q = nn.Linear(dim, dim, **kw)
        self.k = nn.Linear(dim, dim, **kw)
        self.v = nn.Linear(dim, dim, **kw)
        self.o = nn.Linear(dim, dim, **kw)
        # Wan's QK norm spans the full dim (applied before the head split).
        self.q_norm = nn.Parameter(torch.ones(dim, **kw))
        self.k_norm = nn.Parameter(torch.ones(dim, **kw))

    @torch.no_grad()
    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                kv_cache: KVCache | None, layer: int,
                block_boundaries: torch.Tensor | None = None, write: bool = False,
                fused_append: bool = True, fused_qkv: bool = True) -> torch.Tensor:
        b, seq, dim = x.shape
        shape = (b, seq, self.heads, self.head_dim)
        # Read before appending; with a device cursor this is the cursor itself,
        # which the commit after all layers advances.
        cache_len = kv_cache.cache_len if kv_cache is not None else 0
        append = kv_cache is not None and write

        if fused_qkv and b * seq <= 128 and dim % 512 == 0 and self.head_dim % 16 == 0:
            if append:
                kv_cache._check_room(seq)
            q, k, v = ops.qkv_norm_rope(
                x, self.q.weight, self.q.bias, self.k.weight, self.k.bias, self.v.weight,
                self.v.bias, self.q_norm, self.k_norm, cos, sin, self.heads, self.eps,
                cache=kv_cache.cache[layer] if append else None,
                start=kv_cache._start() if append else 0,
                status=kv_cache.status if append else None)
            return self._attend(q, k, v, kv_cache, layer, cache_len, block_boundaries)

        q = F.linear(x, self.q.weight, self.q.bias).view(shape)
        k = F.linear(x, self.k.weight, self.k.bias).view(shape)
        v = F.linear(x, self.v.weight, self.v.bias).view(shape)
        if fused_append and not isinstance(cache_len, torch.Tensor):
            if append:
                kv_cache._check_room(seq)
            out = ops.qk_norm_rope_attention(
                q, k, v, self.q_norm, self.k_norm, cos, sin,
                kv_cache=kv_cache.cache[layer] if kv_cache is not None else None,
                cache_len=cache_len, append=append, block_boundaries=block_boundaries,
                eps=self.eps)
            return F.linear(out.reshape(b, seq, -1), self.o.weight, self.o.bias)
        if append and fused_append:
            q, k = kv_cache.append_fused(layer, q, k, v, self.q_norm, self.k_norm, cos, sin,
                                         self.eps)
        else:
            q, k = ops.qk_norm_rope(q, k, self.q_norm, self.k_norm, cos, sin, self.eps)
            if append:
                kv_cache.append(layer, k, v)
        return self._attend(q, k, v, kv_cache, layer, cache_len, block_boundaries)

    def _attend(self, q, k, v, kv_cache, layer, cache_len, block_boundaries):
        b, seq = q.shape[:2]
        out = ops.blockwise_causal_attention(
            q, k, v,
            kv_cache=kv_cache.cache[layer] if kv_cache is not None else None,
            cache_len=cache_len,
            block_boundaries=block_boundaries,
        )
        return F.linear(out.reshape(b, seq, -1), self.o.weight, self.o.bias)
