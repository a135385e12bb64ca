"""Callers of the attention path: the per-layer KV cache and a self-attention layer."""

from .kv_cache import KVCache
from .attention import SelfAttention

__all__ = ["KVCache", "SelfAttention"]
