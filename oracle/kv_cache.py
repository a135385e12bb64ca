"""The KV-cache contract of ``python/dexter/models/dreamzero/model.py:35-65``, on CPU.

``append(layer, k, v)`` copies into rows ``[length, length+n)`` of planes 0
(k) and 1 (v) without moving the cursor (:53-58) and raises
``RuntimeError("KV cache full: ...")`` first when ``length + n > capacity``
(:55-56); ``commit(n)`` moves the cursor (:60-62); ``reset()`` (:64-65).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import torch


class KVCache:
    def __init__(self, layers, batch, capacity, heads, head_dim, dtype=torch.bfloat16):
        self.cache = [torch.zeros(2, batch, capacity, heads, head_dim, dtype=dtype)
                      for _ in range(layers)]
        self.capacity = capacity
        self.length = 0

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        n = k.shape[1]
        if self.length + n > self.capacity:
            raise RuntimeError(f"KV cache full: {self.length} + {n} > {self.capacity}")
        rows = slice(self.length, self.length + n)
        self.cache[layer][0, :, rows].copy_(k.cpu())
        self.cache[layer][1, :, rows].copy_(v.cpu())

    def commit(self, n: int) -> None:
        self.length += n

    def reset(self) -> None:
        self.length = 0
