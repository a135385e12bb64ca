"""Per-layer self-attention KV cache (contract of ``models/dreamzero/model.py:35-65``).

One ``[2, B, capacity, H, D]`` tensor per layer, allocated once for the
episode. ``append(layer, k, v)`` writes rows ``[length, length+n)`` of both
planes and does **not** move the cursor; ``commit(n)`` moves it once every
layer has appended its block; ``reset()`` rewinds it. Overflow raises
``RuntimeError("KV cache full: ...")`` before anything is written.

Here ``append`` launches the HIP ``cache/append`` kernel through the op
registry instead of two torch slice copies. ``append_fused`` is the
``rope/qk_norm_rope_append`` form: the caller's prologue writes k and v into
the slot in the same pass that produces q and k.

Layout in HBM: the reference's ``[2, B, S, H, D]``, contiguous. A
head-major store (``[2, B, H, S, D]`` behind the same view, so each head's
history is one contiguous run) was measured on MI355X at the Wan-5B chunk
shape and gave no gain (15.77 vs 15.81 us per attention call), so the
reference layout stays.

Sizing on MI355X: a Wan-5B layer at 1,328 rows is 2 x 1328 x 24 x 128 x 2 B
= 16.3 MB, so all 30 layers of a long episode fit many times over in 288 GB.

``device_cursor=True`` keeps the cursor in device memory too (``self.cursor``,
one int32): appends write at it and attention reads ``cache_len`` from it when
the kernels run, and ``commit`` advances it with a device add. A HIP graph
captured once then replays every control step of an episode as the cache grows
(``runtime.graph.CachedStepGraph``). The host ``length`` stays the mirror the
overflow check uses; a block that slips past it is not written and sets
``self.status``, which ``overflowed()`` reports.
"""

from __future__ import annotations

import torch

from .. import ops


class KVCache:
    def __init__(self, layers: int, batch: int, capacity: int, heads: int, head_dim: int,
                 device: torch.device | str, dtype: torch.dtype,
                 device_cursor: bool = False) -> None:
        self.cache = [
            torch.zeros(2, batch, capacity, heads, head_dim, device=device, dtype=dtype)
            for _ in range(layers)
        ]
        self.capacity = capacity
        self.length = 0
        self.cursor = self.status = None
        if device_cursor:
            self.cursor = torch.zeros(1, dtype=torch.int32, device=device)
            self.status = torch.zeros(1, dtype=torch.int32, device=device)

    @property
    def cache_len(self) -> int | torch.Tensor:
        """What attention takes as ``cache_len``: the device cursor, or the host length."""
        return self.cursor if self.cursor is not None else self.length

    def _start(self):
        return self.cursor if self.cursor is not None else self.length

    def _check_room(self, n: int) -> None:
        if self.length + n > self.capacity:
            raise RuntimeError(f"KV cache full: {self.length} + {n} > {self.capacity}")

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write one block's k/v for ``layer`` at the cursor (cursor unchanged)."""
        self._check_room(k.shape[1])
        ops.kv_cache_append(self.cache[layer], k, v, self._start(), self.status)

    def append_fused(self, layer: int, q, k, v, q_weight, k_weight, cos, sin, eps=1e-6,
                     interleaved=True):
        """QK-norm + rotary on q/k, writing rotated k and raw v at the cursor.

        Returns the rotated ``(q, k)``; equivalent to ``ops.qk_norm_rope``
        followed by :meth:`append` of the rotated k.
        """
        self._check_room(k.shape[1])
        return ops.qk_norm_rope_append(q, k, v, q_weight, k_weight, cos, sin,
                                       self.cache[layer], self._start(), eps, interleaved,
                                       self.status)

    def commit(self, n: int) -> None:
        """Advance the write cursor once every layer has appended its block."""
        self.length += n
        if self.cursor is not None:
            self.cursor.add_(n)

    def reset(self) -> None:
        self.length = 0
        if self.cursor is not None:
            self.cursor.zero_()
            self.status.zero_()

    def overflowed(self) -> bool:
        """Whether a device-cursor append found no room (synchronises with the device)."""
        return bool(self.status is not None and int(self.status.item()) != 0)
