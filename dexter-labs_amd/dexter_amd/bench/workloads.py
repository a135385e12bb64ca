"""The five measured/parity configurations (C0-C4) and their synthetic inputs.

Shapes come from dexter's Wan presets (``models/dreamzero/config.py:182-217``:
Wan2.2-TI2V-5B dim 3072 / 24 heads / 30 layers, 83 tokens per control step;
Wan2.1-I2V-14B dim 5120 / 40 heads). Inputs are drawn on the CPU from
``torch.Generator().manual_seed(seed)`` in fp32 -- pre-norm q, pre-norm k, v,
q-norm weight, k-norm weight, then the outlier masks -- and cast/copied
afterwards, so CPU and GPU see identical values.

Algorithmic work counts only visible (query, key) pairs: 4*D FLOP per pair
per head (2*D for q.k, 2*D for p.v). Algorithmic bytes are q read + visible
K/V read + o write, each once, at the storage width.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class Config:
    name: str
    seed: int
    batch: int
    heads: int
    head_dim: int
    q_len: int
    cache_lens: tuple[int, ...]       # per sequence (uniform configs repeat one value)
    block_starts: tuple[int, ...] | None
    dtype: torch.dtype
    prologue: bool
    hidden: int = 0
    outlier_p: float = 0.0
    outlier_scale: float = 1.0
    theta: float = 10000.0
    frame_len: int = 0                # varlen: frame tokens per sequence
    note: str = ""

    @property
    def kv_lens(self) -> tuple[int, ...]:
        return tuple(c + self.q_len for c in self.cache_lens)

    def visible_pairs(self) -> int:
        """Visible (query, key) pairs per head, summed over the batch."""
        total = 0
        for c in self.cache_lens:
            ends = _current_ends(self.q_len, self.block_starts)
            total += sum(c + e for e in ends)
        return total

    def flops(self) -> int:
        return 4 * self.head_dim * self.heads * self.visible_pairs()

    def bytes(self) -> int:
        """Q + O plus each visible K/V row once, per head."""
        es = torch.finfo(self.dtype).bits // 8
        qo = 2 * self.batch * self.q_len * self.heads * self.head_dim * es
        kv_rows = 0
        for c in self.cache_lens:
            kv_rows += c + max(_current_ends(self.q_len, self.block_starts))
        return qo + 2 * kv_rows * self.heads * self.head_dim * es


def _current_ends(q_len: int, starts) -> list[int]:
    if starts is None:
        return [q_len] * q_len
    bounds = list(starts) + [q_len]
    ends = [0] * q_len
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        for i in range(max(lo, 0), min(hi, q_len)):
            ends[i] = max(ends[i], min(hi, q_len))
    return ends


CONFIGS: dict[str, Config] = {
    "C0": Config("C0", 0, 1, 4, 64, 48, (0,), (0, 16, 32), torch.float32, False,
                 note="CPU plumbing: 3 blocks of 16, fp32, no RoPE"),
    "C1": Config("C1", 1, 1, 24, 128, 83, (1245,), None, torch.bfloat16, True, hidden=3072,
                 note="Wan-5B closed-loop chunk: 83 queries over 15 cached blocks + itself"),
    "C2": Config("C2", 2, 1, 24, 128, 8192, (0,), tuple(range(0, 8192, 1024)), torch.bfloat16,
                 True, hidden=3072, note="Wan-5B blockwise-causal prefill, 8 x 1024"),
    "C3": Config("C3", 3, 1, 40, 128, 913, (7304,), None, torch.bfloat16, True, hidden=5120,
                 note="Wan-14B-shaped chunk: 913 queries over 8 cached blocks + itself"),
    "C4": Config("C4", 4, 4, 24, 128, 99, (0, 332, 1245, 3237), (0, 83), torch.bfloat16, False,
                 outlier_p=0.01, outlier_scale=20.0, frame_len=83,
                 note="ragged batch: 83-token frame + 16-token action block per sequence"),
}


def rope_table(positions: torch.Tensor, head_dim: int, theta: float = 10000.0):
    """fp32 ``(cos, sin)`` ``[len(positions), head_dim/2]``, ``inv_j = theta^(-2j/D)``."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = positions.to(torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang), torch.sin(ang)


@dataclass
class Inputs:
    """CPU tensors of one configuration, before any prologue.

    Uniform configs: ``q``/``k``/``v`` are ``[B, cache+q_len, H, D]`` over all
    positions (the cache is the prologue of the first ``cache_len`` rows).
    C4: ``q`` ``[B, q_len, H, D]``; ``k``/``v`` ``[B, max_cache+q_len, H, D]``
    with sequence b's rows ``[0, cache_lens[b])`` as its history and rows
    ``[cache_lens[b], cache_lens[b]+q_len)`` as its current block (rest zero).
    """
    cfg: Config
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    q_weight: torch.Tensor | None = None
    k_weight: torch.Tensor | None = None
    cos: torch.Tensor | None = None
    sin: torch.Tensor | None = None
    extra: dict = field(default_factory=dict)


def make_inputs(cfg: Config) -> Inputs:
    g = torch.Generator().manual_seed(cfg.seed)
    shape_tail = (cfg.heads, cfg.head_dim)
    if cfg.name == "C4":
        max_kv = max(cfg.kv_lens)
        q = torch.zeros(cfg.batch, cfg.q_len, *shape_tail)
        k = torch.zeros(cfg.batch, max_kv, *shape_tail)
        v = torch.zeros(cfg.batch, max_kv, *shape_tail)
        for b, c in enumerate(cfg.cache_lens):
            n = c + cfg.q_len
            qb = torch.randn(1, cfg.q_len, *shape_tail, generator=g)
            kb = torch.randn(1, n, *shape_tail, generator=g)
            vb = torch.randn(1, n, *shape_tail, generator=g)
            for t in (qb, kb, vb):
                hit = torch.rand(t.shape, generator=g) < cfg.outlier_p
                t[hit] *= cfg.outlier_scale
            q[b] = qb[0]
            k[b, :n] = kb[0]
            v[b, :n] = vb[0]
        return Inputs(cfg, q.to(cfg.dtype), k.to(cfg.dtype), v.to(cfg.dtype))
    total = cfg.cache_lens[0] + cfg.q_len
    q = torch.randn(cfg.batch, total, *shape_tail, generator=g)
    k = torch.randn(cfg.batch, total, *shape_tail, generator=g)
    v = torch.randn(cfg.batch, total, *shape_tail, generator=g)
    inp = Inputs(cfg, q.to(cfg.dtype), k.to(cfg.dtype), v.to(cfg.dtype))
    if cfg.prologue:
        hd = cfg.heads * cfg.head_dim
        inp.q_weight = (1.0 + 0.1 * torch.randn(hd, generator=g)).to(cfg.dtype)
        inp.k_weight = (1.0 + 0.1 * torch.randn(hd, generator=g)).to(cfg.dtype)
        inp.cos, inp.sin = rope_table(torch.arange(total), cfg.head_dim, cfg.theta)
    return inp


def block_tensor(cfg: Config, device) -> torch.Tensor | None:
    if cfg.block_starts is None:
        return None
    return torch.tensor(cfg.block_starts, dtype=torch.int32, device=device)


def peak_notes() -> dict:
    return {"peak_bf16_tflops": 2516.6, "peak_hbm_gbps": 8000.0}


def describe(cfg: Config) -> dict:
    return {
        "workload": cfg.name, "note": cfg.note, "batch": cfg.batch, "heads": cfg.heads,
        "head_dim": cfg.head_dim, "q_len": cfg.q_len, "cache_lens": list(cfg.cache_lens),
        "block_starts": list(cfg.block_starts) if cfg.block_starts else None,
        "gflop_per_call": round(cfg.flops() / 1e9, 6), "bytes_per_call": cfg.bytes(),
    }


def _selfcheck():  # pragma: no cover - quick arithmetic check
    for c in CONFIGS.values():
        print(c.name, c.flops() / 1e9, c.bytes(), math.isfinite(c.flops()))


if __name__ == "__main__":  # pragma: no cover
    _selfcheck()
