"""Write the golden vectors in this folder (run from the repository root).

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path, so these are written by
the fp64 brute force (``oracle/brute.py``), which follows the reference's
definitions (``ops/reference/attention.py:22-77``, ``ops/reference/rope.py:10-56``)
with explicit loops and no torch arithmetic:

* ``c0_attention.npz``: config C0 (1 x 48 x 4 x 64, fp32 inputs drawn from
  seed 0, block starts [0, 16, 32], no cache) -- inputs and the fp64 output;
  plus the same inputs with the first 24 rows as a cache and starts [0, 12].
* ``prologue_small.npz``: a 2 x 6 x 3 x 16 bf16 q/k pair (seed 7), weights,
  fp32 cos/sin for positions 3..8 -- inputs (as fp32 values of the bf16
  numbers) and the fp64 prologue output with the reference's bf16 rounding
  after the norm, for interleaved and split-half pairs.

Files are plain ``.npz`` arrays (no pickles).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
for p in (ROOT, ROOT / "dexter-labs_amd"):
    sys.path.insert(0, str(p))

from dexter_amd.bench.workloads import CONFIGS, make_inputs, rope_table  # noqa: E402
from oracle import brute  # noqa: E402

HERE = Path(__file__).resolve().parent


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).double().numpy()


def c0() -> None:
    inp = make_inputs(CONFIGS["C0"])
    q, k, v = (t.numpy().astype(np.float32) for t in (inp.q, inp.k, inp.v))
    out = brute.attention(q, k, v, starts=[0, 16, 32])
    ck, cv = k[:, :24], v[:, :24]
    out_cache = brute.attention(q[:, 24:], k[:, 24:], v[:, 24:], ck, cv, cache_len=24,
                                starts=[0, 12])
    np.savez(HERE / "c0_attention.npz", q=q, k=k, v=v, starts=np.array([0, 16, 32]),
             out=out, cache_len=np.array(24), cache_starts=np.array([0, 12]),
             out_cache=out_cache)


def prologue() -> None:
    g = torch.Generator().manual_seed(7)
    b, l, h, d = 2, 6, 3, 16
    q = torch.randn(b, l, h, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, l, h, d, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(h * d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(h * d, generator=g)).to(torch.bfloat16)
    cos, sin = rope_table(torch.arange(l) + 3, d)
    arrays = {"q": q.float().numpy(), "k": k.float().numpy(), "qw": qw.float().numpy(),
              "kw": kw.float().numpy(), "cos": cos.numpy(), "sin": sin.numpy()}
    for inter in (True, False):
        tag = "interleaved" if inter else "split_half"
        for name, x, w in (("q", q, qw), ("k", k, kw)):
            arrays[f"{name}_out_{tag}"] = brute.qk_norm_rope(
                x.float().numpy(), w.float().numpy(), cos.numpy(), sin.numpy(), 1e-6, inter,
                round_to=bf16_round)
    np.savez(HERE / "prologue_small.npz", **arrays)


if __name__ == "__main__":
    c0()
    prologue()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
