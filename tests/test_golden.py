"""The oracle against the committed golden vectors (``tests/golden/``).

The vectors were written by ``tests/golden/make_golden.py`` with the fp64
brute force; they freeze the expected results of config C0 and of a small
prologue case so that a later change to the oracle, the input recipe or the
brute force itself shows up here.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import rope as orope

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def test_c0_inputs_follow_the_recipe():
    from dexter_amd.bench.workloads import CONFIGS, make_inputs
    g = _load("c0_attention.npz")
    inp = make_inputs(CONFIGS["C0"])
    for name in ("q", "k", "v"):
        assert np.array_equal(getattr(inp, name).numpy(), g[name]), name


def test_c0_oracle_matches_golden():
    g = _load("c0_attention.npz")
    q, k, v = (torch.from_numpy(g[n]) for n in ("q", "k", "v"))
    out = oatt.blockwise_causal_attention(q, k, v, None, 0, torch.from_numpy(g["starts"]), None,
                                          keep_fp32=True)
    assert np.abs(out.double().numpy() - g["out"]).max() < 1e-5


def test_c0_with_cache_oracle_matches_golden():
    g = _load("c0_attention.npz")
    c = int(g["cache_len"])
    q, k, v = (torch.from_numpy(g[n]) for n in ("q", "k", "v"))
    cache = torch.stack((k[:, :c], v[:, :c]))
    out = oatt.blockwise_causal_attention(q[:, c:], k[:, c:], v[:, c:], cache, c,
                                          torch.from_numpy(g["cache_starts"]), None,
                                          keep_fp32=True)
    assert np.abs(out.double().numpy() - g["out_cache"]).max() < 1e-5


@pytest.mark.parametrize("interleaved", [True, False])
def test_prologue_oracle_matches_golden(interleaved):
    g = _load("prologue_small.npz")
    tag = "interleaved" if interleaved else "split_half"
    q, k = (torch.from_numpy(g[n]).to(torch.bfloat16) for n in ("q", "k"))
    qw, kw = (torch.from_numpy(g[n]).to(torch.bfloat16) for n in ("qw", "kw"))
    cos, sin = torch.from_numpy(g["cos"]), torch.from_numpy(g["sin"])
    oq, ok = orope.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6, interleaved, keep_fp32=True)
    for got, ref in ((oq, g[f"q_out_{tag}"]), (ok, g[f"k_out_{tag}"])):
        diff = np.abs(got.double().numpy() - ref)
        # fp32 vs fp64 around the reference's bf16 rounding after the norm: a
        # few fp32 ulps, except where a value sits on a bf16 rounding tie.
        assert np.quantile(diff, 0.99) < 1e-5
        assert diff.max() < 2e-2
