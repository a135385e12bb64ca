"""Comparison helpers shared by the tests."""

from __future__ import annotations

import torch

# Parity bar for bf16 kernels against the fp32 oracle (north star): max-abs
# error <= 2e-2 and mean-abs error <= 2e-3.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def errors(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    d = (got.detach().float().cpu() - ref.detach().float().cpu()).abs()
    return d.max().item(), d.mean().item()


def assert_parity(got, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    mx, mn = errors(g, r)
    assert mx <= max_abs and mn <= mean_abs, (
        f"{what}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})")
    return mx, mn


def close_rel(a, b, tol=2e-2):
    """The reference suite's comparison (test/test_ops.py:12-15): max|a-b| / max|b| < tol."""
    a, b = a.float().cpu(), b.float().cpu()
    err = (a - b).abs().max().item() / max(b.abs().max().item(), 1e-6)
    assert err < tol, f"max rel err {err:.4g}"


def assert_parity_scaled(got, ref, max_rel=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    """Parity where outputs exceed 1 in magnitude: |err| <= max_rel * max(1, |ref|).

    For |ref| <= 1 this is the absolute 2e-2 bar. Above 1 it scales with the
    value, because storing the output in bf16 alone costs up to 2^-9 |ref|
    (0.04 at |ref| = 20), beyond any absolute 2e-2. Mean-abs stays absolute.
    """
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    assert g.shape == r.shape and torch.isfinite(g).all(), what
    d = (g - r).abs()
    scaled = (d / r.abs().clamp_min(1.0)).max().item()
    assert scaled <= max_rel and d.mean().item() <= mean_abs, (
        f"{what}: max-abs {d.max().item():.3e} at scaled {scaled:.3e} (<= {max_rel}), "
        f"mean-abs {d.mean().item():.3e} (<= {mean_abs}), max |ref| {r.abs().max().item():.1f}")
    return d.max().item(), d.mean().item()
