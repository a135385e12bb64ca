"""Comparison helpers shared by the tests."""

from __future__ import annotations

import torch

# Parity bar for bf16 kernels against the fp32 oracle (north star): max-abs
# error <= 2e-2 and mean-abs error <= 2e-3.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def report(what: str, text: str) -> None:
    """One line per named check, shown by ``pytest -s``: the measured errors
    behind each parity figure, not only whether the bar held."""
    if what:
        print(f"[parity] {what}: {text}")


def errors(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    d = (got.detach().float().cpu() - ref.detach().float().cpu()).abs()
    return d.max().item(), d.mean().item()


def assert_parity(got, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    mx, mn = errors(g, r)
    report(what, f"max-abs {mx:.3e} mean-abs {mn:.3e}")
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
    report(what, f"max-abs {d.max().item():.3e} (scaled {scaled:.3e}) mean-abs {d.mean().item():.3e}")
    assert scaled <= max_rel and d.mean().item() <= mean_abs, (
        f"{what}: max-abs {d.max().item():.3e} at scaled {scaled:.3e} (<= {max_rel}), "
        f"mean-abs {d.mean().item():.3e} (<= {mean_abs}), max |ref| {r.abs().max().item():.1f}")
    return d.max().item(), d.mean().item()


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at each entry of the bf16 tensor ``x`` (fp32).

    |x| in [2^(e-1), 2^e) has spacing 2^(e-8) (8 significant bits); zeros and
    subnormals take the subnormal spacing 2^-133.
    """
    _, e = torch.frexp(x.float())
    return torch.where(x.float().abs() >= 2.0 ** -126, torch.ldexp(torch.ones_like(x, dtype=torch.float32), e - 8),
                       torch.full_like(x, 2.0 ** -133, dtype=torch.float32))


def assert_within_ulp(got, ref, ulps=1, frac=0.999, min_abs=1.0, mean_abs=MEAN_ABS, what=""):
    """Strict parity for a bf16 kernel where ``assert_parity_scaled`` relaxes
    the absolute bar (|ref| >= ``min_abs``, 1 by default): against the fp32
    reference rounded to bf16, at least ``frac`` of those elements are within
    ``ulps`` bf16 spacings. The mean-abs error over all elements stays <=
    ``mean_abs``. Elements below ``min_abs`` keep the absolute bar: near zero
    a spacing-based bound is meaningless, since the error of a sum of
    probability-weighted values scales with the terms, not with the sum.
    """
    g = got.detach().cpu()
    assert g.dtype == torch.bfloat16, f"{what}: expected a bf16 output"
    assert torch.isfinite(g.float()).all(), f"{what}: non-finite output"
    r = ref.detach().float().cpu()
    r16 = r.to(torch.bfloat16)
    n_ulp = (g.float() - r16.float()).abs() / bf16_ulp(r16)
    sel = r16.float().abs() >= min_abs
    within = (n_ulp[sel] <= ulps).float().mean().item() if sel.any() else 1.0
    mn = (g.float() - r).abs().mean().item()
    report(what, f"{within:.5f} of |ref| >= {min_abs} within {ulps} bf16 ulp")
    assert within >= frac and mn <= mean_abs, (
        f"{what}: {within:.5f} of {int(sel.sum())} elements with |ref| >= {min_abs} within "
        f"{ulps} bf16 ulp (>= {frac}), max {n_ulp[sel].max().item():.1f} ulp there, "
        f"mean-abs {mn:.3e} (<= {mean_abs})")
    return within
