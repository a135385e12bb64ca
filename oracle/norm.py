"""Torch restatement of dexter's reference adaLN modulation and gated residual.

Follows ``python/dexter/ops/reference/norm.py``:

* ``adaln_modulate`` (:16-20): LayerNorm over the last dim with no affine
  parameters (biased variance, ``eps`` inside the square root), computed by
  torch in fp32 and rounded once to x's dtype; then ``* (1 + scale)`` and
  ``+ shift``, each op rounding to torch's promoted dtype.
* ``gated_residual`` (:23-25): ``x + y * gate``, each op rounding to the
  promoted dtype.

``adaln_modulate_exact`` / ``gated_residual_fp32`` state the arithmetic the
fused kernels perform instead (the Triton kernels, ``ops/gfx1151/norm/adaln.py:36-48``
and :62-67, and the HIP kernels here): everything in wide precision, one
rounding at the end. The exact form is fp64, so a kernel that computes in
fp32 is within one unit in the last place of it; ``gated_residual_fp32`` is
the fp32 product and fp32 sum, each rounded, which the HIP kernel matches bit
for bit.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _promote(*dtypes: torch.dtype) -> torch.dtype:
    out = dtypes[0]
    for d in dtypes[1:]:
        out = torch.promote_types(out, d)
    return out


def adaln_modulate(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                   eps: float = 1e-6) -> torch.Tensor:
    """The reference expression, op by op, with its intermediate roundings."""
    normed = F.layer_norm(x, (x.shape[-1],), eps=eps)  # x's dtype
    gain = 1 + scale                                     # scale's dtype
    return normed * gain + shift


def adaln_modulate_exact(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                         eps: float = 1e-6, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """fp64 LayerNorm statistics and modulation, one rounding to the promoted dtype
    (or ``out_dtype``; pass ``torch.float64`` to keep the unrounded values)."""
    odt = out_dtype or _promote(x.dtype, scale.dtype, shift.dtype)
    xd = x.double()
    mean = xd.mean(dim=-1, keepdim=True)
    var = (xd - mean).pow(2).mean(dim=-1, keepdim=True)
    normed = (xd - mean) / torch.sqrt(var + eps)
    return (normed * (1 + scale.double()) + shift.double()).to(odt)


def gated_residual(x: torch.Tensor, y: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """The reference expression, op by op, with its intermediate roundings."""
    prod = y * gate
    return x + prod


def gated_residual_fp32(x: torch.Tensor, y: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """fp32 product, fp32 sum (each rounded, no fused multiply-add), one rounding
    to the promoted dtype."""
    odt = _promote(x.dtype, y.dtype, gate.dtype)
    prod = y.float() * gate.float()
    return (x.float() + prod).to(odt)
