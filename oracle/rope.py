"""Torch restatement of dexter's reference QK-RMSNorm + rotary.

Follows ``python/dexter/ops/reference/rope.py``:

* ``rms_norm`` (:29-40): the mean of squares spans the token's whole
  ``H*D`` plane (Wan normalises before the head split); fp32
  ``x * rsqrt(mean(x^2) + eps)``, times the ``H*D`` weight, then cast back to
  the input dtype (:40) -- the first rounding.
* ``rotary`` (:10-26): fp32; interleaved pairs ``(2j, 2j+1)`` (:20-24) or
  split-half pairs ``(j, j + D/2)`` (:25-26); ``lo*c - hi*s`` and
  ``lo*s + hi*c`` with cos/sin ``[L, D/2]`` broadcast over batch and heads;
  cast to the input dtype -- the second rounding.
* ``qk_norm_rope`` (:43-56): norm then rotary, for q and k.
* ``qkv_project`` restates the three ``nn.Linear`` projections in front of it
  (``models/dreamzero/model.py:162-165``): fp32 products and sums of the io-dtype
  operands plus the bias, rounded once to the io dtype (what a bf16
  ``F.linear`` returns, up to the summation order).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    b, seq, heads, dim = x.shape
    plane = x.reshape(b, seq, heads * dim).float()
    inv = torch.rsqrt(plane.pow(2).mean(dim=-1, keepdim=True) + eps)
    normed = (plane * inv) * weight.float().reshape(1, 1, heads * dim)
    return normed.reshape(b, seq, heads, dim).to(x.dtype)


def rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, interleaved: bool,
           keep_fp32: bool = False) -> torch.Tensor:
    b, seq, heads, dim = x.shape
    c = cos.float().reshape(1, -1, 1, dim // 2)
    s = sin.float().reshape(1, -1, 1, dim // 2)
    xf = x.float()
    if interleaved:
        lo, hi = xf[..., 0::2], xf[..., 1::2]
        out = torch.stack((lo * c - hi * s, lo * s + hi * c), dim=-1).reshape(b, seq, heads, dim)
    else:
        lo, hi = xf[..., : dim // 2], xf[..., dim // 2:]
        out = torch.cat((lo * c - hi * s, lo * s + hi * c), dim=-1)
    return out if keep_fp32 else out.to(x.dtype)


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps: float = 1e-6,
                 interleaved: bool = True, keep_fp32: bool = False):
    """Both tensors through ``rms_norm`` then ``rotary``.

    ``keep_fp32`` skips only the final cast (the intermediate rounding stays,
    since it is part of what the reference computes).
    """
    qn, kn = rms_norm(q, q_weight, eps), rms_norm(k, k_weight, eps)
    return (rotary(qn, cos, sin, interleaved, keep_fp32),
            rotary(kn, cos, sin, interleaved, keep_fp32))


def qkv_project(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, heads: int,
                keep_fp64: bool = False) -> torch.Tensor:
    """``F.linear(x, w, b)`` of ``x [B, L, C]``, viewed as ``[B, L, heads, D]``.

    Computed in fp64 from the io-dtype operands; rounded once to x's dtype
    unless ``keep_fp64``.
    """
    y = x.double() @ w.double().t()
    if b is not None:
        y = y + b.double()
    y = y.reshape(x.shape[0], x.shape[1], heads, -1)
    return y if keep_fp64 else y.to(x.dtype)
