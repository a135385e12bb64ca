"""Adaptive LayerNorm modulation and gated residual on gfx950 (``dx_adaln_modulate``,
``dx_gated_residual``).

Registered as ``norm/adaln`` and ``norm/gated_residual`` with the signatures of
dexter's implementations (``ops/reference/norm.py:16-25``,
``ops/gfx1151/norm/adaln.py:108-148``):

* ``adaln_modulate(x, scale, shift, eps)`` = ``layer_norm(x) * (1 + scale) + shift``
* ``gated_residual(x, y, gate)`` = ``x + y * gate``

Shapes broadcast as the reference's torch expressions do: a Wan block passes
``[B, 1, C]`` modulation rows (``models/dreamzero/model.py:264-278``), the
affine ``norm3`` passes ``[C]`` (``models/layers.py:81-83``). Broadcast operands
are read in place through stride-0 rows, never expanded in memory; the
reference's Triton launcher copies a ``[B, 1, C]`` modulation out to ``[B*L, C]``
(``ops/gfx1151/norm/adaln.py:96-105``). The result dtype is torch's promotion
of the operand dtypes, as the reference expression gives; the arithmetic is
fp32 with one rounding at the end.
"""

from __future__ import annotations

import math

import torch

from ...registry import Priority, register
from . import _lib
from ._common import CDNA4

_FLOAT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_PACKS_PER_LANE = 4
_MAX_WAVES = 16
_MAX_BATCH_GRID = 65535


def _max_cols(dtype: torch.dtype) -> int:
    per_pack = 16 // torch.empty((), dtype=dtype).element_size()
    return _PACKS_PER_LANE * 64 * per_pack * _MAX_WAVES


def _promote(*dtypes: torch.dtype) -> torch.dtype:
    out = dtypes[0]
    for d in dtypes[1:]:
        out = torch.promote_types(out, d)
    return out


def _broadcast_ok(x, *others) -> bool:
    tensors = (x, *others)
    if not all(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype in _FLOAT_DTYPES
               and t.device == x.device for t in tensors):
        return False
    if x.dim() == 0:
        return False
    try:
        shape = torch.broadcast_shapes(*(t.shape for t in tensors))
    except RuntimeError:
        return False
    cols = x.shape[-1]
    return shape[-1] == cols and cols <= _max_cols(x.dtype)


def _accepts_adaln(x, scale, shift, *args, **kwargs) -> bool:
    return _broadcast_ok(x, scale, shift)


def _accepts_gated(x, y, gate, *args, **kwargs) -> bool:
    return _broadcast_ok(x, y, gate) and _max_cols(_promote(x.dtype, y.dtype)) >= x.shape[-1]


def _rows3(t: torch.Tensor, shape: torch.Size, b: int, seq: int) -> tuple[torch.Tensor, int, int]:
    """``t`` broadcast to ``shape`` and viewed as ``[b, seq, C]`` rows: the tensor and its
    batch and row strides in elements. Broadcast dims keep stride 0 (no copy); a copy is
    made only when the last dim is not contiguous or the leading dims cannot be merged."""
    cols = shape[-1]
    e = t.expand(shape).reshape(b, seq, cols)
    if cols > 1 and e.stride(-1) != 1:
        e = e.contiguous()
    sb = 0 if e.shape[0] == 1 else e.stride(0)
    sl = 0 if e.shape[1] == 1 else e.stride(1)
    return e, sb, sl


def _row_grid(shape: torch.Size) -> tuple[int, int]:
    """``(B, L)`` for ``shape[:-1]``: the last leading dim is L, the rest fold into B.
    The kernel's batch grid dimension holds at most 65535, so a larger B folds into L."""
    lead = list(shape[:-1])
    if not lead:
        return 1, 1
    seq = lead[-1]
    b = math.prod(lead[:-1]) if len(lead) > 1 else 1
    if b > _MAX_BATCH_GRID:
        return 1, b * seq
    return b, seq


@register("norm", "adaln", name="hip_adaln_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts_adaln)
def adaln_modulate(x, scale, shift, eps):
    shape = torch.broadcast_shapes(x.shape, scale.shape, shift.shape)
    if shape[-1] != x.shape[-1]:
        raise ValueError(f"scale/shift {tuple(scale.shape)}/{tuple(shift.shape)} must broadcast "
                         f"to rows of x {tuple(x.shape)}")
    mdt = _promote(scale.dtype, shift.dtype)
    scale, shift = scale.to(mdt), shift.to(mdt)
    odt = _promote(x.dtype, mdt)
    b, seq = _row_grid(shape)
    cols = shape[-1]
    out = torch.empty(shape, device=x.device, dtype=odt)
    if out.numel() == 0:
        return out
    xv, x_sb, x_sl = _rows3(x, shape, b, seq)
    sc, sc_sb, sc_sl = _rows3(scale, shape, b, seq)
    sh, sh_sb, sh_sl = _rows3(shift, shape, b, seq)
    o3 = out.view(b, seq, cols)
    lib = _lib.load()
    rc = lib.dx_adaln_modulate(
        xv.data_ptr(), x_sb, x_sl, _lib.dtype_code(x.dtype),
        sc.data_ptr(), sc_sb, sc_sl, sh.data_ptr(), sh_sb, sh_sl, _lib.dtype_code(mdt),
        o3.data_ptr(), o3.stride(0), o3.stride(1), _lib.dtype_code(odt),
        b, seq, cols, float(eps), _lib.stream_handle(x.device))
    _lib.check(rc, "adaln_modulate")
    return out


@register("norm", "gated_residual", name="hip_gated_residual_gfx950",
          capability=CDNA4, priority=Priority.SPECIALISED, accepts=_accepts_gated)
def gated_residual(x, y, gate):
    shape = torch.broadcast_shapes(x.shape, y.shape, gate.shape)
    if shape[-1] != x.shape[-1]:
        raise ValueError(f"y/gate {tuple(y.shape)}/{tuple(gate.shape)} must broadcast to rows "
                         f"of x {tuple(x.shape)}")
    xdt = _promote(x.dtype, y.dtype)
    x, y = x.to(xdt), y.to(xdt)
    odt = _promote(xdt, gate.dtype)
    b, seq = _row_grid(shape)
    cols = shape[-1]
    out = torch.empty(shape, device=x.device, dtype=odt)
    if out.numel() == 0:
        return out
    xv, x_sb, x_sl = _rows3(x, shape, b, seq)
    yv, y_sb, y_sl = _rows3(y, shape, b, seq)
    gv, g_sb, g_sl = _rows3(gate, shape, b, seq)
    o3 = out.view(b, seq, cols)
    lib = _lib.load()
    rc = lib.dx_gated_residual(
        xv.data_ptr(), x_sb, x_sl, yv.data_ptr(), y_sb, y_sl, _lib.dtype_code(xdt),
        gv.data_ptr(), g_sb, g_sl, _lib.dtype_code(gate.dtype),
        o3.data_ptr(), o3.stride(0), o3.stride(1), _lib.dtype_code(odt),
        b, seq, cols, _lib.stream_handle(x.device))
    _lib.check(rc, "gated_residual")
    return out
