"""Capability gate and tensor plumbing shared by the gfx950 implementations."""

from __future__ import annotations

import torch

from ...platform import ArchVersion, Capability

# Every kernel here is written for gfx950 only: wave64, v_mfma_f32_32x32x16
# (bf16/f16), 160 KB of LDS. The gate pins the arch to (9, 5) exactly, so it
# never admits RDNA3 (11.x) and RDNA3 gates (min 11.0) never admit it.
CDNA4 = Capability(
    vendors=frozenset({"amd"}),
    min_arch=ArchVersion(9, 5),
    max_arch=ArchVersion(9, 5),
    features=frozenset({"mma:mfma", "matrix:bf16"}),
)

MATRIX_DTYPES = (torch.bfloat16, torch.float16)


def rows_ok(t: torch.Tensor) -> bool:
    """Last dim contiguous and every other stride keeps 16-byte row alignment."""
    if t.stride(-1) != 1 and t.shape[-1] != 1:
        return False
    per16 = 16 // t.element_size()
    return (t.data_ptr() % 16 == 0
            and all(s % per16 == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1))


def as_rows(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself when the kernels can read it in place, else a contiguous copy."""
    return t if rows_ok(t) else t.contiguous()


def strides(t: torch.Tensor, dims: int) -> list[int]:
    """The first ``dims`` strides; a size-1 dim gets stride 0 (it is never stepped)."""
    return [0 if t.shape[i] == 1 else t.stride(i) for i in range(dims)]


def device_cursor(t: torch.Tensor, device: torch.device, what: str) -> torch.Tensor:
    """A device-resident cache cursor: a one-element int32 tensor on ``device``.

    Kernels read it when they run, so a captured graph follows it as it moves.
    It is never copied or converted here: the kernels must read the caller's
    tensor, the one the caller advances.
    """
    if t.dtype != torch.int32 or t.numel() != 1 or t.device != device:
        raise ValueError(f"{what}: a device cursor must be one int32 element on {device}, got "
                         f"{t.dtype} x {t.numel()} on {t.device}")
    return t
