"""The general attention kernel (MI355X): fp32 inputs and head dims 16, 32, 256.

The reference op is dtype-generic (``ops/reference/attention.py:62-77``: fp32
logits, softmax and product, then ``.to(q.dtype)``) and the Triton kernel it
stands beside takes any power-of-two head dim
(``ops/gfx1151/attention/blockwise_causal.py:162-172``). Calls the bf16/f16
MFMA kernels do not take run on ``csrc/attn_any.hip`` (fp32 softmax and sums;
fp32 MFMA for fp32 inputs and head dim 16, 16-bit MFMA for bf16/f16 at head
dims 32 and 256); everything goes through the registry and the C ABI and is
compared with ``oracle/attention.py``.

Parity bars:

* fp32 inputs: max-abs <= 1e-4 and mean-abs <= 1e-5 against the fp32 oracle on
  N(0, 1) data. Rounding any operand or probability to 16 bits costs 1e-3 to
  1e-2 here, so a kernel that did would fail by one to two orders of magnitude.
* bf16/f16 inputs: the north-star bar, max-abs <= 2e-2 and mean-abs <= 2e-3.

Rows that see no key are NaN in both, as the reference's softmax of an all
``-inf`` row is.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.bench.workloads import CONFIGS, make_inputs
from dexter_amd.ops.gfx950 import _lib
from oracle import attention as oatt

from _util import assert_parity

pytestmark = pytest.mark.gpu

FP32_MAX_ABS = 1e-4
FP32_MEAN_ABS = 1e-5


def _rand(shape, dtype, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _check(got, ref, dtype, what):
    assert got.dtype == dtype
    got = got.float().cpu()
    nan_ref = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan_ref), f"{what}: NaN rows differ"
    seen = ~nan_ref
    if dtype == torch.float32:
        assert_parity(got[seen], ref[seen], FP32_MAX_ABS, FP32_MEAN_ABS, what=what)
    else:
        assert_parity(got[seen], ref[seen], what=what)


def _run(device, q, k, v, cache=None, cache_len=0, bb=None, scale=None, causal=False):
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    got = ops.blockwise_causal_attention(dev(q), dev(k), dev(v), kv_cache=dev(cache),
                                         cache_len=cache_len, block_boundaries=dev(bb),
                                         softmax_scale=scale, causal=causal)
    ref = oatt.blockwise_causal_attention(q, k, v, cache, cache_len, bb, scale, causal,
                                          keep_fp32=True)
    return got, ref


def test_c0_native_fp32(device, built_lib):
    """C0, the reference's own CPU case (fp32, 4 heads, head dim 64, three
    16-token blocks), in fp32 on the GPU: no cast."""
    cfg = CONFIGS["C0"]
    inp = make_inputs(cfg)
    assert inp.q.dtype == torch.float32
    bb = torch.tensor(cfg.block_starts)
    got, ref = _run(device, inp.q, inp.k, inp.v, bb=bb)
    _check(got, ref, torch.float32, "C0 fp32")


@pytest.mark.parametrize("splits", [0, 1, 3, 8])
def test_c1_shape_fp32(device, built_lib, splits):
    """The Wan-5B decode chunk (83 queries over 1,245 cached + 83 keys, 24 heads,
    head dim 128) in fp32, with the planner's split count and forced ones."""
    q = _rand((1, 83, 24, 128), torch.float32, 1.0, 1)
    k = _rand((1, 83, 24, 128), torch.float32, 1.0, 2)
    v = _rand((1, 83, 24, 128), torch.float32, 1.0, 3)
    cache = _rand((2, 1, 1328, 24, 128), torch.float32, 1.0, 4)
    with _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
        got, ref = _run(device, q, k, v, cache, 1245)
    _check(got, ref, torch.float32, f"C1 fp32 splits={splits}")


MODES = ["cache", "causal", "blocks", "blocks_any", "cross"]
# (dtype, head dim) pairs the general kernel runs: fp32 at any head dim, 16-bit
# types at those the MFMA kernels do not take.
GENERAL = [(dt, d) for dt in (torch.float32, torch.bfloat16, torch.float16)
           for d in (16, 32, 64, 256) if dt == torch.float32 or d != 64]


@pytest.mark.parametrize("dtype,d", GENERAL,
                         ids=[f"{str(dt)[6:]}-D{d}" for dt, d in GENERAL])
@pytest.mark.parametrize("mode", MODES)
def test_head_dims_dtypes_masks(device, built_lib, dtype, d, mode):
    b, lq, h = 2, 77, 4
    lk = 130 if mode == "cross" else lq
    cache_len = 0 if mode in ("causal", "cross") else 200
    q = _rand((b, lq, h, d), dtype, 1.0, 11)
    k = _rand((b, lk, h, d), dtype, 1.0, 12)
    v = _rand((b, lk, h, d), dtype, 1.0, 13)
    cache = _rand((2, b, cache_len + 5, h, d), dtype, 1.0, 14) if cache_len else None
    bb = {"blocks": torch.tensor([0, 30, 64]),
          "blocks_any": torch.tensor([40, -60, 10, 70])}.get(mode)
    got, ref = _run(device, q, k, v, cache, cache_len, bb, causal=mode == "causal")
    _check(got, ref, dtype, f"{mode} D={d} {dtype}")


@pytest.mark.parametrize("cache_len", [0, 10])
def test_negative_block_start_on_short_cache_fp32(device, built_lib, cache_len):
    """[0, -40, 83] where cache_len + hi < 0: the reference's column stop wraps
    (ops/reference/attention.py:43-46); rows without a pair see no key (NaN)."""
    q = _rand((1, 83, 2, 64), torch.float32, 1.0, 21)
    k = _rand((1, 83, 2, 64), torch.float32, 1.0, 22)
    v = _rand((1, 83, 2, 64), torch.float32, 1.0, 23)
    cache = _rand((2, 1, 16, 2, 64), torch.float32, 1.0, 24) if cache_len else None
    got, ref = _run(device, q, k, v, cache, cache_len, torch.tensor([0, -40, 83]))
    _check(got, ref, torch.float32, f"[0,-40,83] cache_len={cache_len}")


def test_rows_without_keys_are_nan(device, built_lib):
    """Rows before the first block start, no cache: NaN (fp32 and at D=256)."""
    for dtype, d in ((torch.float32, 64), (torch.bfloat16, 256)):
        q = _rand((1, 48, 2, d), dtype, 1.0, 31)
        k = _rand((1, 48, 2, d), dtype, 1.0, 32)
        v = _rand((1, 48, 2, d), dtype, 1.0, 33)
        got, ref = _run(device, q, k, v, bb=torch.tensor([16, 32]))
        assert torch.isnan(got[:, :16].float()).all()
        _check(got, ref, dtype, f"NaN rows {dtype} D={d}")


@pytest.mark.parametrize("scale", [-0.09, 0.0, 0.5])
def test_scales_fp32(device, built_lib, scale):
    """Negative, zero (uniform weights over the visible keys) and large scales."""
    q = _rand((1, 40, 2, 32), torch.float32, 1.0, 41)
    k = _rand((1, 40, 2, 32), torch.float32, 1.0, 42)
    v = _rand((1, 40, 2, 32), torch.float32, 1.0, 43)
    cache = _rand((2, 1, 100, 2, 32), torch.float32, 1.0, 44)
    got, ref = _run(device, q, k, v, cache, 90, torch.tensor([0, 20]), scale=scale)
    _check(got, ref, torch.float32, f"scale={scale}")


def test_grouped_query_heads(device, built_lib):
    """8 query heads over 2 K/V heads, fp32 D=128 and bf16 D=256, with a cache."""
    for dtype, d in ((torch.float32, 128), (torch.bfloat16, 256)):
        q = _rand((1, 50, 8, d), dtype, 1.0, 51)
        k = _rand((1, 50, 2, d), dtype, 1.0, 52)
        v = _rand((1, 50, 2, d), dtype, 1.0, 53)
        cache = _rand((2, 1, 400, 2, d), dtype, 1.0, 54)
        got, ref = _run(device, q, k, v, cache, 333, torch.tensor([0, 25]))
        _check(got, ref, dtype, f"GQA {dtype} D={d}")


@pytest.mark.parametrize("splits", [1, 2, 5, 16])
def test_split_counts_d256(device, built_lib, splits):
    """A long cache at head dim 256 (bf16 and fp32) under forced split counts."""
    for dtype in (torch.bfloat16, torch.float32):
        q = _rand((1, 20, 2, 256), dtype, 0.5, 61)
        k = _rand((1, 20, 2, 256), dtype, 1.0, 62)
        v = _rand((1, 20, 2, 256), dtype, 1.0, 63)
        cache = _rand((2, 1, 3000, 2, 256), dtype, 1.0, 64)
        with _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
            got, ref = _run(device, q, k, v, cache, 2999)
        _check(got, ref, dtype, f"D=256 {dtype} splits={splits}")


def test_ragged_batch_fp32(device, built_lib):
    """Per-sequence cache lengths (varlen entry point), fp32 at head dim 64."""
    lens = [5, 300, 0, 1000]
    b, lq, h, d = 4, 16, 3, 64
    q = _rand((b, lq, h, d), torch.float32, 1.0, 71)
    k = _rand((b, lq, h, d), torch.float32, 1.0, 72)
    v = _rand((b, lq, h, d), torch.float32, 1.0, 73)
    cache = _rand((2, b, 1000, h, d), torch.float32, 1.0, 74)
    got = ops.blockwise_causal_attention_varlen(q.to(device), k.to(device), v.to(device),
                                                kv_cache=cache.to(device), cache_lens=lens,
                                                block_boundaries=torch.tensor([0], device=device))
    for i, c in enumerate(lens):
        ref = oatt.blockwise_causal_attention(q[i:i + 1], k[i:i + 1], v[i:i + 1],
                                              cache[:, i:i + 1], c, torch.tensor([0]), None,
                                              keep_fp32=True)
        _check(got[i:i + 1], ref, torch.float32, f"ragged seq {i} (cache {c})")


def test_device_cursor_fp32(device, built_lib):
    """cache_len read from device memory, clamped to the capacity, fp32."""
    q = _rand((1, 32, 2, 64), torch.float32, 1.0, 81)
    k = _rand((1, 32, 2, 64), torch.float32, 1.0, 82)
    v = _rand((1, 32, 2, 64), torch.float32, 1.0, 83)
    cache = _rand((2, 1, 512, 2, 64), torch.float32, 1.0, 84)
    for c in (0, 77, 512):
        cursor = torch.tensor([c], dtype=torch.int32, device=device)
        got = ops.blockwise_causal_attention(q.to(device), k.to(device), v.to(device),
                                             kv_cache=cache.to(device), cache_len=cursor)
        ref = oatt.blockwise_causal_attention(q, k, v, cache, c, None, None, keep_fp32=True)
        _check(got, ref, torch.float32, f"cursor {c}")


def test_general_kernel_leaves_the_counter_region_alone(device, built_lib):
    """The workspace's first 256 KiB are the arrival counters of the 16-bit
    kernels: zero before a call, zero after. A split call of the general kernel
    writes its partials after them and leaves them zero, and a bf16
    prefill-shaped call on the same workspace (whose key splits, merged in the
    launch, count arrivals there) still meets the bar."""
    dt32 = torch.float32
    q = _rand((1, 64, 4, 256), dt32, 1.0, 91)
    k = _rand((1, 64, 4, 256), dt32, 1.0, 92)
    v = _rand((1, 64, 4, 256), dt32, 1.0, 93)
    cache = _rand((2, 1, 2048, 4, 256), dt32, 1.0, 94)
    with _lib.tuning(_lib.TUNE_ATTN_SPLITS, 4):
        got, ref = _run(device, q, k, v, cache, 2048)
    _check(got, ref, dt32, "D=256 fp32 with 4 splits")
    ws = _lib.workspace(device, 1)
    torch.cuda.synchronize()
    assert ws is not None and not ws[: 256 << 10].any(), "counter region written"
    # A bf16 prefill-shaped call on the same workspace.
    qb = _rand((1, 300, 8, 128), torch.bfloat16, 1.0, 95)
    kb = _rand((1, 300, 8, 128), torch.bfloat16, 1.0, 96)
    vb = _rand((1, 300, 8, 128), torch.bfloat16, 1.0, 97)
    cb = _rand((2, 1, 2400, 8, 128), torch.bfloat16, 1.0, 98)
    gotb, refb = _run(device, qb, kb, vb, cb, 2400)
    _check(gotb, refb, torch.bfloat16, "bf16 after the general kernel")
