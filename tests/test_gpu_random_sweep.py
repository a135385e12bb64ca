"""Seeded random sweep of the attention op against the oracle (MI355X).

Thirty configurations drawn once from a fixed seed. Each mixes:
* batch, query count (1-160) and cache length (0-2,049);
* query and K/V heads (grouped-query included), head_dim 64/128, bf16/f16;
* a softmax scale that may be custom or negative;
* a mask mode:
  * none;
  * causal;
  * ascending block starts;
  * block starts in any order with negative entries;
  * cross-attention onto another key count.

Every configuration goes through the registry and the C ABI and is compared with
``oracle/attention.py`` (ref ``ops/reference/attention.py:22-77``). Rows that see no key are
NaN in both: the reference's softmax of an all ``-inf`` row. The other rows meet the parity
bar. The point is breadth: shapes and combinations that the targeted tests do not pin one by
one, such as odd row counts over partial tiles, splits of short caches, and grouped K/V under
block lists.
"""

from __future__ import annotations

import random

import pytest
import torch

import dexter_amd.ops as ops
from oracle import attention as oatt

from _util import assert_parity

pytestmark = pytest.mark.gpu


def _cases(n=30, seed=2026):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        h = rng.choice([1, 2, 4, 8])
        mode = rng.choice(["none", "causal", "blocks", "blocks_any", "cross"])
        out.append(dict(
            idx=i,
            b=rng.choice([1, 2]),
            lq=rng.choice([1, 7, 32, 83, 99, 128, 160]),
            cache=rng.choice([0, 5, 64, 333, 1245, 2049]) if mode != "cross" or rng.random() < 0.5
            else 0,
            h=h,
            hkv=rng.choice([x for x in (1, 2, 4, 8) if h % x == 0]),
            d=rng.choice([64, 128]),
            dtype=rng.choice([torch.bfloat16, torch.float16]),
            scale=rng.choice([None, None, 0.05, -0.09]),
            mode=mode,
            lk=rng.choice([1, 77, 257]),
            seed=rng.randrange(1 << 30),
        ))
    return out


CASES = _cases()


def _blocks(rng, lq, mode):
    if mode == "blocks":
        cuts = sorted(rng.sample(range(1, lq), min(3, lq - 1))) if lq > 1 else []
        return [0] + cuts
    starts = [rng.randrange(-lq, lq + 1) for _ in range(rng.randint(2, 5))]
    return starts


@pytest.mark.parametrize("case", CASES, ids=[
    f"{c['idx']}-{c['mode']}-b{c['b']}q{c['lq']}c{c['cache']}h{c['h']}/{c['hkv']}d{c['d']}"
    f"{'bf' if c['dtype'] == torch.bfloat16 else 'f'}" for c in CASES])
def test_random_configuration(device, built_lib, case):
    c = case
    g = torch.Generator().manual_seed(c["seed"])
    rng = random.Random(c["seed"])
    b, lq, h, hkv, d, dt = c["b"], c["lq"], c["h"], c["hkv"], c["d"], c["dtype"]
    lk = c["lk"] if c["mode"] == "cross" else lq
    cache_len = c["cache"]
    q = (torch.randn(b, lq, h, d, generator=g) * 0.5).to(dt)
    k = torch.randn(b, lk, hkv, d, generator=g).to(dt)
    v = torch.randn(b, lk, hkv, d, generator=g).to(dt)
    cache = (torch.randn(2, b, cache_len + 3, hkv, d, generator=g).to(dt)
             if cache_len else None)
    bb = None
    if c["mode"] in ("blocks", "blocks_any"):
        bb = torch.tensor(_blocks(rng, lq, c["mode"]), dtype=torch.int64)
    causal = c["mode"] == "causal"
    ref = oatt.blockwise_causal_attention(q, k, v, cache, cache_len, bb, c["scale"], causal,
                                          keep_fp32=True)
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    got = ops.blockwise_causal_attention(dev(q), dev(k), dev(v), kv_cache=dev(cache),
                                         cache_len=cache_len, block_boundaries=dev(bb),
                                         softmax_scale=c["scale"], causal=causal)
    assert got.shape == q.shape and got.dtype == dt
    got = got.float().cpu()
    nan_ref = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan_ref), f"case {c['idx']}: NaN rows differ ({bb})"
    seen = ~nan_ref
    assert_parity(got[seen], ref[seen], what=f"case {c['idx']} blocks={None if bb is None else bb.tolist()}")


# A second sweep over what the first leaves out: fp32 inputs and head dims 16,
# 32 and 256 (the general kernel), and prefill-sized query counts (the paired
# kernel, its key splits and in-launch merges). fp32 calls meet a bar ten times
# tighter on max-abs and a hundred times on mean-abs: rounding any operand to
# 16 bits would fail it.
FP32_MAX_ABS, FP32_MEAN_ABS = 2e-3, 2e-5


def _cases_wide(n=24, seed=3035):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        h = rng.choice([1, 2, 4, 6])
        mode = rng.choice(["none", "causal", "blocks", "blocks_any", "cross"])
        dt = rng.choice([torch.float32, torch.bfloat16, torch.float16])
        out.append(dict(
            idx=i,
            b=rng.choice([1, 2]),
            lq=rng.choice([1, 19, 83, 200, 333, 600]),
            cache=rng.choice([0, 17, 300, 1100]) if mode != "cross" else 0,
            h=h,
            hkv=rng.choice([x for x in (1, 2, 3, 6) if h % x == 0]),
            d=rng.choice([16, 32, 64, 128, 256]),
            dtype=dt,
            scale=rng.choice([None, None, 0.07, -0.05]),
            mode=mode,
            lk=rng.choice([1, 64, 300]),
            seed=rng.randrange(1 << 30),
        ))
    return out


CASES_WIDE = _cases_wide()


@pytest.mark.parametrize("case", CASES_WIDE, ids=[
    f"w{c['idx']}-{c['mode']}-b{c['b']}q{c['lq']}c{c['cache']}h{c['h']}k{c['hkv']}d{c['d']}"
    f"{ {torch.float32: 'f32', torch.bfloat16: 'bf', torch.float16: 'f'}[c['dtype']] }"
    for c in CASES_WIDE])
def test_random_configuration_wide(device, built_lib, case):
    c = case
    g = torch.Generator().manual_seed(c["seed"])
    rng = random.Random(c["seed"])
    b, lq, h, hkv, d, dt = c["b"], c["lq"], c["h"], c["hkv"], c["d"], c["dtype"]
    lk = c["lk"] if c["mode"] == "cross" else lq
    cache_len = c["cache"]
    q = (torch.randn(b, lq, h, d, generator=g) * 0.5).to(dt)
    k = torch.randn(b, lk, hkv, d, generator=g).to(dt)
    v = torch.randn(b, lk, hkv, d, generator=g).to(dt)
    cache = (torch.randn(2, b, cache_len + 5, hkv, d, generator=g).to(dt)
             if cache_len else None)
    bb = None
    if c["mode"] in ("blocks", "blocks_any"):
        bb = torch.tensor(_blocks(rng, lq, c["mode"]), dtype=torch.int64)
    causal = c["mode"] == "causal"
    ref = oatt.blockwise_causal_attention(q, k, v, cache, cache_len, bb, c["scale"], causal,
                                          keep_fp32=True)
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    got = ops.blockwise_causal_attention(dev(q), dev(k), dev(v), kv_cache=dev(cache),
                                         cache_len=cache_len, block_boundaries=dev(bb),
                                         softmax_scale=c["scale"], causal=causal)
    assert got.shape == q.shape and got.dtype == dt
    got = got.float().cpu()
    nan_ref = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan_ref), f"case w{c['idx']}: NaN rows differ ({bb})"
    seen = ~nan_ref
    what = f"case w{c['idx']} blocks={None if bb is None else bb.tolist()}"
    if dt == torch.float32:
        assert_parity(got[seen], ref[seen], FP32_MAX_ABS, FP32_MEAN_ABS, what=what)
    else:
        assert_parity(got[seen], ref[seen], what=what)
