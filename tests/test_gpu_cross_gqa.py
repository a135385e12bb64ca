"""Cross-attention and grouped-query attention through the HIP attention kernels (MI355X).

* Cross-attention: ``k``/``v`` of another length than ``q``, no mask: every key
  visible. The DiT's ``CrossAttention`` calls the op so for the text (512
  tokens) and CLIP image (257 tokens) conditioning of a chunk
  (``models/dreamzero/model.py:234-241``).
* Grouped-query attention: ``k``/``v`` (and the cache) with fewer heads;
  query head ``h`` reads K/V head ``h // (H/Hkv)``, GR00T's Qwen3 layout
  (16 query heads over 8 K/V heads, ``vla/groot/backbone.py:100-114``).

Parity bar as for self-attention: max-abs <= 2e-2 and mean-abs <= 2e-3 against
the fp32 oracle. The grouped kernels must also equal, bit for bit, the same
kernels run on K/V materialised with ``repeat_interleave``: the grouping only
changes which head's rows a workgroup reads.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from oracle import attention as oatt

from _util import assert_parity, close_rel

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _rand(shape, device, dtype=DT, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def _oracle(q, k, v, cache=None, cache_len=0, bb=None, causal=False):
    return oatt.blockwise_causal_attention(
        q.cpu(), k.cpu(), v.cpu(), None if cache is None else cache.cpu(), cache_len,
        None if bb is None else bb.cpu(), None, causal, keep_fp32=True)


def _equal_nan(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(torch.nan_to_num(a.float(), nan=7.0), torch.nan_to_num(b.float(), nan=7.0))


# ------------------------------------------------------------ cross-attention -----

@pytest.mark.parametrize("ctx", [512, 257])
def test_wan5b_cross_attention(device, built_lib, ctx):
    """The 83-token chunk against the text (512) and CLIP (257) context of Wan-5B."""
    q = _rand((1, 83, 24, 128), device, scale=0.3, seed=1)
    k = _rand((1, ctx, 24, 128), device, seed=2)
    v = _rand((1, ctx, 24, 128), device, seed=3)
    got = ops.blockwise_causal_attention(q, k, v)
    ref = _oracle(q, k, v)
    assert got.shape == q.shape and got.dtype == DT
    assert_parity(got, ref, what=f"ctx={ctx}")
    close_rel(got, ref, tol=3e-2)


def test_cross_attention_block_sum_like_the_model(device, built_lib):
    """CrossAttention.forward: text attention plus image attention with one query."""
    q = _rand((1, 83, 24, 128), device, scale=0.3, seed=4)
    kt, vt = _rand((1, 512, 24, 128), device, seed=5), _rand((1, 512, 24, 128), device, seed=6)
    ki, vi = _rand((1, 257, 24, 128), device, seed=7), _rand((1, 257, 24, 128), device, seed=8)
    got = ops.blockwise_causal_attention(q, kt, vt).float() + \
        ops.blockwise_causal_attention(q, ki, vi).float()
    ref = _oracle(q, kt, vt) + _oracle(q, ki, vi)
    assert_parity(got, ref, max_abs=4e-2, mean_abs=4e-3, what="text + image")


@pytest.mark.parametrize("lq,lk,d,dtype", [
    (83, 1, 128, DT), (83, 64, 128, DT), (83, 65, 64, DT), (83, 2048, 128, torch.float16),
    (300, 77, 128, DT), (1024, 512, 128, DT), (2048, 257, 64, torch.float16), (7, 8192, 128, DT),
])
def test_cross_attention_shapes(device, built_lib, lq, lk, d, dtype):
    """Short and long contexts, fewer keys than queries, both head dims and dtypes:
    the decode (split-KV) and prefill (paired-group) kernels both take these."""
    b, h = 2, 4
    q = _rand((b, lq, h, d), device, dtype, scale=0.3, seed=lq)
    k = _rand((b, lk, h, d), device, dtype, seed=lk)
    v = _rand((b, lk, h, d), device, dtype, seed=lk + 1)
    got = ops.blockwise_causal_attention(q, k, v)
    assert_parity(got, _oracle(q, k, v), what=f"lq={lq} lk={lk} d={d}")


def test_cross_attention_with_cache(device, built_lib):
    """A cache in front of a context of another length: all cache_len + Lk keys visible."""
    q = _rand((1, 83, 8, 128), device, scale=0.3, seed=11)
    k = _rand((1, 200, 8, 128), device, seed=12)
    v = _rand((1, 200, 8, 128), device, seed=13)
    cache = _rand((2, 1, 300, 8, 128), device, scale=0.3, seed=14)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=250)
    assert_parity(got, _oracle(q, k, v, cache, 250))


def test_cross_attention_refuses_a_mask(device, built_lib):
    q = _rand((1, 16, 2, 128), device)
    k = _rand((1, 24, 2, 128), device)
    with pytest.raises(ValueError, match="must equal q length"):
        ops.blockwise_causal_attention(q, k, k, causal=True)
    with pytest.raises(ValueError, match="must equal q length"):
        ops.blockwise_causal_attention(q, k, k, block_boundaries=torch.tensor([0, 8], device=device))
    with pytest.raises(ValueError, match="no keys"):
        ops.blockwise_causal_attention(q, k[:, :0], k[:, :0])


# ------------------------------------------------------------------------ GQA -----

@pytest.mark.parametrize("hkv", [8, 4, 1])
def test_groot_gqa_causal(device, built_lib, hkv):
    """GR00T's Qwen3 attention: 16 query heads, causal, over 8 (or 4, or 1) K/V heads."""
    b, l, h, d = 1, 300, 16, 128
    q = _rand((b, l, h, d), device, scale=0.3, seed=21)
    k = _rand((b, l, hkv, d), device, seed=22)
    v = _rand((b, l, hkv, d), device, seed=23)
    got = ops.blockwise_causal_attention(q, k, v, causal=True)
    assert_parity(got, _oracle(q, k, v, causal=True), what=f"hkv={hkv}")
    r = h // hkv
    full = ops.blockwise_causal_attention(q, k.repeat_interleave(r, dim=2).contiguous(),
                                          v.repeat_interleave(r, dim=2).contiguous(), causal=True)
    assert torch.equal(got, full), "grouped K/V differ from the materialised expansion"


@pytest.mark.parametrize("case", ["decode_cache", "blocks", "prefill", "cross", "decode_long",
                                  "chunk_long"])
def test_gqa_paths_equal_the_expansion(device, built_lib, case):
    """Every kernel path with grouped K/V against the same path on expanded K/V
    (bit-exact) and the oracle (parity)."""
    h, hkv, d = 24, 6, 128
    r = h // hkv
    cache, cache_len, bb, lk = None, 0, None, None
    if case == "decode_cache":
        lq, cache_len = 83, 1245
        cache = _rand((2, 1, 1328, hkv, d), device, scale=0.5, seed=31)
    elif case == "decode_long":  # one query over 32,749 cached keys: 16 splits
        lq, cache_len = 1, 32749
        cache = _rand((2, 1, cache_len + lq, hkv, d), device, scale=0.5, seed=35)
    elif case == "chunk_long":  # a 512-query chunk over 12,001 cached keys
        lq, cache_len = 512, 12001
        cache = _rand((2, 1, cache_len + lq, hkv, d), device, scale=0.5, seed=36)
    elif case == "blocks":
        lq = 512
        bb = torch.tensor([0, 128, 256, 384], device=device)
    elif case == "prefill":
        lq = 2048
        bb = torch.arange(0, 2048, 512, device=device)
    else:
        lq, lk = 83, 512
    lk = lk or lq
    q = _rand((1, lq, h, d), device, scale=0.3, seed=32)
    k = _rand((1, lk, hkv, d), device, seed=33)
    v = _rand((1, lk, hkv, d), device, seed=34)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len,
                                         block_boundaries=bb)
    ex = lambda t, dim: t.repeat_interleave(r, dim=dim).contiguous()  # noqa: E731
    full = ops.blockwise_causal_attention(q, ex(k, 2), ex(v, 2),
                                          kv_cache=None if cache is None else ex(cache, 3),
                                          cache_len=cache_len, block_boundaries=bb)
    assert _equal_nan(got, full), f"{case}: grouped K/V differ from the expansion"
    assert_parity(got, _oracle(q, k, v, cache, cache_len, bb), what=case)


def test_gqa_varlen(device, built_lib):
    """The ragged-batch entry point with grouped K/V: equal to one call per sequence."""
    h, hkv, d, lq = 8, 2, 128, 48
    lens = [0, 100, 333]
    cache = _rand((2, 3, 400, hkv, d), device, scale=0.5, seed=41)
    q = _rand((3, lq, h, d), device, scale=0.3, seed=42)
    k = _rand((3, lq, hkv, d), device, seed=43)
    v = _rand((3, lq, hkv, d), device, seed=44)
    bb = torch.tensor([0, 16, 32], device=device)
    got = ops.blockwise_causal_attention_varlen(q, k, v, kv_cache=cache, cache_lens=lens,
                                                block_boundaries=bb)
    for i, c in enumerate(lens):
        one = ops.blockwise_causal_attention(q[i:i + 1], k[i:i + 1], v[i:i + 1],
                                             kv_cache=cache[:, i:i + 1].contiguous(),
                                             cache_len=c, block_boundaries=bb)
        ref = _oracle(q[i:i + 1], k[i:i + 1], v[i:i + 1], cache[:, i:i + 1], c, bb)
        assert_parity(got[i:i + 1], ref, what=f"seq {i}")
        assert_parity(one, ref, what=f"seq {i} alone")


def test_gqa_rejects_indivisible_heads(device, built_lib):
    q = _rand((1, 16, 6, 128), device)
    k = _rand((1, 16, 4, 128), device)
    with pytest.raises(LookupError):
        ops.blockwise_causal_attention(q, k, k)  # no implementation accepts 6 over 4 heads
