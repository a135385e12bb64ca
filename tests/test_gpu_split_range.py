"""Split-KV partials keep the reference's value range, and block lists in any
order give the reference's mask (MI355X).

The reference computes in fp32 from logits to output and casts once
(``python/dexter/ops/reference/attention.py:71-77``), so any finite bf16 V
gives a finite result. Here a split key range leaves a partial output in the
workspace as f16 values scaled by a per-row power of two, with the exponent
beside the row's (max, sum). Attention is linear in V, and scaling V by a
power of two is exact in bf16, f16 and fp32 alike, so the output for V * 2^k
must be the output for V times 2^k bit for bit, on every path and split
count, for |V| well above the f16 range (2^17: entries near 1e5) and well
below its normal range (2^-20: near 1e-6). Each call is also compared with
the oracle on the same scaled inputs, the north-star bar scaled by 2^k.

Block lists: the reference's mask is the union over consecutive pairs
(starts[i], starts[i+1]) in the order given, Python slicing rules included
(``ops/reference/attention.py:43-46``); unsorted and negative entries are
checked against the oracle on every kernel.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.ops.gfx950 import _lib
from oracle import attention as oatt

from _util import MAX_ABS, MEAN_ABS, assert_parity

pytestmark = pytest.mark.gpu
DT = torch.bfloat16

# (name, TUNE_ATTN_KERNEL, TUNE_ATTN_MERGE): planner default (dual-stream
# kernel + merge kernel for decode shapes), the one-launch decode kernel
# (merging through the L2 where its splits share an XCD), the decode kernel
# merging at device scope only, and the single-stream and paired-group kernels.
PATHS = [("default", 0, 0), ("decode", 4, 1), ("decode-device", 4, 2), ("single", 1, 0),
         ("paired", 3, 0)]


def _rand(shape, device, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(DT).to(device)


def _oracle(q, k, v, cache, cache_len, bb=None):
    return oatt.blockwise_causal_attention(
        q.cpu(), k.cpu(), v.cpu(), None if cache is None else cache.cpu(), cache_len,
        None if bb is None else bb.cpu(), None, False, keep_fp32=True)


def _scaled(v, cache, k2):
    f = 2.0 ** k2
    vs = (v.float() * f).to(DT)
    cs = None
    if cache is not None:
        cs = cache.clone()
        cs[1] = (cache[1].float() * f).to(DT)
    return vs, cs


def _check_scaled(got, base, ref, k2, what):
    f = 2.0 ** k2
    g = got.float().cpu()
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    assert torch.equal(got, (base.float() * f).to(DT)), f"{what}: not base * 2^{k2} bit for bit"
    d = (g - ref).abs()
    assert d.max().item() <= MAX_ABS * f and d.mean().item() <= MEAN_ABS * f, (
        f"{what}: max-abs {d.max().item():.3e} (<= {MAX_ABS * f:.3e}), "
        f"mean-abs {d.mean().item():.3e}")


@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
@pytest.mark.parametrize("splits", [0, 2, 5, 8, 16])
def test_decode_chunk_partials_keep_range(device, built_lib, path, splits):
    """C1's shape (83 queries over 1245 cached + 83 new keys, 24 heads)."""
    name, kernel, merge = path
    b, l, h, d, c = 1, 83, 24, 128, 1245
    q, k, v = (_rand((b, l, h, d), device, seed=300 + i) for i in range(3))
    cache = _rand((2, b, c + l, h, d), device, seed=303)
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge), \
            _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
        base = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)
        for k2 in (17, -20):
            vs, cs = _scaled(v, cache, k2)
            got = ops.blockwise_causal_attention(q, k, vs, kv_cache=cs, cache_len=c)
            torch.cuda.synchronize()
            _check_scaled(got, base, _oracle(q, k, vs, cs, c), k2,
                          f"{name} splits={splits} V*2^{k2}")


@pytest.mark.parametrize("path", PATHS[:3], ids=[p[0] for p in PATHS[:3]])
def test_cross_attention_partials_keep_range(device, built_lib, path):
    """83 queries over 512 keys, no cache and no mask (split on every path)."""
    name, kernel, merge = path
    q = _rand((1, 83, 24, 128), device, seed=310)
    k, v = _rand((1, 512, 24, 128), device, seed=311), _rand((1, 512, 24, 128), device, seed=312)
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge):
        for splits in (2, 4, 8):
            with _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
                base = ops.blockwise_causal_attention(q, k, v)
                for k2 in (17, -20):
                    vs, _ = _scaled(v, None, k2)
                    got = ops.blockwise_causal_attention(q, k, vs)
                    torch.cuda.synchronize()
                    _check_scaled(got, base, _oracle(q, k, vs, None, 0), k2,
                                  f"{name} cross splits={splits} V*2^{k2}")


@pytest.mark.parametrize("path", PATHS[:3], ids=[p[0] for p in PATHS[:3]])
def test_ragged_batch_partials_keep_range(device, built_lib, path):
    """The C4 ragged batch's lengths (0, 332, 1245, 3237 cached keys), 99-token
    chunks in blocks [0, 83), [83, 99), 8 heads."""
    name, kernel, merge = path
    lens = [0, 332, 1245, 3237]
    h, d = 8, 128
    q, k, v = (_rand((4, 99, h, d), device, seed=320 + i) for i in range(3))
    cache = _rand((2, 4, max(lens), h, d), device, seed=323)
    bb = torch.tensor([0, 83], dtype=torch.int32, device=device)
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge):
        base = ops.blockwise_causal_attention_varlen(q, k, v, kv_cache=cache, cache_lens=lens,
                                                     block_boundaries=bb)
        for k2 in (17, -20):
            vs, cs = _scaled(v, cache, k2)
            got = ops.blockwise_causal_attention_varlen(q, k, vs, kv_cache=cs, cache_lens=lens,
                                                        block_boundaries=bb)
            torch.cuda.synchronize()
            for i, c in enumerate(lens):
                _check_scaled(got[i:i + 1], base[i:i + 1],
                              _oracle(q[i:i + 1], k[i:i + 1], vs[i:i + 1], cs[:, i:i + 1], c, bb),
                              k2, f"{name} seq {i} (cache {c}) V*2^{k2}")


BLOCK_LISTS = [[0, 50, 30], [40, 0, 83], [30, 0, 60, 10], [0, -40, 83], [50, 20], [0, 83, 20, 60]]


@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
@pytest.mark.parametrize("blocks", BLOCK_LISTS, ids=[str(b) for b in BLOCK_LISTS])
def test_unordered_block_lists_match_reference(device, built_lib, path, blocks):
    """83 queries over 300 cached + 83 new keys: unsorted, overlapping and
    negative block starts give the reference's union mask on every kernel."""
    name, kernel, merge = path
    b, l, h, d, c = 1, 83, 8, 128, 300
    q, k, v = (_rand((b, l, h, d), device, seed=330 + i) for i in range(3))
    cache = _rand((2, b, c + l, h, d), device, seed=333)
    bb = torch.tensor(blocks, dtype=torch.int32, device=device)
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge):
        got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c, block_boundaries=bb)
    torch.cuda.synchronize()
    assert_parity(got, _oracle(q, k, v, cache, c, bb), what=f"{name} blocks {blocks}")


SHORT_CACHE_LISTS = [[0, -40, 83], [0, -82, 83], [0, -60, 30, -70], [50, 20], [-90, 10]]


@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
@pytest.mark.parametrize("cache_len", [0, 10, 39])
@pytest.mark.parametrize("blocks", SHORT_CACHE_LISTS, ids=[str(b) for b in SHORT_CACHE_LISTS])
def test_negative_starts_on_short_caches(device, built_lib, path, cache_len, blocks):
    """Negative starts whose column stop ``cache_len + hi`` falls below zero:
    the reference's slice then counts from the end of the key axis
    (``ops/reference/attention.py:45``), so those rows see current keys
    ``[0, cache_len + 83 + hi)``. Rows that see no key are NaN in both (the
    reference's softmax over an all ``-inf`` row); the rest meet the bar."""
    name, kernel, merge = path
    b, l, h, d = 1, 83, 8, 128
    q, k, v = (_rand((b, l, h, d), device, seed=340 + i) for i in range(3))
    cache = _rand((2, b, cache_len + l, h, d), device, seed=343) if cache_len else None
    bb = torch.tensor(blocks, dtype=torch.int64, device=device)
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge):
        got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len,
                                             block_boundaries=bb)
    torch.cuda.synchronize()
    ref = _oracle(q, k, v, cache, cache_len, bb)
    g = got.float().cpu()
    nan_ref = torch.isnan(ref)
    assert torch.equal(torch.isnan(g), nan_ref), f"{name} {blocks} cache {cache_len}: NaN rows differ"
    keep = ~nan_ref.all(dim=-1).all(dim=-1).squeeze(0)
    assert keep.any()
    assert_parity(got[:, keep], ref[:, keep], what=f"{name} blocks {blocks} cache {cache_len}")


@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
@pytest.mark.parametrize("q_len,k_len,cache_len", [(1, 1, 0), (1, 100, 0), (1, 83, 300),
                                                   (2, 1, 0), (33, 70, 0)])
def test_few_query_rows(device, built_lib, path, q_len, k_len, cache_len):
    """One-row (and few-row) queries on every kernel. The op passes stride 0 for a
    size-1 dim, so a kernel that moves whole row blocks (Q into LDS, results out of
    it) must bound them by the row count, not by the stride: with stride 0, every
    row past the first aliases it (a one-row call once came back NaN)."""
    _, kern, merge = path
    q = _rand((2, q_len, 3, 128), device, seed=30)
    k = _rand((2, k_len, 3, 128), device, seed=31)
    v = _rand((2, k_len, 3, 128), device, seed=32)
    cache = _rand((2, 2, cache_len + k_len, 3, 128), device, seed=33) if cache_len else None
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kern), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge):
        got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len)
    ref = _oracle(q, k, v, cache, cache_len)
    assert_parity(got, ref, what=f"{path[0]} q={q_len} k={k_len} cache={cache_len}")
