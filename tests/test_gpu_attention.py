"""HIP blockwise-causal attention against the oracle (MI355X).

The first three tests restate the reference suite's attention tests
(``test/test_ops.py:93-103, 118-135, 166-181``) with the oracle in place of
the REFERENCE spec; the rest widen coverage: both MFMA dtypes and head dims,
ragged tile edges, split-KV, strided inputs, fully masked rows, bit-exact
future invisibility, and the ragged-batch entry point.

Parity bar (bf16/f16 kernel vs fp32 oracle on identical inputs): max-abs
<= 2e-2, mean-abs <= 2e-3; the reference's own relative check (3e-2) too.
"""

from __future__ import annotations

import math

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.ops.gfx950 import _lib
from dexter_amd.registry import select_spec
from oracle import attention as oatt

from _util import assert_parity, close_rel

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _oracle(q, k, v, cache, cache_len, bb, scale=None, causal=False):
    return oatt.blockwise_causal_attention(
        q.cpu(), k.cpu(), v.cpu(), None if cache is None else cache.cpu(), cache_len,
        None if bb is None else bb.cpu(), scale, causal, keep_fp32=True)


def _rand(shape, device, dtype=DT, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def test_selected_kernel_is_hip(device, built_lib):
    q = torch.zeros(1, 8, 2, 128, dtype=DT, device=device)
    assert select_spec("attention", "blockwise_causal", q, q, q).name == "hip_blockwise_causal_gfx950"


@pytest.mark.parametrize("cache_len", [0, 256])
@pytest.mark.parametrize("blocks", [None, [0, 50, 100]])
def test_attention(device, built_lib, cache_len, blocks):
    b, l, h, d = 1, 125, 24, 128
    q = _rand((b, l, h, d), device, scale=0.3, seed=1)
    k = _rand((b, l, h, d), device, seed=2)
    v = _rand((b, l, h, d), device, seed=3)
    cache = _rand((2, b, 512, h, d), device, scale=0.3, seed=4) if cache_len else None
    bb = torch.tensor(blocks, device=device) if blocks else None
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len,
                                         block_boundaries=bb)
    ref = _oracle(q, k, v, cache, cache_len, bb)
    assert got.dtype == DT and got.shape == q.shape
    assert_parity(got, ref, what=f"cache_len={cache_len} blocks={blocks}")
    close_rel(got, ref, tol=3e-2)


@pytest.mark.parametrize("scale", [1.0, 60.0])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_attention_survives_extreme_scores(device, built_lib, scale, sign):
    b, l, h, d = 1, 96, 4, 128
    q = torch.full((b, l, h, d), sign * scale, device=device, dtype=DT)
    k = torch.full((b, l, h, d), scale, device=device, dtype=DT)
    v = _rand((b, l, h, d), device, seed=5)
    bb = torch.tensor([0, 48], device=device)
    got = ops.blockwise_causal_attention(q, k, v, block_boundaries=bb)
    assert torch.isfinite(got.float()).all(), "attention produced non-finite output"
    ref = _oracle(q, k, v, None, 0, bb)
    assert_parity(got, ref)
    close_rel(got, ref, tol=3e-2)


@pytest.mark.parametrize("cache_len", [0, 32])
def test_attention_causal_matches_reference(device, built_lib, cache_len):
    b, l, h, d = 1, 64, 4, 128
    q = _rand((b, l, h, d), device, scale=0.3, seed=6)
    k = _rand((b, l, h, d), device, scale=0.3, seed=7)
    v = _rand((b, l, h, d), device, scale=0.3, seed=8)
    cache = _rand((2, b, 128, h, d), device, scale=0.3, seed=9) if cache_len else None
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len, causal=True)
    ref = _oracle(q, k, v, cache, cache_len, None, causal=True)
    assert_parity(got, ref)
    # A causal query must not see the future: bumping the last key changes only
    # the last row -- bit-exactly here, not just within a tolerance.
    k2 = k.clone()
    k2[:, -1] += 5.0
    other = ops.blockwise_causal_attention(q, k2, v, kv_cache=cache, cache_len=cache_len,
                                           causal=True)
    assert torch.equal(got[:, :-1], other[:, :-1])
    assert not torch.equal(got[:, -1:], other[:, -1:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("q_len,cache_len,blocks", [
    (1, 0, None), (31, 0, [0, 7, 19]), (83, 1245, None), (99, 332, [0, 83]),
    (130, 63, [0, 64, 65]), (200, 1, [0, 100]), (257, 0, None),
])
def test_shapes_and_dtypes(device, built_lib, dtype, d, q_len, cache_len, blocks):
    b, h = 2, 3
    q = _rand((b, q_len, h, d), device, dtype, seed=10)
    k = _rand((b, q_len, h, d), device, dtype, seed=11)
    v = _rand((b, q_len, h, d), device, dtype, seed=12)
    cache = _rand((2, b, cache_len + 5, h, d), device, dtype, seed=13) if cache_len else None
    bb = torch.tensor(blocks, device=device, dtype=torch.int64) if blocks else None
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len,
                                         block_boundaries=bb)
    ref = _oracle(q, k, v, cache, cache_len, bb)
    assert got.dtype == dtype
    assert_parity(got, ref, what=f"{dtype} d={d} q={q_len} cache={cache_len} blocks={blocks}")


def test_explicit_scale_and_strided_inputs(device, built_lib):
    b, l, h, d = 2, 70, 4, 128
    base = _rand((b, h, l, d), device, seed=14)           # [B, H, L, D] storage
    q = base.transpose(1, 2)                              # strided [B, L, H, D] view
    k = _rand((b, l, h, d), device, seed=15)
    v = _rand((b, l, 2 * h, d), device, seed=16)[:, :, ::2]  # head stride 2*D
    got = ops.blockwise_causal_attention(q, k, v, softmax_scale=0.05,
                                         block_boundaries=torch.tensor([0, 30], device=device))
    ref = _oracle(q, k, v, None, 0, torch.tensor([0, 30]), scale=0.05)
    assert_parity(got, ref)


def test_split_kv_decode_shape(device, built_lib):
    """The Wan-5B chunk shape: 83 queries over 1245 cached + 83 new keys (split-KV path)."""
    b, l, h, d, cache_len = 1, 83, 24, 128, 1245
    q = _rand((b, l, h, d), device, seed=17)
    k = _rand((b, l, h, d), device, seed=18)
    v = _rand((b, l, h, d), device, seed=19)
    cache = _rand((2, b, 1328, h, d), device, seed=20)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len)
    ref = _oracle(q, k, v, cache, cache_len, None)
    assert_parity(got, ref)


def test_head_major_cache_matches_contiguous_bit_exact(device, built_lib):
    """A cache stored [2, B, H, S, D] and viewed as [2, B, S, H, D] is read
    through its strides, with results identical to the contiguous layout."""
    b, l, h, d, cache_len = 2, 83, 24, 128, 1245
    q, k, v = (_rand((b, l, h, d), device, seed=s) for s in (43, 44, 45))
    dense = _rand((2, b, cache_len + l, h, d), device, seed=46)
    hm = torch.zeros(2, b, h, cache_len + l, d, device=device, dtype=DT).permute(0, 1, 3, 2, 4)
    hm.copy_(dense)
    assert not hm.is_contiguous() and hm.stride(2) == d
    a = ops.blockwise_causal_attention(q, k, v, kv_cache=dense, cache_len=cache_len)
    c = ops.blockwise_causal_attention(q, k, v, kv_cache=hm, cache_len=cache_len)
    assert torch.equal(a, c)
    assert_parity(c, _oracle(q, k, v, dense, cache_len, None))


def _decode_case(device, seed=50):
    b, l, h, d, cache_len = 1, 83, 24, 128, 1245
    q, k, v = (_rand((b, l, h, d), device, seed=seed + i) for i in range(3))
    cache = _rand((2, b, cache_len + l, h, d), device, seed=seed + 3)
    return q, k, v, cache, cache_len


@pytest.mark.parametrize("splits", [2, 3, 7, 16])
def test_split_kv_any_split_count(device, built_lib, splits):
    """The merge of split-KV partials for 2..16 splits (16 is the maximum; the
    one-launch decode kernel takes up to 8, more go to the separate merge
    kernel) against the oracle, and bit-identical on a second call."""
    q, k, v, cache, c = _decode_case(device)
    with _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
        got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)
        again = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)
    assert torch.equal(got, again)
    assert_parity(got, _oracle(q, k, v, cache, c, None), what=f"{splits} splits")


def test_split_kv_graph_replays_match_eager(device, built_lib):
    """A captured decode call replayed several times, with other split-KV work
    (a ragged batch) run eagerly between replays: every replay equals the
    eager result bit for bit."""
    q, k, v, cache, c = _decode_case(device)
    eager = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)
    lens = [83, 1245, 415]
    qv, kv_, vv = (_rand((3, 99, 8, 128), device, seed=60 + i) for i in range(3))
    cv = _rand((2, 3, 1245, 8, 128), device, seed=63)
    other_ref = ops.blockwise_causal_attention_varlen(qv, kv_, vv, kv_cache=cv, cache_lens=lens)
    out = {}
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):  # warm the capture stream's workspace outside capture
        ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out["o"] = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out["o"], eager), f"replay {i}"
        other = ops.blockwise_causal_attention_varlen(qv, kv_, vv, kv_cache=cv, cache_lens=lens)
        torch.cuda.synchronize()
        assert torch.equal(other, other_ref)


def test_rows_before_the_first_block_match_the_reference(device, built_lib):
    """Rows before block_boundaries[0] see only the cache; with no cache they are NaN."""
    b, l, h, d = 1, 40, 2, 64
    q, k, v = (_rand((b, l, h, d), device, seed=s) for s in (21, 22, 23))
    bb = torch.tensor([8, 20], device=device)
    got = ops.blockwise_causal_attention(q, k, v, block_boundaries=bb)
    ref = _oracle(q, k, v, None, 0, bb)
    assert torch.isnan(got[:, :8].float()).all() and torch.isnan(ref[:, :8]).all()
    assert_parity(got[:, 8:], ref[:, 8:])
    cache = _rand((2, b, 16, h, d), device, seed=24)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=16, block_boundaries=bb)
    assert_parity(got, _oracle(q, k, v, cache, 16, bb))


def test_empty_block_list_sees_only_history(device, built_lib):
    b, l, h, d = 1, 16, 2, 64
    q, k, v = (_rand((b, l, h, d), device, seed=s) for s in (25, 26, 27))
    cache = _rand((2, b, 8, h, d), device, seed=28)
    bb = torch.zeros(0, dtype=torch.int64, device=device)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=8, block_boundaries=bb)
    assert_parity(got, _oracle(q, k, v, cache, 8, bb))


@pytest.mark.parametrize("poison", ["finite", "inf", "nan"])
def test_future_blocks_are_invisible_bit_exact(device, built_lib, poison):
    """Whatever the keys/values of a future block hold, earlier blocks' outputs do not move.

    Blocks are 128 queries long (a whole query tile), so a future block's rows
    are never even loaded by the workgroups of earlier blocks: NaN/Inf there
    cannot leak through 0 * Inf.
    """
    b, l, h, d = 1, 384, 4, 128
    q, k, v = (_rand((b, l, h, d), device, seed=s) for s in (29, 30, 31))
    cache = _rand((2, b, 64, h, d), device, seed=32)
    bb = torch.tensor([0, 128, 256], device=device)
    base = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=64, block_boundaries=bb)
    k2, v2 = k.clone(), v.clone()
    fill = {"finite": 3.0, "inf": float("inf"), "nan": float("nan")}[poison]
    k2[:, 256:] = fill
    v2[:, 256:] = fill
    other = ops.blockwise_causal_attention(q, k2, v2, kv_cache=cache, cache_len=64,
                                           block_boundaries=bb)
    assert torch.equal(base[:, :256], other[:, :256])
    assert_parity(base, _oracle(q, k, v, cache, 64, bb))


def test_future_block_perturbation_unaligned_blocks(device, built_lib):
    """Blocks of 83 tokens (not tile aligned): finite changes to a future block stay invisible."""
    b, l, h, d = 1, 249, 4, 128
    q, k, v = (_rand((b, l, h, d), device, seed=s) for s in (33, 34, 35))
    bb = torch.tensor([0, 83, 166], device=device)
    base = ops.blockwise_causal_attention(q, k, v, block_boundaries=bb)
    k2, v2 = k.clone(), v.clone()
    k2[:, 166:] *= -2.0
    v2[:, 166:] += 1.5
    other = ops.blockwise_causal_attention(q, k2, v2, block_boundaries=bb)
    assert torch.equal(base[:, :166], other[:, :166])
    assert not torch.equal(base[:, 166:], other[:, 166:])


def test_varlen_matches_per_sequence_calls(device, built_lib):
    h, d, q_len = 4, 128, 99
    lens = [0, 40, 300, 131]
    b = len(lens)
    q = _rand((b, q_len, h, d), device, seed=36)
    k = _rand((b, q_len, h, d), device, seed=37)
    v = _rand((b, q_len, h, d), device, seed=38)
    cache = _rand((2, b, max(lens), h, d), device, seed=39)
    bb = torch.tensor([0, 83], device=device)
    got = ops.blockwise_causal_attention_varlen(q, k, v, kv_cache=cache, cache_lens=lens,
                                                block_boundaries=bb)
    for i, c in enumerate(lens):
        ref = _oracle(q[i:i + 1], k[i:i + 1], v[i:i + 1], cache[:, i:i + 1], c, bb)
        assert_parity(got[i:i + 1], ref, what=f"seq {i} cache {c}")
        one = ops.blockwise_causal_attention(q[i:i + 1], k[i:i + 1], v[i:i + 1],
                                             kv_cache=cache[:, i:i + 1].contiguous() if c else None,
                                             cache_len=c, block_boundaries=bb)
        assert_parity(one, ref)


@pytest.mark.parametrize("q_len,cache_len,h,d,dtype", [
    (1, 65535, 8, 128, torch.bfloat16), (16, 32749, 8, 128, torch.bfloat16),
    (83, 16381, 24, 128, torch.bfloat16), (1, 65535, 8, 64, torch.bfloat16),
    (83, 16381, 24, 128, torch.float16)])
def test_long_cache_decode(device, built_lib, q_len, cache_len, h, d, dtype):
    """Decode-shaped calls far past the benchmark's cache: up to 1,024 key tiles at the
    planner's largest split count (16), cache lengths that leave a partial last tile, and
    tile counts that do not divide evenly over the splits; head_dim 64 and f16 too."""
    b = 1
    q, k, v = (_rand((b, q_len, h, d), device, dtype, seed=60 + i) for i in range(3))
    cache = _rand((2, b, cache_len + q_len, h, d), device, dtype, seed=63)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len)
    assert torch.isfinite(got).all()
    assert_parity(got, _oracle(q, k, v, cache, cache_len, None), what=f"{q_len} x {cache_len}")


@pytest.mark.parametrize("q_len,cache_len,h,blocks", [(1024, 15360, 4, None),
                                                       (777, 20001, 8, [0, 333])])
def test_long_chunked_prefill(device, built_lib, q_len, cache_len, h, blocks):
    """Prefill-shaped chunks over long caches (the paired kernel, its key splits merged in
    the launch), past the 8,217 keys of the largest benchmark chunk, with and without a block
    list inside the chunk."""
    b, d = 1, 128
    q, k, v = (_rand((b, q_len, h, d), device, seed=80 + i) for i in range(3))
    cache = _rand((2, b, cache_len + q_len, h, d), device, seed=83)
    bb = torch.tensor(blocks, device=device) if blocks else None
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len,
                                         block_boundaries=bb)
    assert_parity(got, _oracle(q, k, v, cache, cache_len, bb),
                  what=f"{q_len} x {cache_len} blocks={blocks}")


def test_long_ragged_batch(device, built_lib):
    """A ragged batch with one sequence of 40,000 cached keys and one with none: the long
    sequence takes more splits than a merge inside the launch holds (the merge kernel runs)."""
    h, d, q_len = 8, 128, 99
    lens = [40000, 0]
    b = len(lens)
    q, k, v = (_rand((b, q_len, h, d), device, seed=70 + i) for i in range(3))
    cache = _rand((2, b, max(lens), h, d), device, seed=73)
    bb = torch.tensor([0, 83], device=device)
    got = ops.blockwise_causal_attention_varlen(q, k, v, kv_cache=cache, cache_lens=lens,
                                                block_boundaries=bb)
    for i, c in enumerate(lens):
        ref = _oracle(q[i:i + 1], k[i:i + 1], v[i:i + 1], cache[:, i:i + 1], c, bb)
        assert_parity(got[i:i + 1], ref, what=f"seq {i} cache {c}")


def test_kv_length_mismatch_with_a_mask_is_an_error(device, built_lib):
    """Lk != Lq is cross-attention (every key visible); with a causal or block
    mask it has no meaning (the mask is [q_len, cache_len + q_len]) and raises."""
    q = torch.zeros(1, 8, 2, 64, dtype=DT, device=device)
    k = torch.zeros(1, 9, 2, 64, dtype=DT, device=device)
    with pytest.raises(ValueError, match="must equal q length"):
        ops.blockwise_causal_attention(q, k, k, causal=True)
    with pytest.raises(ValueError, match="must equal q length"):
        ops.blockwise_causal_attention(q, k, k, block_boundaries=torch.tensor([0, 4]))


def test_default_scale(device, built_lib):
    q, k, v = (_rand((1, 40, 2, 64), device, seed=s) for s in (40, 41, 42))
    a = ops.blockwise_causal_attention(q, k, v)
    b = ops.blockwise_causal_attention(q, k, v, softmax_scale=1.0 / math.sqrt(64))
    assert torch.equal(a, b)


# Prefill-shaped calls run on the paired-group kernel (two four-wave groups
# half a tile apart, three LDS stages, its loops unrolled over the stages);
# the single-stream kernel (TUNE_ATTN_KERNEL 1) is the plain schedule, whose arithmetic
# is the same in the same order (with one split, so no partials are rounded;
# tiles a 256-row item visits past a 128-row item's range are fully masked
# for the earlier rows and add exact zeros). Tile counts 1..7 per work item cover every
# stage residue and loop exit; the cache cases put a partial tile at the
# cache boundary, and 300 rows leave the second work item's group 1 partly
# and wholly idle.
@pytest.mark.parametrize("d,dtype,q_len,cache_len,blocks", [
    (128, torch.bfloat16, 64, 0, None),
    (128, torch.bfloat16, 128, 0, None),
    (128, torch.bfloat16, 192, 0, None),
    (128, torch.bfloat16, 256, 0, None),
    (128, torch.bfloat16, 320, 0, None),
    (128, torch.bfloat16, 384, 0, None),
    (128, torch.bfloat16, 448, 0, None),
    (128, torch.bfloat16, 300, 100, [0, 96, 160]),
    (128, torch.float16, 256, 200, [0, 128]),
    (64, torch.bfloat16, 300, 0, [0, 96, 160]),
    (64, torch.float16, 192, 100, None),
])
def test_prefill_schedules_agree_bit_exact(device, built_lib, d, dtype, q_len, cache_len, blocks):
    h = 4
    q = _rand((1, q_len, h, d), device, dtype=dtype, scale=0.5, seed=71)
    k = _rand((1, q_len, h, d), device, dtype=dtype, seed=72)
    v = _rand((1, q_len, h, d), device, dtype=dtype, seed=73)
    cache = (_rand((2, 1, cache_len + q_len, h, d), device, dtype=dtype, scale=0.5, seed=74)
             if cache_len else None)
    bb = torch.tensor(blocks, device=device) if blocks else None

    def run(kernel):
        # One split (whole key ranges: no partials to round), kernel forced.
        with _lib.tuning(_lib.TUNE_ATTN_SPLITS, 1), _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel):
            return ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len,
                                                  block_boundaries=bb)

    paired, single = run(3), run(1)
    torch.cuda.synchronize()
    assert torch.equal(paired, single) or (
        torch.isnan(paired).equal(torch.isnan(single))
        and torch.equal(paired.nan_to_num(), single.nan_to_num()))
    assert_parity(paired, _oracle(q, k, v, cache, cache_len, bb),
                  what=f"d={d} {dtype} q_len={q_len} cache_len={cache_len} blocks={blocks}")
