"""Key splits merged inside the attention kernel itself (MI355X): the paired
prefill kernel and the dual-stream decode kernel.

With key splits, each split of a (batch, head, query tile) group leaves a
partial output. Under ``DX_TUNE_ATTN_PMERGE`` 2 the split of the group that
finishes last merges them all in the same launch (the paired kernel's default,
and the dual-stream kernel's on ragged batches); under 3 every split of the
group waits for the others and merges a chunk of the rows (dual-stream
kernel), from its XCD's L2 when the group shares one, else at device scope;
and under 1 the separate merge kernel does (the dual-stream kernel's default
on uniform calls, and every kernel's for groups of more than eight splits). Both merges add the splits' terms in the same order with the same
arithmetic, so their outputs must agree bit for bit; the merged result is also
held to the north-star bar against the oracle
(``python/dexter/ops/reference/attention.py:71-77``). The arrival counters
must come back to zero after every call, which repeated calls and graph
replays on the same workspace check.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.bench import harness
from dexter_amd.ops.gfx950 import _lib
from oracle import attention as oatt

from _util import assert_parity

pytestmark = pytest.mark.gpu

MERGE_KERNEL = 1
# (name, DX_TUNE_ATTN_KERNEL, DX_TUNE_ATTN_PMERGE) of the in-launch merges:
# the last split of a group merges it (2) on the paired and dual-stream
# kernels, or every split merges a chunk of its rows (3, dual-stream).
KERNELS = [("paired", 3, 2), ("dual", 2, 2), ("dual-spread", 2, 3)]


def _rand(shape, device, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(device)


def _oracle(q, k, v, cache, cache_len, bb=None):
    return oatt.blockwise_causal_attention(
        q.cpu(), k.cpu(), v.cpu(), None if cache is None else cache.cpu(), cache_len,
        None if bb is None else bb.cpu(), None, False, keep_fp32=True)


def _run(fn, kernel, merge, splits=0):
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_PMERGE, merge), \
            _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
        out = fn()
    torch.cuda.synchronize()
    return out


# (q_len, new keys, cache_len, heads, head_dim, dtype): two query tiles with a
# partial second one, a single partial tile, one query row, head_dim 64, f16.
# Head counts that are not multiples of 8 spread a group's splits over several
# XCDs (merged from memory); 8 keeps them on one (merged through its L2).
SHAPES = [(300, 300, 700, 8, 128, torch.bfloat16), (145, 145, 900, 5, 128, torch.bfloat16),
          (1, 1, 400, 4, 128, torch.bfloat16), (300, 300, 500, 8, 64, torch.bfloat16),
          (257, 257, 600, 3, 128, torch.float16)]


@pytest.mark.parametrize("kernel", KERNELS, ids=[k[0] for k in KERNELS])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"q{s[0]}-c{s[2]}-h{s[3]}-d{s[4]}-{str(s[5])[6:]}"
                                               for s in SHAPES])
@pytest.mark.parametrize("splits", [2, 3, 5, 8])
def test_in_kernel_merge_matches_merge_kernel(device, built_lib, kernel, shape, splits):
    lq, lk, c, h, d, dt = shape
    q = _rand((1, lq, h, d), device, dt, seed=400)
    k = _rand((1, lk, h, d), device, dt, seed=401)
    v = _rand((1, lk, h, d), device, dt, seed=402)
    cache = _rand((2, 1, c + lk, h, d), device, dt, seed=403)

    def call():
        return ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)

    got = _run(call, kernel[1], kernel[2], splits)
    ref = _run(call, kernel[1], MERGE_KERNEL, splits)
    assert torch.equal(got, ref), f"{kernel[0]} splits={splits}: in-kernel merge differs"
    if dt == torch.bfloat16:
        assert_parity(got, _oracle(q, k, v, cache, c), what=f"{kernel[0]} {shape} splits={splits}")


@pytest.mark.parametrize("kernel", KERNELS, ids=[k[0] for k in KERNELS])
def test_in_kernel_merge_cross_attention_and_blocks(device, built_lib, kernel):
    """No cache and no mask (cross-attention), then a block list over a cache."""
    kern, in_kernel = kernel[1], kernel[2]
    q = _rand((2, 300, 4, 128), device, seed=410)
    k, v = _rand((2, 700, 4, 128), device, seed=411), _rand((2, 700, 4, 128), device, seed=412)
    for splits in (2, 4, 7):
        got = _run(lambda: ops.blockwise_causal_attention(q, k, v), kern, in_kernel, splits)
        ref = _run(lambda: ops.blockwise_causal_attention(q, k, v), kern, MERGE_KERNEL, splits)
        assert torch.equal(got, ref), f"cross splits={splits}"
        assert_parity(got, _oracle(q, k, v, None, 0), what=f"cross splits={splits}")
    cache = _rand((2, 2, 1000, 4, 128), device, seed=413)
    kn, vn = k[:, :300].contiguous(), v[:, :300].contiguous()
    bb = torch.tensor([0, 100, 200], dtype=torch.int32, device=device)

    def blocks():
        return ops.blockwise_causal_attention(q, kn, vn, kv_cache=cache, cache_len=700,
                                              block_boundaries=bb)

    got = _run(blocks, kern, in_kernel, 3)
    assert torch.equal(got, _run(blocks, kern, MERGE_KERNEL, 3)), "block list splits=3"
    assert_parity(got, _oracle(q, kn, vn, cache, 700, bb), what="block list splits=3")


@pytest.mark.parametrize("kernel", KERNELS, ids=[k[0] for k in KERNELS])
@pytest.mark.parametrize("h", [8, 5])
def test_in_kernel_merge_ragged_batch(device, built_lib, kernel, h):
    """The C4 ragged lengths with the planner's splits (several per long
    sequence, one for the short ones); 5 heads spread each group's splits over
    several XCDs (merged from memory)."""
    lens = [0, 332, 1245, 3237]
    d = 128
    q, k, v = (_rand((4, 99, h, d), device, seed=420 + i) for i in range(3))
    cache = _rand((2, 4, max(lens), h, d), device, seed=423)
    bb = torch.tensor([0, 83], dtype=torch.int32, device=device)

    def call():
        return ops.blockwise_causal_attention_varlen(q, k, v, kv_cache=cache, cache_lens=lens,
                                                     block_boundaries=bb)

    got = _run(call, kernel[1], kernel[2])
    assert torch.equal(got, _run(call, kernel[1], MERGE_KERNEL)), f"{kernel[0]} ragged h={h}"
    for i, c in enumerate(lens):
        assert_parity(got[i:i + 1], _oracle(q[i:i + 1], k[i:i + 1], v[i:i + 1],
                                            cache[:, i:i + 1], c, bb), what=f"seq {i}")


@pytest.mark.parametrize("kernel", KERNELS, ids=[k[0] for k in KERNELS])
@pytest.mark.parametrize("h", [8, 5])
def test_in_kernel_merge_repeats_and_graph_replays(device, built_lib, kernel, h):
    """Calls of different split counts one after another on the same workspace,
    then a captured call replayed with eager calls in between: every result
    equals the merge kernel's (a counter left nonzero would skip or repeat a
    group's merge). With 8 heads every group's splits share an XCD (merged
    through its L2); with 5 they are spread over several (merged from memory)."""
    lq, c, d = 300, 600, 128
    ins = [(_rand((1, lq, h, d), device, seed=430 + 4 * i),
            _rand((1, lq, h, d), device, seed=431 + 4 * i),
            _rand((1, lq, h, d), device, seed=432 + 4 * i),
            _rand((2, 1, c + lq, h, d), device, seed=433 + 4 * i)) for i in range(3)]

    def call(i):
        q, k, v, cache = ins[i]
        return ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)

    refs = [_run(lambda i=i: call(i), kernel[1], MERGE_KERNEL, 3) for i in range(3)]
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel[1]), \
            _lib.tuning(_lib.TUNE_ATTN_PMERGE, kernel[2]):
        for splits in (3, 2, 5, 3):
            with _lib.tuning(_lib.TUNE_ATTN_SPLITS, splits):
                for i in range(3):
                    got = call(i)
                    torch.cuda.synchronize()
                    if splits == 3:
                        assert torch.equal(got, refs[i]), f"repeat splits={splits} input {i}"
        with _lib.tuning(_lib.TUNE_ATTN_SPLITS, 3):
            out = {}
            graph = harness.capture(lambda: out.__setitem__("o", call(0)))
            for rep in range(3):
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out["o"], refs[0]), f"graph replay {rep}"
                eager = call(1)
                torch.cuda.synchronize()
                assert torch.equal(eager, refs[1]), f"eager call after replay {rep}"


@pytest.mark.parametrize("kernel", KERNELS, ids=[k[0] for k in KERNELS])
@pytest.mark.parametrize("heads", [(8, 2), (6, 3), (16, 4)])
def test_in_kernel_merge_grouped_query(device, built_lib, kernel, heads):
    """Grouped-query K/V (fewer K/V heads than query heads): the work-item map
    keeps the query heads of a K/V head together, and each query head's splits
    still merge in the launch, from the L2 or from memory."""
    h, hkv = heads
    lq, c = 200, 600
    q = _rand((1, lq, h, 128), device, seed=440)
    k = _rand((1, lq, hkv, 128), device, seed=441)
    v = _rand((1, lq, hkv, 128), device, seed=442)
    cache = _rand((2, 1, c + lq, hkv, 128), device, seed=443)

    def call():
        return ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c)

    for splits in (2, 5):
        got = _run(call, kernel[1], kernel[2], splits)
        assert torch.equal(got, _run(call, kernel[1], MERGE_KERNEL, splits)), (
            f"{kernel[0]} GQA {h}/{hkv} splits={splits}")
        assert_parity(got, _oracle(q, k, v, cache, c), what=f"{kernel[0]} GQA {h}/{hkv}")
