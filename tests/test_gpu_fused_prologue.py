"""SelfAttention's decode step in one call (MI355X): ``ops.qk_norm_rope_attention``
against the three ops it replaces.

``SelfAttention.forward`` runs ``ops.qk_norm_rope``, ``KVCache.append`` and
``ops.blockwise_causal_attention`` (``models/dreamzero/model.py:166-182``).
The one call must give the same bits for the rotated q and k, the cache rows
it appends and the attention output; the C1 case is also held to the
north-star bar against the oracle chain (``oracle/rope.py``,
``oracle/attention.py``).
"""

from __future__ import annotations

import math

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.bench import harness
from oracle import attention as oatt
from oracle import rope as orope

from _util import assert_parity

pytestmark = pytest.mark.gpu


def _rand(shape, device, dtype=torch.bfloat16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def _tables(l, d, dtype, device, offset=0):
    pos = torch.arange(offset, offset + l, dtype=torch.float64)[:, None]
    inv = 1.0 / (1e4 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = pos * inv[None, :]
    return torch.cos(ang).to(dtype).to(device), torch.sin(ang).to(dtype).to(device)


def _case(device, b, l, h, d, cache_len, dt=torch.bfloat16, wdt=torch.bfloat16,
          tdt=torch.float32, seed=0, capacity=None):
    q = _rand((b, l, h, d), device, dt, seed)
    k = _rand((b, l, h, d), device, dt, seed + 1)
    v = _rand((b, l, h, d), device, dt, seed + 2)
    qw = (1 + 0.1 * _rand((h * d,), device, torch.float32, seed + 3)).to(wdt)
    kw = (1 + 0.1 * _rand((h * d,), device, torch.float32, seed + 4)).to(wdt)
    cos, sin = _tables(l, d, tdt, device, offset=cache_len)
    cap = capacity if capacity is not None else cache_len + l
    cache = _rand((2, b, cap, h, d), device, dt, seed + 5) if cap else None
    return q, k, v, qw, kw, cos, sin, cache


def _three_ops(q, k, v, qw, kw, cos, sin, cache, cache_len, append, bb, causal, interleaved):
    qr, kr = ops.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6, interleaved)
    if append:
        ops.kv_cache_append(cache, kr, v, cache_len)
    out = ops.blockwise_causal_attention(qr, kr, v, kv_cache=cache, cache_len=cache_len,
                                         block_boundaries=bb, causal=causal)
    return out, qr, kr


def _fused(q, k, v, qw, kw, cos, sin, cache, cache_len, append, bb, causal, interleaved):
    return ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache,
                                      cache_len=cache_len, append=append, block_boundaries=bb,
                                      causal=causal, interleaved=interleaved, return_qk=True)


def _check(device, case, cache_len, append=False, bb=None, causal=False, interleaved=True,
           what=""):
    q, k, v, qw, kw, cos, sin, cache = case
    ref_cache = cache.clone() if cache is not None else None
    ref = _three_ops(q, k, v, qw, kw, cos, sin, ref_cache, cache_len, append, bb, causal,
                     interleaved)
    c = cache.clone() if cache is not None else None
    got = _fused(q, k, v, qw, kw, cos, sin, c, cache_len, append, bb, causal, interleaved)
    torch.cuda.synchronize()
    for name, g, r in zip(("out", "q", "k"), got, ref):
        assert torch.equal(g, r), f"{what}: {name} differs from the three ops"
    if c is not None:
        assert torch.equal(c, ref_cache), f"{what}: cache differs"
    return got


# (B, L, H, D, cache_len): the Wan-5B decode chunk (C1), a batch of two, one
# token, 32 heads, 40 heads (Wan-14B), head_dim 64.
SHAPES = [(1, 83, 24, 128, 1245), (2, 40, 8, 128, 300), (1, 1, 24, 128, 500),
          (1, 64, 32, 128, 700), (1, 83, 40, 128, 900), (1, 83, 24, 64, 1245)]


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
@pytest.mark.parametrize("append", [False, True])
def test_fused_equals_three_ops(device, built_lib, shape, append):
    b, l, h, d, c = shape
    case = _case(device, b, l, h, d, c, seed=sum(shape))
    _check(device, case, c, append=append, what=f"{shape} append={append}")


@pytest.mark.parametrize("dtypes", [(torch.bfloat16, torch.bfloat16, torch.bfloat16),
                                    (torch.bfloat16, torch.float32, torch.float32),
                                    (torch.float16, torch.float16, torch.float32),
                                    (torch.float16, torch.float32, torch.float16)],
                         ids=["bf16-bf16w-bf16t", "bf16-f32w-f32t", "f16-f16w-f32t",
                              "f16-f32w-f16t"])
@pytest.mark.parametrize("interleaved", [True, False])
def test_fused_dtypes_and_pairings(device, built_lib, dtypes, interleaved):
    dt, wdt, tdt = dtypes
    case = _case(device, 1, 83, 24, 128, 1245, dt, wdt, tdt, seed=50)
    _check(device, case, 1245, append=True, interleaved=interleaved,
           what=f"{dtypes} interleaved={interleaved}")


def test_fused_masks(device, built_lib):
    """Block starts (ascending and not) and token-causal on the new keys."""
    case = _case(device, 1, 83, 24, 128, 600, seed=60)
    for bb in ([0, 40], [0, 50, 30], [0, -40, 83]):
        _check(device, case, 600, bb=torch.tensor(bb, dtype=torch.int32, device=device),
               what=f"blocks {bb}")
    _check(device, case, 600, causal=True, what="causal")


def test_fused_without_cache(device, built_lib):
    """No history: the chunk attends to itself (block starts of C0's form)."""
    case = _case(device, 1, 48, 8, 128, 0, seed=70)
    bb = torch.tensor([0, 16, 32], dtype=torch.int32, device=device)
    _check(device, case, 0, bb=bb, what="no cache")
    case = _case(device, 1, 48, 8, 128, 0, seed=71, capacity=64)
    _check(device, case, 0, append=True, what="no cache, append")


def test_fused_c1_against_oracle_chain(device, built_lib):
    """The C1 chunk from pre-norm activations: output within the north-star bar of the
    oracle's prologue followed by the oracle's attention."""
    q, k, v, qw, kw, cos, sin, cache = _case(device, 1, 83, 24, 128, 1245, seed=80)
    out = ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache, cache_len=1245)
    torch.cuda.synchronize()
    rq, rk = orope.qk_norm_rope(q.cpu(), k.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), 1e-6)
    ref = oatt.blockwise_causal_attention(rq, rk, v.cpu(), cache.cpu(), 1245, None, None,
                                          keep_fp32=True)
    assert_parity(out, ref, what="fused C1 vs oracle chain")


def test_fused_cache_full(device, built_lib):
    """Appending past the capacity raises the reference's error before any launch."""
    q, k, v, qw, kw, cos, sin, cache = _case(device, 1, 83, 8, 128, 100, seed=90, capacity=150)
    before = cache.clone()
    with pytest.raises(RuntimeError, match="KV cache full"):
        ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache, cache_len=100,
                                   append=True)
    torch.cuda.synchronize()
    assert torch.equal(cache, before)


def test_fused_graph_replays_and_repeats(device, built_lib):
    """Calls of different shapes one after another on the shared workspace, then a
    captured call replayed with eager calls in between, each equal to the three ops."""
    cases = [(_case(device, 1, 83, 24, 128, 1245, seed=100), 1245),
             (_case(device, 2, 40, 8, 128, 300, seed=110), 300),
             (_case(device, 1, 83, 24, 128, 1245, seed=120), 1245)]
    refs = []
    for case, c in cases:
        q, k, v, qw, kw, cos, sin, cache = case
        refs.append(_three_ops(q, k, v, qw, kw, cos, sin, cache, c, False, None, False, True))
    for rep in range(2):
        for (case, c), ref in zip(cases, refs):
            q, k, v, qw, kw, cos, sin, cache = case
            got = ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache,
                                             cache_len=c)
            torch.cuda.synchronize()
            assert torch.equal(got, ref[0]), f"repeat {rep} cache_len {c}"
    (q, k, v, qw, kw, cos, sin, cache), c = cases[0]
    res = {}
    graph = harness.capture(lambda: res.__setitem__(
        "o", ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache, cache_len=c)))
    for rep in range(3):
        res["o"].zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res["o"], refs[0][0]), f"graph replay {rep}"
        (q2, k2, v2, qw2, kw2, cos2, sin2, cache2), c2 = cases[1]
        eager = ops.qk_norm_rope_attention(q2, k2, v2, qw2, kw2, cos2, sin2, kv_cache=cache2,
                                           cache_len=c2)
        torch.cuda.synchronize()
        assert torch.equal(eager, refs[1][0]), f"eager call after replay {rep}"


def test_fused_scale_default_and_explicit(device, built_lib):
    q, k, v, qw, kw, cos, sin, cache = _case(device, 1, 83, 24, 128, 500, seed=130)
    a = ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache, cache_len=500)
    b = ops.qk_norm_rope_attention(q, k, v, qw, kw, cos, sin, kv_cache=cache, cache_len=500,
                                   softmax_scale=1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    assert torch.equal(a, b)
