"""HIP QK-RMSNorm+RoPE prologue and KV-cache append against the oracle (MI355X).

The prologue restates the reference's intermediate rounding (bf16 after the
norm, then fp32 rotation), so it agrees with the oracle up to the summation
order of the plane mean: almost every element is bit-identical and the rest
differ by one unit in the last place. The append is a copy: bit-exact.
Reference tests mirrored: ``test/test_ops.py:53-65, 184-199`` and
``test/test_model.py:42-66``.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.bench.workloads import rope_table
from dexter_amd.models import KVCache, SelfAttention
from dexter_amd.registry import select_spec
from oracle import attention as oatt
from oracle import kv_cache as okv
from oracle import rope as orope

from _util import assert_parity, close_rel

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _pair_norm(x: torch.Tensor, interleaved: bool) -> torch.Tensor:
    """Per element, the norm of its rotary pair (rotation preserves it)."""
    if interleaved:
        n = (x[..., 0::2] ** 2 + x[..., 1::2] ** 2).sqrt()
        return n.repeat_interleave(2, dim=-1)
    h = x.shape[-1] // 2
    n = (x[..., :h] ** 2 + x[..., h:] ** 2).sqrt()
    return torch.cat((n, n), dim=-1)


def _ulp_agreement(got: torch.Tensor, ref: torch.Tensor, what="", interleaved=True):
    """Outputs agree to one rounding step; nearly all elements bit-identically.

    A one-ulp difference in a normalised pair (lo, hi) -- the mean's summation
    order can flip a rounding -- moves both rotated outputs by about one ulp
    of the pair's norm, which for a small output is many of its own ulps. So
    the bound is two ulps of the pair norm.
    """
    g, r = got.float().cpu(), ref.float().cpu()
    assert torch.isfinite(g).all()
    eps = torch.finfo(got.dtype).eps
    tol = 2 * eps * torch.maximum(_pair_norm(r, interleaved), r.abs()).clamp_min(1e-3)
    bad = (g - r).abs() > tol
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one ulp"
    differ = (g != r).float().mean().item()
    assert differ < 0.01, f"{what}: {differ:.2%} of elements not bit-identical"


def _inputs(b, l, h, d, dtype=DT, wdtype=DT, tdtype=torch.float32, seed=0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, l, h, d, generator=g).to(dtype)
    k = torch.randn(b, l, h, d, generator=g).to(dtype)
    qw = torch.randn(h * d, generator=g).to(wdtype)
    kw = torch.randn(h * d, generator=g).to(wdtype)
    cos, sin = rope_table(torch.arange(l), d)
    cos, sin = cos.to(tdtype), sin.to(tdtype)
    return [t.to(device) for t in (q, k, qw, kw, cos, sin)]


def test_selected_kernel_is_hip(device, built_lib):
    q = torch.zeros(1, 2, 24, 128, dtype=DT, device=device)
    assert select_spec("rope", "qk_norm_rope", q, q).name == "hip_qk_norm_rope_gfx950"


def test_qk_norm_rope(device, built_lib):
    q, k, qw, kw, cos, sin = _inputs(1, 125, 24, 128, device=device)
    gq, gk = ops.qk_norm_rope(q, k, qw, kw, cos, sin)
    rq, rk = orope.qk_norm_rope(q.cpu(), k.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), 1e-6)
    close_rel(gq, rq)
    close_rel(gk, rk)
    _ulp_agreement(gq, rq, "q")
    _ulp_agreement(gk, rk, "k")


@pytest.mark.parametrize("interleaved", [True, False])
def test_qk_norm_rope_both_pairings(device, built_lib, interleaved):
    q, k, w, _, cos, sin = _inputs(1, 48, 8, 128, tdtype=DT, device=device)
    gq, gk = ops.qk_norm_rope(q, k, w, w, cos, sin, interleaved=interleaved)
    rq, rk = orope.qk_norm_rope(q.cpu(), k.cpu(), w.cpu(), w.cpu(), cos.cpu(), sin.cpu(), 1e-6,
                                interleaved)
    _ulp_agreement(gq, rq, interleaved=interleaved)
    _ulp_agreement(gk, rk, interleaved=interleaved)
    other, _ = ops.qk_norm_rope(q, k, w, w, cos, sin, interleaved=not interleaved)
    assert not torch.allclose(gq.float(), other.float(), atol=1e-3)


@pytest.mark.parametrize("shape", [(1, 83, 24, 128), (2, 33, 40, 128), (1, 7, 4, 64), (3, 5, 2, 16)])
@pytest.mark.parametrize("dtype,wdtype,tdtype", [
    (torch.bfloat16, torch.bfloat16, torch.float32),
    (torch.bfloat16, torch.float32, torch.bfloat16),
    (torch.float16, torch.float16, torch.float16),
])
def test_prologue_shapes_and_dtypes(device, built_lib, shape, dtype, wdtype, tdtype):
    q, k, qw, kw, cos, sin = _inputs(*shape, dtype=dtype, wdtype=wdtype, tdtype=tdtype,
                                     seed=3, device=device)
    gq, gk = ops.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-5)
    rq, rk = orope.qk_norm_rope(q.cpu(), k.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), 1e-5)
    assert gq.dtype == dtype
    _ulp_agreement(gq, rq, f"{shape} {dtype}")
    _ulp_agreement(gk, rk, f"{shape} {dtype}")


def test_prologue_strided_input(device, built_lib):
    q, k, qw, kw, cos, sin = _inputs(2, 20, 6, 128, device=device)
    qs = torch.cat([q, q], dim=2)[:, :, ::2]  # head stride 2*D
    gq, _ = ops.qk_norm_rope(qs, k, qw, kw, cos, sin)
    rq, _ = orope.qk_norm_rope(qs.cpu(), k.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), 1e-6)
    _ulp_agreement(gq, rq)


def test_fused_append_equals_prologue_then_append(device, built_lib):
    b, l, h, d, start = 1, 83, 24, 128, 166
    q, k, qw, kw, cos, sin = _inputs(b, l, h, d, seed=5, device=device)
    v = torch.randn(b, l, h, d, device=device).to(DT)
    cache = torch.randn(2, b, 400, h, d, device=device).to(DT)
    before = cache.clone()
    fq, fk = ops.qk_norm_rope_append(q, k, v, qw, kw, cos, sin, cache, start)
    uq, uk = ops.qk_norm_rope(q, k, qw, kw, cos, sin)
    assert torch.equal(fq, uq) and torch.equal(fk, uk)
    assert torch.equal(cache[0, :, start:start + l], uk)
    assert torch.equal(cache[1, :, start:start + l], v)
    assert torch.equal(cache[:, :, :start], before[:, :, :start])
    assert torch.equal(cache[:, :, start + l:], before[:, :, start + l:])


def test_kv_append_bit_exact(device, built_lib):
    ref = okv.KVCache(1, 2, 64, 3, 128)
    cache = torch.zeros(2, 2, 64, 3, 128, dtype=DT, device=device)
    for step in range(3):
        k = torch.randn(2, 17, 3, 128).to(DT)
        v = torch.randn(2, 17, 3, 128).to(DT)
        ops.kv_cache_append(cache, k.to(device), v.to(device), ref.length)
        ref.append(0, k, v)
        ref.commit(17)
    assert torch.equal(cache.cpu(), ref.cache[0])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_kv_append_other_dtypes_and_strides(device, built_lib, dtype):
    cache = torch.zeros(2, 1, 32, 4, 64, dtype=dtype, device=device)
    kk = torch.randn(1, 4, 10, 64, device=device).to(dtype).transpose(1, 2)  # [1,10,4,64] view
    vv = torch.randn(1, 10, 4, 64, device=device).to(dtype)
    ops.kv_cache_append(cache, kk, vv, 5)
    assert torch.equal(cache[0, :, 5:15], kk) and torch.equal(cache[1, :, 5:15], vv)
    assert not cache[:, :, :5].any() and not cache[:, :, 15:].any()


def test_kv_cache_overflow_is_an_error_and_writes_nothing(device, built_lib):
    cache = KVCache(layers=2, batch=1, capacity=100, heads=2, head_dim=64, device=device, dtype=DT)
    k = torch.ones(1, 60, 2, 64, dtype=DT, device=device)
    cache.append(0, k, k)
    cache.commit(60)
    snapshot = cache.cache[0].clone()
    with pytest.raises(RuntimeError, match="KV cache full: 60 \\+ 60 > 100"):
        cache.append(0, k, k)
    with pytest.raises(RuntimeError, match="KV cache full"):
        ops.kv_cache_append(cache.cache[0], k, k, 60)
    assert torch.equal(cache.cache[0], snapshot)


def test_kv_cache_holds_only_committed_blocks(device, built_lib):
    """The cache prefix [0, length) is exactly the committed blocks, in order."""
    c = KVCache(layers=3, batch=1, capacity=50, heads=2, head_dim=64, device=device, dtype=DT)
    blocks = []
    for step in range(4):
        k = torch.randn(1, 12, 2, 64, device=device).to(DT)
        v = torch.randn(1, 12, 2, 64, device=device).to(DT)
        for layer in range(3):
            c.append(layer, k, v)
        assert c.length == 12 * step
        c.commit(12)
        blocks.append((k, v))
    for layer in range(3):
        assert torch.equal(c.cache[layer][0, :, :48], torch.cat([x[0] for x in blocks], 1))
        assert torch.equal(c.cache[layer][1, :, :48], torch.cat([x[1] for x in blocks], 1))


@pytest.mark.parametrize("fused", [True, False])
def test_self_attention_layer_drop_in(device, built_lib, fused):
    """A DiT-style layer over three steps: prime (write) then read, vs the oracle chain."""
    torch.manual_seed(0)
    dim, heads, blk = 768, 6, 40
    layer = SelfAttention(dim, heads, dtype=DT, device=device)
    with torch.no_grad():
        layer.q_norm.copy_(1 + 0.1 * torch.randn(dim))
        layer.k_norm.copy_(1 + 0.1 * torch.randn(dim))
    cache = KVCache(1, 1, 200, heads, dim // heads, device, DT)
    ocache = okv.KVCache(1, 1, 200, heads, dim // heads)
    for step in range(3):
        x = torch.randn(1, blk, dim, device=device).to(DT)
        cos, sin = rope_table(torch.arange(blk) + step * blk, dim // heads)
        cos, sin = cos.to(device), sin.to(device)
        # read pass (denoise step): attends to history + itself, writes nothing
        out = layer(x, cos, sin, cache, 0, write=False)
        # oracle of the same pass
        with torch.no_grad():
            shp = (1, blk, heads, dim // heads)
            q = torch.nn.functional.linear(x, layer.q.weight, layer.q.bias).view(shp).cpu()
            k = torch.nn.functional.linear(x, layer.k.weight, layer.k.bias).view(shp).cpu()
            v = torch.nn.functional.linear(x, layer.v.weight, layer.v.bias).view(shp).cpu()
        rq, rk = orope.qk_norm_rope(q, k, layer.q_norm.cpu(), layer.k_norm.cpu(), cos.cpu(),
                                    sin.cpu(), layer.eps)
        att = oatt.blockwise_causal_attention(rq, rk, v, ocache.cache[0], ocache.length, None, None)
        ref = torch.nn.functional.linear(att.reshape(1, blk, dim).to(device), layer.o.weight,
                                         layer.o.bias)
        close_rel(out, ref, tol=3e-2)
        # prime pass: write this block, then commit
        layer(x, cos, sin, cache, 0, write=True, fused_append=fused)
        ocache.append(0, rk, v)
        cache.commit(blk)
        ocache.commit(blk)
        assert_parity(cache.cache[0][:, :, :cache.length], ocache.cache[0][:, :, :ocache.length],
                      max_abs=0.05, mean_abs=1e-3, what="cache contents")
