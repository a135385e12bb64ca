"""Pin the CPU oracle before trusting it (no GPU).

The reference ships no golden vectors for this path, so each oracle function
is pinned three independent ways, chosen so that a plausible mistake (a
dropped scale, a mask off by one block, a transposed operand, a lost
rounding step) fails at least one:

* an fp64 brute force written from the definitions (``oracle/brute.py``);
* a library routine: ``torch.nn.functional.scaled_dot_product_attention``;
* closed forms: identical keys average exactly the visible values; one-hot
  values read out the attention probabilities; RoPE preserves pair norms;
  ``cos=1, sin=0`` reduces to the plain RMS norm; adaLN with zero modulation
  is ``torch.nn.functional.layer_norm``, a hand-computed row gives known
  values, and a constant shift of x changes nothing; a zero gate returns x.

The last tests plant mistakes in copies of the oracle and check the pins
catch them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import brute
from oracle import kv_cache as okv
from oracle import norm as onorm
from oracle import rope as orope


def _c0_inputs():
    from dexter_amd.bench.workloads import CONFIGS, make_inputs
    return make_inputs(CONFIGS["C0"])


# ---------------------------------------------------------------- mask -----

@pytest.mark.parametrize("cache_len", [0, 5])
@pytest.mark.parametrize("mode", ["none", "causal", "blocks", "ragged_blocks", "late_first"])
def test_mask_matches_brute_rule(cache_len, mode):
    q_len = 13
    starts = {"none": None, "causal": None, "blocks": [0, 4, 9],
              "ragged_blocks": [0, 1, 7, 12], "late_first": [3, 8]}[mode]
    causal = mode == "causal"
    bb = torch.tensor(starts) if starts is not None else None
    mask = oatt.block_causal_mask(q_len, cache_len, bb, causal=causal)
    assert mask.shape == (q_len, cache_len + q_len)
    for i in range(q_len):
        for j in range(cache_len + q_len):
            assert bool(mask[i, j]) == brute.key_visible(i, j, q_len, cache_len, starts, causal)


# Block lists the reference accepts beyond ascending starts: unsorted,
# overlapping and negative entries (the GPU tests run the same lists).
ODD_BLOCK_LISTS = [[0, 50, 30], [40, 0, 83], [30, 0, 60, 10], [0, -40, 83], [50, 20],
                   [0, 83, 20, 60], [-90, 10], [0, -100, 40], [-5, -83, 2], [0, -82, 83],
                   [0, -60, 30, -70]]


@pytest.mark.parametrize("cache_len", [0, 10, 39, 300])
@pytest.mark.parametrize("starts", ODD_BLOCK_LISTS, ids=[str(s) for s in ODD_BLOCK_LISTS])
def test_mask_matches_python_slices_on_odd_lists(cache_len, starts):
    """The oracle's mask equals the reference's construction done with real
    slice assignment on nested lists (``brute.slice_mask``) and the per-key
    rule of ``brute.key_visible``, for lists in any order and negative starts,
    including stops ``cache_len + hi`` below zero, which wrap."""
    q_len = 83
    mask = oatt.block_causal_mask(q_len, cache_len, torch.tensor(starts))
    want = torch.tensor(brute.slice_mask(q_len, cache_len, starts))
    assert torch.equal(mask, want)
    for i in range(0, q_len, 7):
        for j in range(cache_len + q_len):
            assert bool(mask[i, j]) == brute.key_visible(i, j, q_len, cache_len, starts, False)


@pytest.mark.parametrize("cache_len", [0, 5])
@pytest.mark.parametrize("mode", ["none", "causal", "blocks", "late_first"])
def test_slice_mask_matches_brute_rule(cache_len, mode):
    """The two brute restatements agree with each other on ordinary inputs."""
    q_len = 13
    starts = {"none": None, "causal": None, "blocks": [0, 4, 9], "late_first": [3, 8]}[mode]
    causal = mode == "causal"
    want = brute.slice_mask(q_len, cache_len, starts, causal)
    for i in range(q_len):
        for j in range(cache_len + q_len):
            assert want[i][j] == brute.key_visible(i, j, q_len, cache_len, starts, causal)


def test_wrapped_negative_stop_is_visible():
    """Known answer: ``[0, -40, 83]`` over 83 queries at cache_len 0. The pair
    (0, -40) sets rows 0..42 (``0:-40`` of 83) and columns ``0:-40``, i.e. keys
    0..42; the pair (-40, 83) sets rows 43..82 and every key."""
    mask = oatt.block_causal_mask(83, 0, torch.tensor([0, -40, 83]))
    assert mask[:43, :43].all() and not mask[:43, 43:].any()
    assert mask[43:].all()
    # At cache_len 10 the stop 10 - 40 still wraps: current keys [0, 10 + 83 - 40).
    mask = oatt.block_causal_mask(83, 10, torch.tensor([0, -40, 83]))
    assert mask[:43, :10 + 53].all() and not mask[:43, 10 + 53:].any()
    # At cache_len 39 the stop -1 wraps to the last column: all but the last key.
    mask = oatt.block_causal_mask(83, 39, torch.tensor([0, -40, 83]))
    assert mask[:43, :39 + 82].all() and not mask[:43, 39 + 82:].any()
    # At cache_len 40 the stop is 0, before the slice's start: only the cache.
    mask = oatt.block_causal_mask(83, 40, torch.tensor([0, -40, 83]))
    assert mask[:43, :40].all() and not mask[:43, 40:].any()


def test_slice_pin_catches_an_unwrapped_stop():
    """A planted oracle that takes ``min(hi, q_len)`` for every pair (no wrap
    of a negative stop) fails the slice-built mask."""
    q_len, cache_len, starts = 83, 0, [0, -40, 83]
    bounds = starts + [q_len]
    end = torch.zeros(q_len, dtype=torch.int64)
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        end[lo:hi] = torch.clamp(end[lo:hi], min=min(hi, q_len))
    planted = torch.arange(cache_len + q_len)[None, :] < (cache_len + end)[:, None]
    assert not torch.equal(planted, torch.tensor(brute.slice_mask(q_len, cache_len, starts)))


def test_mask_c0_structure():
    """C0: 3 blocks of 16; block b sees keys [0, 16(b+1)) exactly."""
    mask = oatt.block_causal_mask(48, 0, torch.tensor([0, 16, 32]))
    for b in range(3):
        rows = mask[16 * b:16 * (b + 1)]
        assert rows[:, :16 * (b + 1)].all()
        assert not rows[:, 16 * (b + 1):].any()


# ----------------------------------------------------------- attention -----

def test_c0_matches_fp64_brute_force():
    inp = _c0_inputs()
    q, k, v = inp.q, inp.k, inp.v
    got = oatt.blockwise_causal_attention(q, k, v, None, 0, torch.tensor([0, 16, 32]), None)
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), starts=[0, 16, 32])
    assert got.dtype == torch.float32
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=2e-6)


@pytest.mark.parametrize("cache_len", [0, 7])
@pytest.mark.parametrize("causal", [False, True])
def test_with_cache_matches_fp64_brute_force(cache_len, causal):
    g = torch.Generator().manual_seed(11)
    b, l, h, d, s = 2, 10, 3, 16, 12
    q, k, v = (torch.randn(b, l, h, d, generator=g) for _ in range(3))
    cache = torch.randn(2, b, s, h, d, generator=g)
    starts = None if causal else [0, 3, 8]
    bb = None if starts is None else torch.tensor(starts)
    got = oatt.blockwise_causal_attention(q, k, v, cache, cache_len, bb, 0.37, causal)
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), cache[0].numpy(), cache[1].numpy(),
                          cache_len, starts, causal, scale=0.37)
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=2e-6)


@pytest.mark.parametrize("mode", ["blocks", "causal", "none"])
def test_matches_sdpa(mode):
    g = torch.Generator().manual_seed(3)
    b, l, h, d, cache_len = 1, 40, 4, 64, 24
    q, k, v = (torch.randn(b, l, h, d, generator=g) for _ in range(3))
    cache = torch.randn(2, b, 32, h, d, generator=g)
    bb = torch.tensor([0, 10, 25]) if mode == "blocks" else None
    got = oatt.blockwise_causal_attention(q, k, v, cache, cache_len, bb, None, mode == "causal")
    keys = torch.cat((cache[0, :, :cache_len], k), 1).transpose(1, 2)
    vals = torch.cat((cache[1, :, :cache_len], v), 1).transpose(1, 2)
    mask = oatt.block_causal_mask(l, cache_len, bb, causal=mode == "causal")
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), keys, vals, attn_mask=mask)
    torch.testing.assert_close(got, ref.transpose(1, 2), rtol=0, atol=2e-6)


def test_no_mask_is_plain_softmax_attention():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 20, 2, 32, generator=g) for _ in range(3))
    got = oatt.blockwise_causal_attention(q, k, v)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    torch.testing.assert_close(got, ref.transpose(1, 2), rtol=0, atol=2e-6)


def test_identical_keys_average_exactly_the_visible_values():
    """All keys equal => uniform weights over the visible set: the mean of visible v rows."""
    g = torch.Generator().manual_seed(8)
    b, l, h, d, cache_len = 1, 12, 2, 8, 4
    q = torch.randn(b, l, h, d, generator=g)
    k = torch.ones(b, l, h, d)
    v = torch.randn(b, l, h, d, generator=g, dtype=torch.float64).float()
    cache = torch.zeros(2, b, 6, h, d)
    cache[0, :, :cache_len] = 1.0
    cache[1, :, :cache_len] = torch.randn(b, cache_len, h, d, generator=g)
    starts = [0, 5, 9]
    got = oatt.blockwise_causal_attention(q, k, v, cache, cache_len, torch.tensor(starts), None)
    vals = torch.cat((cache[1, :, :cache_len], v), 1)
    ends = [5] * 5 + [9] * 4 + [12] * 3
    for i in range(l):
        expect = vals[:, : cache_len + ends[i]].mean(1)
        torch.testing.assert_close(got[:, i], expect, rtol=0, atol=1e-6)


def test_one_hot_values_read_out_probabilities():
    """v[j] = e_j => out[i, j] = P(i attends j); future-block probabilities are exactly 0."""
    g = torch.Generator().manual_seed(9)
    l, d = 48, 64
    q = torch.randn(1, l, 1, d, generator=g)
    k = torch.randn(1, l, 1, d, generator=g)
    v = torch.zeros(1, l, 1, d)
    v[0, torch.arange(l), 0, torch.arange(l)] = 1.0
    p = oatt.blockwise_causal_attention(q, k, v, None, 0, torch.tensor([0, 16, 32]), None)[0, :, 0, :l]
    for blk in range(3):
        rows = p[16 * blk:16 * (blk + 1)]
        assert torch.equal(rows[:, 16 * (blk + 1):], torch.zeros_like(rows[:, 16 * (blk + 1):]))
        torch.testing.assert_close(rows.sum(1), torch.ones(16), rtol=0, atol=1e-6)


def test_future_blocks_are_invisible_bit_exact():
    inp = _c0_inputs()
    q, k, v = inp.q, inp.k, inp.v
    bb = torch.tensor([0, 16, 32])
    base = oatt.blockwise_causal_attention(q, k, v, None, 0, bb, None)
    k2, v2 = k.clone(), v.clone()
    k2[:, 32:] += 7.0
    v2[:, 32:] = -v2[:, 32:] * 3.0
    other = oatt.blockwise_causal_attention(q, k2, v2, None, 0, bb, None)
    assert torch.equal(base[:, :32], other[:, :32])
    assert not torch.equal(base[:, 32:], other[:, 32:])


def test_rows_before_first_block_are_nan_without_cache():
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 12, 2, 16, generator=g) for _ in range(3))
    out = oatt.blockwise_causal_attention(q, k, v, None, 0, torch.tensor([4, 8]), None)
    assert torch.isnan(out[:, :4]).all()
    assert torch.isfinite(out[:, 4:]).all()
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), starts=[4, 8])
    assert np.isnan(ref[:, :4]).all()


def test_output_dtype_follows_q():
    q = torch.randn(1, 8, 2, 16).bfloat16()
    out = oatt.blockwise_causal_attention(q, q, q)
    assert out.dtype == torch.bfloat16
    assert oatt.blockwise_causal_attention(q, q, q, keep_fp32=True).dtype == torch.float32


# ------------------------------------------ cross-attention and GQA -----

def _cross_inputs(seed=3, b=2, lq=7, lk=19, h=4, hkv=4, d=16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, lq, h, d, generator=g)
    k = torch.randn(b, lk, hkv, d, generator=g)
    v = torch.randn(b, lk, hkv, d, generator=g)
    return q, k, v


@pytest.mark.parametrize("lk", [1, 5, 19, 70])
def test_cross_attention_matches_brute_force_and_sdpa(lk):
    """kv_len != q_len without a mask: every key visible, against the fp64 brute force
    and torch's scaled_dot_product_attention with no mask."""
    q, k, v = _cross_inputs(lk=lk)
    got = oatt.blockwise_causal_attention(q, k, v, keep_fp32=True)
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)
    sd = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    torch.testing.assert_close(got, sd.transpose(1, 2), rtol=1e-5, atol=1e-5)


def test_cross_attention_with_cache_sees_cache_then_keys():
    q, k, v = _cross_inputs(lk=11)
    cache = torch.randn(2, 2, 9, 4, 16)
    got = oatt.blockwise_causal_attention(q, k, v, cache, 6, keep_fp32=True)
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), cache[0].numpy(), cache[1].numpy(), 6)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)


def test_cross_attention_refuses_a_mask():
    q, k, v = _cross_inputs(lk=9)
    with pytest.raises(ValueError):
        oatt.blockwise_causal_attention(q, k, v, causal=True)
    with pytest.raises(ValueError):
        oatt.blockwise_causal_attention(q, k, v, block_boundaries=torch.tensor([0, 4]))


@pytest.mark.parametrize("hkv", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_matches_brute_force_and_sdpa(hkv, causal):
    """k/v heads shared by H/Hkv query heads: fp64 brute force (explicit head index)
    and sdpa(enable_gqa=True)."""
    q, k, v = _cross_inputs(lk=7, h=4, hkv=hkv)
    got = oatt.blockwise_causal_attention(q, k, v, causal=causal, keep_fp32=True)
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), causal=causal)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)
    sd = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                        is_causal=causal, enable_gqa=True)
    torch.testing.assert_close(got, sd.transpose(1, 2), rtol=1e-5, atol=1e-5)


def test_gqa_head_map_is_interleaved_not_tiled():
    """Query head h reads k/v head h // (H/Hkv) (repeat_interleave), not h % Hkv
    (repeat): a planted tiling fails the brute force."""
    q, k, v = _cross_inputs(lk=7, h=4, hkv=2)
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy())
    tiled = oatt.blockwise_causal_attention(q, k.repeat(1, 1, 2, 1), v.repeat(1, 1, 2, 1),
                                            keep_fp32=True)
    assert not np.allclose(tiled.numpy(), ref, atol=1e-3)


# ---------------------------------------------------------------- rope -----

def _bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.float32).to(torch.bfloat16).to(torch.float64).numpy()


def _rope_inputs(seed=0, b=1, l=6, h=3, d=16, dtype=torch.bfloat16):
    from dexter_amd.bench.workloads import rope_table
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, l, h, d, generator=g).to(dtype)
    k = torch.randn(b, l, h, d, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(h * d, generator=g)).to(dtype)
    cos, sin = rope_table(torch.arange(l) + 3, d)
    return q, k, w, cos, sin


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_matches_fp64_with_the_reference_rounding(interleaved):
    q, k, w, cos, sin = _rope_inputs()
    got_q, _ = orope.qk_norm_rope(q, k, w, w, cos, sin, 1e-6, interleaved, keep_fp32=True)
    ref = brute.qk_norm_rope(q.float().numpy(), w.float().numpy(), cos.numpy(), sin.numpy(),
                             1e-6, interleaved, round_to=_bf16_round)
    # fp32 arithmetic on bf16-rounded operands: agreement to a few fp32 ulps,
    # except where the fp32 norm lands on the other side of a bf16 rounding tie.
    diff = np.abs(got_q.numpy() - ref)
    assert np.quantile(diff, 0.99) < 1e-5
    assert diff.max() < 2e-2


def test_rope_identity_rotation_is_plain_rms_norm():
    q, k, w, cos, sin = _rope_inputs(l=4)
    one, zero = torch.ones_like(cos), torch.zeros_like(sin)
    got, _ = orope.qk_norm_rope(q, k, w, w, one, zero, 1e-6, True, keep_fp32=True)
    plane = q.float().reshape(1, 4, -1)
    expect = (plane / torch.sqrt(plane.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float())
    expect = expect.to(torch.bfloat16).float().reshape(q.shape)
    torch.testing.assert_close(got, expect, rtol=0, atol=1e-6)


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_preserves_pair_norms(interleaved):
    q, k, w, cos, sin = _rope_inputs(dtype=torch.float32)
    normed = orope.rms_norm(q, w, 1e-6)
    rot = orope.rotary(normed, cos, sin, interleaved)
    if interleaved:
        a = normed[..., 0::2] ** 2 + normed[..., 1::2] ** 2
        b = rot[..., 0::2] ** 2 + rot[..., 1::2] ** 2
    else:
        h = q.shape[-1] // 2
        a = normed[..., :h] ** 2 + normed[..., h:] ** 2
        b = rot[..., :h] ** 2 + rot[..., h:] ** 2
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


def test_unit_weight_gives_unit_plane_rms():
    q, k, _, cos, sin = _rope_inputs(dtype=torch.float32, h=4, d=32)
    w = torch.ones(4 * 32)
    out, _ = orope.qk_norm_rope(q, k, w, w, cos, sin, 0.0, True)
    rms = out.reshape(1, out.shape[1], -1).pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=1e-5, atol=1e-5)


def test_pairings_differ():
    q, k, w, cos, sin = _rope_inputs()
    a, _ = orope.qk_norm_rope(q, k, w, w, cos, sin, 1e-6, True)
    b, _ = orope.qk_norm_rope(q, k, w, w, cos, sin, 1e-6, False)
    assert not torch.allclose(a.float(), b.float(), atol=1e-3)


def test_qkv_project_is_linear():
    """The projection restatement against torch's F.linear (fp32) and a closed form."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 5, 64, generator=g).to(torch.bfloat16)
    w = (torch.randn(48, 64, generator=g) * 0.1).to(torch.bfloat16)
    b = torch.randn(48, generator=g).to(torch.bfloat16)
    got = orope.qkv_project(x, w, b, heads=3, keep_fp64=True)
    lib = F.linear(x.float(), w.float(), b.float()).reshape(2, 5, 3, 16)
    torch.testing.assert_close(got.float(), lib, rtol=1e-5, atol=1e-5)
    eye = torch.eye(64, dtype=torch.bfloat16)
    same = orope.qkv_project(x, eye, None, heads=4)
    assert torch.equal(same.reshape(2, 5, 64), x)
    assert orope.qkv_project(x, w, b, heads=3).dtype == torch.bfloat16


# ------------------------------------------------------------ kv cache -----

def test_kv_cache_contract():
    c = okv.KVCache(layers=2, batch=1, capacity=10, heads=2, head_dim=8)
    blocks = []
    for step in range(2):
        k = torch.randn(1, 4, 2, 8).bfloat16()
        v = torch.randn(1, 4, 2, 8).bfloat16()
        for layer in range(2):
            c.append(layer, k, v)
        assert c.length == 4 * step  # append does not move the cursor
        c.commit(4)
        blocks.append((k, v))
    assert torch.equal(c.cache[1][0, :, :8], torch.cat([b[0] for b in blocks], 1))
    assert torch.equal(c.cache[1][1, :, :8], torch.cat([b[1] for b in blocks], 1))
    with pytest.raises(RuntimeError, match="KV cache full"):
        c.append(0, torch.zeros(1, 4, 2, 8).bfloat16(), torch.zeros(1, 4, 2, 8).bfloat16())
    c.reset()
    assert c.length == 0


# --------------------------------------------- the pins catch mistakes -----

def _planted_scale_dropped(q, k, v, *a, **kw):
    return oatt.blockwise_causal_attention(q, k, v, *a[:3], softmax_scale=1.0, **kw)


def _planted_mask_one_block_late(q, k, v, kv_cache, cache_len, bb, scale):
    shifted = None if bb is None else torch.cat((bb[:1], bb[2:]))
    return oatt.blockwise_causal_attention(q, k, v, kv_cache, cache_len, shifted, scale)


def _planted_kt_not_transposed(q, k, v, kv_cache, cache_len, bb, scale):
    # Keys read with head and position swapped: a transposed operand.
    return oatt.blockwise_causal_attention(q, k.transpose(1, 2).reshape(k.shape), v,
                                           kv_cache, cache_len, bb, scale)


@pytest.mark.parametrize("planted", [_planted_scale_dropped, _planted_mask_one_block_late,
                                     _planted_kt_not_transposed])
def test_brute_force_pin_catches_planted_mistakes(planted):
    inp = _c0_inputs()
    bb = torch.tensor([0, 16, 32])
    got = planted(inp.q, inp.k, inp.v, None, 0, bb, None)
    ref = brute.attention(inp.q.numpy(), inp.k.numpy(), inp.v.numpy(), starts=[0, 16, 32])
    assert not np.allclose(got.numpy(), ref, atol=1e-3)


def test_rounding_pin_catches_a_lost_rounding_step():
    q, k, w, cos, sin = _rope_inputs(l=16, h=4, d=32)
    no_round = brute.qk_norm_rope(q.float().numpy(), w.float().numpy(), cos.numpy(), sin.numpy(),
                                  1e-6, True)
    got, _ = orope.qk_norm_rope(q, k, w, w, cos, sin, 1e-6, True, keep_fp32=True)
    # Without the reference's bf16 rounding after the norm the fp32 results
    # differ by far more than fp32 arithmetic noise.
    assert np.quantile(np.abs(got.numpy() - no_round), 0.5) > 1e-4


def test_scale_default_is_inverse_sqrt_head_dim():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(1, 8, 1, 16, generator=g) for _ in range(3))
    a = oatt.blockwise_causal_attention(q, k, v)
    b = oatt.blockwise_causal_attention(q, k, v, softmax_scale=1 / math.sqrt(16))
    assert torch.equal(a, b)


# ---------------------------------------------------- adaLN / gated residual -----

def _norm_inputs(seed=0, b=2, l=5, c=64, dtype=torch.bfloat16, mod_rows=1):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, l, c, generator=g).to(dtype)
    scale = torch.randn(b, mod_rows, c, generator=g).to(dtype)
    shift = torch.randn(b, mod_rows, c, generator=g).to(dtype)
    return x, scale, shift


def _adaln_known_case():
    """x = [0, 1, 2, 3]: mean 1.5, biased variance 1.25; with eps 0.75 the
    denominator is sqrt(2). Gains 1 + scale = [2, 1, 0, 1.5]."""
    x = torch.tensor([[0.0, 1.0, 2.0, 3.0]], dtype=torch.float64)
    scale = torch.tensor([1.0, 0.0, -1.0, 0.5], dtype=torch.float64)
    shift = torch.tensor([0.0, 1.0, 2.0, 3.0], dtype=torch.float64)
    r2 = math.sqrt(2.0)
    expect = torch.tensor([[-1.5 / r2 * 2, -0.5 / r2 + 1, 2.0, 1.5 / r2 * 1.5 + 3]],
                          dtype=torch.float64)
    return x, scale, shift, 0.75, expect


def test_adaln_known_answer():
    x, scale, shift, eps, expect = _adaln_known_case()
    got = onorm.adaln_modulate_exact(x, scale, shift, eps)
    torch.testing.assert_close(got, expect, rtol=0, atol=1e-12)
    got = onorm.adaln_modulate(x.float(), scale.float(), shift.float(), eps)
    torch.testing.assert_close(got.double(), expect, rtol=0, atol=1e-6)
    got = brute.adaln_modulate(x.numpy(), scale.numpy(), shift.numpy(), eps)
    np.testing.assert_allclose(got, expect.numpy(), rtol=0, atol=1e-12)


def test_adaln_zero_modulation_is_layer_norm():
    x, _, _ = _norm_inputs(dtype=torch.float64)
    zero = torch.zeros(x.shape[-1], dtype=torch.float64)
    lib = F.layer_norm(x, (x.shape[-1],), eps=1e-6)
    torch.testing.assert_close(onorm.adaln_modulate_exact(x, zero, zero), lib, rtol=0, atol=1e-12)
    torch.testing.assert_close(torch.from_numpy(brute.adaln_modulate(x.numpy(), 0.0, 0.0)), lib,
                               rtol=0, atol=1e-12)


def test_adaln_exact_matches_fp64_brute_force():
    x, scale, shift = _norm_inputs(c=96)
    got = onorm.adaln_modulate_exact(x, scale, shift, 1e-6, out_dtype=torch.float64)
    ref = brute.adaln_modulate(x.double().numpy(), scale.double().numpy(), shift.double().numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-12)


def test_adaln_matches_fp64_with_the_reference_rounding():
    x, scale, shift = _norm_inputs(c=128, l=8)
    got = onorm.adaln_modulate(x, scale, shift).double().numpy()
    ref = brute.adaln_modulate(x.double().numpy(), scale.double().numpy(), shift.double().numpy(),
                               round_to=_bf16_round)
    # torch normalises in fp32 before its bf16 rounding, the brute force in
    # fp64: a rare element lands on the other side of a rounding tie.
    assert np.mean(got == ref) > 0.99
    assert np.abs(got - ref).max() <= 0.05 * np.abs(ref).max()


def test_adaln_output_dtype_is_the_promotion():
    x, scale, shift = _norm_inputs()
    assert onorm.adaln_modulate(x, scale, shift).dtype == torch.bfloat16
    assert onorm.adaln_modulate(x, scale.float(), shift.float()).dtype == torch.float32
    assert onorm.adaln_modulate_exact(x, scale.half(), shift.half()).dtype == torch.float32


def test_adaln_shift_of_x_changes_nothing():
    x, scale, shift = _norm_inputs(dtype=torch.float64)
    a = onorm.adaln_modulate_exact(x, scale, shift)
    b = onorm.adaln_modulate_exact(x + 7.0, scale, shift)
    torch.testing.assert_close(a, b, rtol=0, atol=1e-9)


def test_gated_residual_closed_forms():
    x, y, _ = _norm_inputs()
    zero, one = torch.zeros(1, 1, x.shape[-1]), torch.ones(1, 1, x.shape[-1])
    assert torch.equal(onorm.gated_residual_fp32(x, y, zero.bfloat16()), x)
    assert torch.equal(onorm.gated_residual(x, y, zero.bfloat16()), x)
    assert torch.equal(onorm.gated_residual_fp32(x, y, one.bfloat16()), x + y)


def test_gated_residual_matches_fp64_brute_force():
    x, y, g = _norm_inputs(l=16, c=128)
    ref = brute.gated_residual(x.double().numpy(), y.double().numpy(), g.double().numpy())
    got = onorm.gated_residual_fp32(x.float(), y.float(), g.float()).double().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    chain = onorm.gated_residual(x, y, g).double().numpy()
    ref_r = brute.gated_residual(x.double().numpy(), y.double().numpy(), g.double().numpy(),
                                 round_to=_bf16_round)
    assert np.mean(chain == ref_r) > 0.999
    single = onorm.gated_residual_fp32(x, y, g).double().numpy()
    # One rounding vs two: the single-rounding form is closer to the exact sum.
    assert np.abs(single - ref).mean() < np.abs(chain - ref).mean()


def _planted_unbiased_variance(x, scale, shift, eps):
    xd = x.double()
    mean = xd.mean(-1, keepdim=True)
    var = (xd - mean).pow(2).sum(-1, keepdim=True) / (xd.shape[-1] - 1)
    return (xd - mean) / torch.sqrt(var + eps) * (1 + scale) + shift


def _planted_gain_without_one(x, scale, shift, eps):
    return onorm.adaln_modulate_exact(x, scale - 1, shift, eps)


def _planted_eps_outside_sqrt(x, scale, shift, eps):
    xd = x.double()
    mean = xd.mean(-1, keepdim=True)
    var = (xd - mean).pow(2).mean(-1, keepdim=True)
    return (xd - mean) / (torch.sqrt(var) + eps) * (1 + scale) + shift


@pytest.mark.parametrize("planted", [_planted_unbiased_variance, _planted_gain_without_one,
                                     _planted_eps_outside_sqrt])
def test_adaln_known_answer_catches_planted_mistakes(planted):
    x, scale, shift, eps, expect = _adaln_known_case()
    assert not torch.allclose(planted(x, scale, shift, eps), expect, atol=1e-3)
