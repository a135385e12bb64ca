"""The five measured configurations end to end (MI355X), at their full sizes.

Each config runs the path the way the model does: prologue (QK-RMSNorm +
RoPE) over the history, appended into the cache, then the current chunk's
prologue and attention over cache + chunk. Checks, per config:

* the chained result against the oracle chain on the same seeded inputs;
* attention alone on identical bf16 q/k/v/cache against the fp32 oracle;
* size-independent properties: future-block perturbation leaves earlier
  rows bit-identical (C2), per-sequence agreement of the ragged batch (C4).

C0 is the reference's CPU plumbing case; here its inputs are cast to bf16 and
run through the HIP kernel. For C2/C3 the fp32 oracle runs on the GPU (torch,
a few heads at a time) because the CPU would need minutes.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.bench.workloads import CONFIGS, block_tensor, make_inputs
from oracle import attention as oatt
from oracle import rope as orope

from _util import assert_parity, assert_parity_scaled, assert_within_ulp

pytestmark = pytest.mark.gpu


def _oracle_attention_chunked(q, k, v, cache, cache_len, bb, heads_per_chunk=4):
    """fp32 oracle on q's device, a few heads at a time (bounded memory).

    On the GPU the oracle's products are torch's fp32 GEMMs, which must stay
    full fp32: TF32 (xf32 on ROCm) would round their operands to 10-bit
    mantissas, a coarser reference than the bf16 kernel it checks.
    """
    if q.is_cuda:
        assert not torch.backends.cuda.matmul.allow_tf32, "oracle GEMMs must be full fp32"
        assert torch.get_float32_matmul_precision() == "highest", "oracle GEMMs must be full fp32"
    outs = []
    for h0 in range(0, q.shape[2], heads_per_chunk):
        hs = slice(h0, h0 + heads_per_chunk)
        c = None if cache is None else cache[:, :, :, hs]
        outs.append(oatt.blockwise_causal_attention(q[:, :, hs], k[:, :, hs], v[:, :, hs], c,
                                                    cache_len, bb, None, keep_fp32=True))
    return torch.cat(outs, dim=2)


def _prologue_and_cache(inp, device, cache_len, capacity):
    """HIP prologue over positions [0, cache_len), appended into a fresh cache."""
    cfg = inp.cfg
    q, k, v = inp.q.to(device), inp.k.to(device), inp.v.to(device)
    qw, kw = inp.q_weight.to(device), inp.k_weight.to(device)
    cos, sin = inp.cos.to(device), inp.sin.to(device)
    cache = torch.zeros(2, cfg.batch, capacity, cfg.heads, cfg.head_dim, dtype=cfg.dtype,
                        device=device)
    if cache_len:
        _, kr = ops.qk_norm_rope(q[:, :cache_len], k[:, :cache_len], qw, kw, cos[:cache_len],
                                 sin[:cache_len])
        ops.kv_cache_append(cache, kr, v[:, :cache_len], 0)
    return q, k, v, qw, kw, cos, sin, cache


def test_c0_plumbing_case_in_bf16(device, built_lib):
    cfg = CONFIGS["C0"]
    inp = make_inputs(cfg)
    q, k, v = (t.to(torch.bfloat16) for t in (inp.q, inp.k, inp.v))
    bb = torch.tensor(cfg.block_starts)
    got = ops.blockwise_causal_attention(q.to(device), k.to(device), v.to(device),
                                         block_boundaries=bb.to(device))
    ref = oatt.blockwise_causal_attention(q, k, v, None, 0, bb, None, keep_fp32=True)
    assert_parity(got, ref, what="C0")


def test_c1_wan5b_chunk_chain(device, built_lib):
    cfg = CONFIGS["C1"]
    inp = make_inputs(cfg)
    c = cfg.cache_lens[0]
    q, k, v, qw, kw, cos, sin, cache = _prologue_and_cache(inp, device, c, c + cfg.q_len)
    qc, kc = ops.qk_norm_rope(q[:, c:], k[:, c:], qw, kw, cos[c:], sin[c:])
    got = ops.blockwise_causal_attention(qc, kc, v[:, c:], kv_cache=cache, cache_len=c)

    # Oracle chain from the same pre-norm activations.
    rq, rk = orope.qk_norm_rope(inp.q, inp.k, inp.q_weight, inp.k_weight, inp.cos, inp.sin, 1e-6)
    ocache = torch.stack((rk[:, :c], inp.v[:, :c]))
    ref = oatt.blockwise_causal_attention(rq[:, c:], rk[:, c:], inp.v[:, c:], ocache, c, None,
                                          None, keep_fp32=True)
    assert_parity(got, ref, what="C1 chain")
    # Attention alone on the kernel's own bf16 inputs.
    alone = oatt.blockwise_causal_attention(qc.cpu(), kc.cpu(), inp.v[:, c:], cache.cpu(), c, None,
                                            None, keep_fp32=True)
    assert_parity(got, alone, what="C1 attention")


def test_c2_wan5b_prefill(device, built_lib):
    cfg = CONFIGS["C2"]
    inp = make_inputs(cfg)
    q, k, v, qw, kw, cos, sin, _ = _prologue_and_cache(inp, device, 0, 1)
    qr, kr = ops.qk_norm_rope(q, k, qw, kw, cos, sin)
    bb = block_tensor(cfg, device)
    got = ops.blockwise_causal_attention(qr, kr, v, block_boundaries=bb)
    ref = _oracle_attention_chunked(qr, kr, v, None, 0, bb)
    assert_parity(got, ref, what="C2 attention")
    # The prologue at full size against the CPU oracle.
    rq, rk = orope.qk_norm_rope(inp.q, inp.k, inp.q_weight, inp.k_weight, inp.cos, inp.sin, 1e-6)
    assert_parity(qr, rq, max_abs=0.07, mean_abs=1e-4, what="C2 prologue q")
    assert (qr.cpu() == rq).float().mean().item() > 0.99
    # Block causality at full size: rewriting block 7 leaves blocks 0-6 bit-identical.
    k2 = kr.clone()
    v2 = v.clone()
    k2[:, 7168:] = k2[:, 7168:].flip(1)
    v2[:, 7168:] = -v2[:, 7168:]
    other = ops.blockwise_causal_attention(qr, k2, v2, block_boundaries=bb)
    assert torch.equal(got[:, :7168], other[:, :7168])


def test_c3_wan14b_chunk(device, built_lib):
    cfg = CONFIGS["C3"]
    inp = make_inputs(cfg)
    c = cfg.cache_lens[0]
    q, k, v, qw, kw, cos, sin, cache = _prologue_and_cache(inp, device, c, c + cfg.q_len)
    qc, kc = ops.qk_norm_rope(q[:, c:], k[:, c:], qw, kw, cos[c:], sin[c:])
    got = ops.blockwise_causal_attention(qc, kc, v[:, c:], kv_cache=cache, cache_len=c)
    ref = _oracle_attention_chunked(qc, kc, v[:, c:], cache, c, None)
    assert_parity(got, ref, what="C3 attention")


def test_c4_ragged_batch(device, built_lib):
    cfg = CONFIGS["C4"]
    inp = make_inputs(cfg)
    lens = list(cfg.cache_lens)
    b, h, d = cfg.batch, cfg.heads, cfg.head_dim
    cache = torch.zeros(2, b, max(lens), h, d, dtype=cfg.dtype)
    kq = torch.zeros(b, cfg.q_len, h, d, dtype=cfg.dtype)
    vq = torch.zeros_like(kq)
    for i, c in enumerate(lens):
        cache[0, i, :c] = inp.k[i, :c]
        cache[1, i, :c] = inp.v[i, :c]
        kq[i] = inp.k[i, c:c + cfg.q_len]
        vq[i] = inp.v[i, c:c + cfg.q_len]
    bb = block_tensor(cfg, device)
    got = ops.blockwise_causal_attention_varlen(inp.q.to(device), kq.to(device), vq.to(device),
                                                kv_cache=cache.to(device), cache_lens=lens,
                                                block_boundaries=bb)
    for i, c in enumerate(lens):
        ref = oatt.blockwise_causal_attention(inp.q[i:i + 1], kq[i:i + 1], vq[i:i + 1],
                                              cache[:, i:i + 1], c, torch.tensor(cfg.block_starts),
                                              None, keep_fp32=True)
        # x20 outliers push |out| to tens: the bf16 output alone rounds by
        # up to 2^-9 |out|, so the max-abs bar scales with |ref| above 1.
        assert_parity_scaled(got[i:i + 1], ref, what=f"C4 seq {i} (cache {c})")
        # Strict beside it: within one bf16 spacing of the rounded oracle.
        assert_within_ulp(got[i:i + 1], ref, what=f"C4 seq {i} (cache {c})")
