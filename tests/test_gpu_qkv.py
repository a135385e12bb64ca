"""Fused QKV projection + QK-norm + rotary + cache write (MI355X).

``ops.qkv_norm_rope`` against the oracle: the fp64 projection
(``oracle.rope.qkv_project``) then the reference prologue
(``oracle.rope.qk_norm_rope``). The HIP projection accumulates in fp32 over
split-K partials, in another order than the oracle, so:

* ``v`` (the projection itself) is within one bf16 ulp of the fp64 result plus
  the fp32 accumulation error, 2^-18 of the sum of |x w| over the row;
* ``q``/``k`` (after the norm and the rotation) meet the parity bar against the
  oracle run on the oracle's projection: mean-abs 2e-3, and an error of at most
  2e-2 x max(1, |ref|) (the normalised outputs reach |4|-|5|, where one bf16 ulp
  is 0.03: a one-ulp difference in the projection, from the fp32 summation
  order, can surface as one ulp of the output);
* the cache rows equal ``k``/``v`` bit for bit, at a host start and at a device
  cursor, and the call equals the unfused HIP path (three ``F.linear`` + the
  prologue) within the parity bar.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import dexter_amd.ops as ops
from dexter_amd.bench.workloads import rope_table
from dexter_amd.registry import select_spec
from oracle import rope as orope

from _util import assert_parity, assert_parity_scaled

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _setup(b, l, c, heads, dim, dtype=DT, bias=True, seed=0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    hd = heads * dim
    x = torch.randn(b, l, c, generator=g).to(dtype)
    ws = [(torch.randn(hd, c, generator=g) * c ** -0.5).to(dtype) for _ in range(3)]
    bs = [torch.randn(hd, generator=g).mul(0.1).to(dtype) if bias else None for _ in range(3)]
    nq = (1 + 0.1 * torch.randn(hd, generator=g)).to(dtype)
    nk = (1 + 0.1 * torch.randn(hd, generator=g)).to(dtype)
    cos, sin = rope_table(torch.arange(l) + 17, dim)
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    return (dev(x), [dev(w) for w in ws], [dev(t) for t in bs], dev(nq), dev(nk),
            dev(cos), dev(sin))


def _oracle(x, ws, bs, nq, nk, cos, sin, heads, interleaved=True):
    cpu = lambda t: None if t is None else t.cpu()  # noqa: E731
    q, k, v = (orope.qkv_project(cpu(x), cpu(w), cpu(b), heads) for w, b in zip(ws, bs))
    v64 = orope.qkv_project(cpu(x), cpu(ws[2]), cpu(bs[2]), heads, keep_fp64=True)
    mag = (cpu(x).double().abs() @ cpu(ws[2]).double().abs().t()).reshape(v64.shape)
    rq, rk = orope.qk_norm_rope(q, k, cpu(nq), cpu(nk), cpu(cos), cpu(sin), 1e-6, interleaved,
                                keep_fp32=True)
    return rq, rk, v64, mag


def _check(got, ref, what):
    rq, rk, v64, mag = ref
    q, k, v = got
    assert_parity_scaled(q, rq, what=f"{what} q")
    assert_parity_scaled(k, rk, what=f"{what} k")
    fi = torch.finfo(v.dtype)
    e = v64.abs().clamp_min(fi.tiny)
    ulp = torch.exp2(torch.floor(torch.log2(e))) * fi.eps
    err = (v.cpu().double() - v64).abs()
    bad = err > ulp + 2.0 ** -18 * mag
    assert not bad.any(), f"{what} v: {int(bad.sum())} elements beyond one ulp"


def test_selects_the_hip_kernel(device, built_lib):
    x, ws, bs, nq, nk, cos, sin = _setup(1, 8, 512, 2, 64)
    spec = select_spec("rope", "qkv_norm_rope", x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2],
                       nq, nk, cos, sin, 2)
    assert spec.name == "hip_qkv_norm_rope_gfx950"


@pytest.mark.parametrize("bias", [True, False])
def test_wan5b_chunk(device, built_lib, bias):
    """The C1 chunk: 83 tokens of 3072 channels, 24 heads x 128."""
    args = _setup(1, 83, 3072, 24, 128, bias=bias, seed=1)
    got = ops.qkv_norm_rope(*args[:1], args[1][0], args[2][0], args[1][1], args[2][1],
                            args[1][2], args[2][2], *args[3:], 24)
    _check(got, _oracle(*args, 24), f"C1 bias={bias}")


@pytest.mark.parametrize("b,l,c,heads,dim,dtype,interleaved", [
    (1, 1, 3072, 24, 128, DT, True),
    (1, 32, 3072, 24, 128, DT, True),
    (1, 33, 1024, 8, 128, DT, False),
    (2, 48, 2048, 16, 128, torch.float16, True),
    (4, 32, 3072, 48, 64, DT, True),
    (1, 128, 5120, 40, 128, DT, True),
    (1, 96, 1536, 6, 64, torch.float16, False),
])
def test_shapes(device, built_lib, b, l, c, heads, dim, dtype, interleaved):
    args = _setup(b, l, c, heads, dim, dtype=dtype, seed=l + c)
    x, ws, bs, nq, nk, cos, sin = args
    got = ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin, heads,
                            1e-6, interleaved)
    _check(got, _oracle(*args, heads, interleaved), f"{b}x{l}x{c} {heads}x{dim}")


def test_cache_write_host_and_device_cursor(device, built_lib):
    heads, dim, cap = 24, 128, 300
    x, ws, bs, nq, nk, cos, sin = _setup(1, 83, 3072, heads, dim, seed=5)
    a = torch.zeros(2, 1, cap, heads, dim, dtype=DT, device=device)
    b = torch.zeros_like(a)
    q1, k1, v1 = ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin,
                                   heads, cache=a, start=100)
    assert torch.equal(a[0, :, 100:183], k1) and torch.equal(a[1, :, 100:183], v1)
    assert torch.count_nonzero(a[:, :, :100]) == 0 and torch.count_nonzero(a[:, :, 183:]) == 0
    cursor = torch.tensor([100], dtype=torch.int32, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    q2, k2, v2 = ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin,
                                   heads, cache=b, start=cursor, status=status)
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(a, b) and int(status.item()) == 0
    cursor.fill_(cap - 50)  # does not fit: nothing written, status set
    before = b.clone()
    ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin, heads,
                      cache=b, start=cursor, status=status)
    assert torch.equal(b, before) and int(status.item()) == 1
    with pytest.raises(RuntimeError, match="KV cache full"):
        ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin, heads,
                          cache=a, start=cap - 50)


def test_matches_the_unfused_path(device, built_lib):
    """Three F.linear (hipBLASLt) + the HIP prologue, the path the fused call replaces."""
    heads, dim = 24, 128
    x, ws, bs, nq, nk, cos, sin = _setup(1, 83, 3072, heads, dim, seed=9)
    q, k, v = (F.linear(x, w, b).view(1, 83, heads, dim) for w, b in zip(ws, bs))
    uq, uk = ops.qk_norm_rope(q, k, nq, nk, cos, sin)
    fq, fk, fv = ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin,
                                   heads)
    assert_parity_scaled(fq, uq.float(), what="q vs unfused")
    assert_parity_scaled(fk, uk.float(), what="k vs unfused")
    assert_parity_scaled(fv, v.float(), what="v vs unfused")


QKV_SHAPES = [(1, 83, 3072, 24, 128), (1, 128, 5120, 40, 128), (2, 16, 512, 1, 128),
              (1, 96, 1536, 6, 64), (1, 1, 8192, 1, 128)]


@pytest.mark.parametrize("b,l,c,heads,dim", QKV_SHAPES)
def test_repeats_bit_for_bit(device, built_lib, b, l, c, heads, dim):
    """Repeated calls give the same bits (the split-K partials are summed in
    split order), and meet the bar against the oracle: 83 and 128 tokens, one
    token over 8,192 channels, head_dim 64 and 128."""
    args = _setup(b, l, c, heads, dim, seed=b * l + c)
    x, ws, bs, nq, nk, cos, sin = args
    call = lambda: ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk,  # noqa: E731
                                     cos, sin, heads)
    first = call()
    for _ in range(3):
        again = call()
        assert all(torch.equal(u, w) for u, w in zip(first, again))
    _check(first, _oracle(*args, heads), f"{b}x{l}x{c} {heads}x{dim}")


def test_graph_replays(device, built_lib):
    """Captured once, replayed with eager calls in between: every replay equals
    the eager result bit for bit."""
    from dexter_amd.bench import harness
    heads, dim = 24, 128
    x, ws, bs, nq, nk, cos, sin = _setup(1, 83, 3072, heads, dim, seed=13)
    outs = []

    def step():
        outs.clear()
        outs.extend(ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos,
                                      sin, heads))
    step()
    eager = [t.clone() for t in outs]
    graph = harness.capture(step)
    captured = list(outs)  # the graph's own output buffers
    for _ in range(3):
        for t in captured:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(u, w) for u, w in zip(captured, eager))
        step()
        torch.cuda.synchronize()


@pytest.mark.parametrize("waves", [2, 4])
def test_register_ring_form_under_tuning(device, built_lib, waves):
    """dx_set_tuning(DX_TUNE_QKV_WAVES, 2 or 4) selects the register-ring GEMM
    (weights through registers into per-wave LDS chunks) instead of the DMA
    form: it meets the same bar, at 83 and 128 tokens."""
    from dexter_amd.ops.gfx950 import _lib
    for shape in [(1, 83, 3072, 24, 128), (4, 32, 3072, 48, 64)]:
        args = _setup(*shape, seed=shape[1] + waves)
        x, ws, bs, nq, nk, cos, sin = args
        with _lib.tuning(_lib.TUNE_QKV_WAVES, waves):
            got = ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos,
                                    sin, shape[3])
        _check(got, _oracle(*args, shape[3]), f"ring{waves} {shape}")


def test_rejects_long_chunks(device, built_lib):
    x, ws, bs, nq, nk, cos, sin = _setup(1, 129, 512, 2, 64)
    with pytest.raises(LookupError):
        ops.qkv_norm_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], nq, nk, cos, sin, 2)


@pytest.mark.parametrize("write", [False, True])
def test_self_attention_fused_projection_matches_unfused(device, built_lib, write):
    """SelfAttention over a decode chunk with and without the fused projection."""
    from dexter_amd.models import KVCache, SelfAttention
    torch.manual_seed(3)
    dim, heads, rows = 1024, 8, 83
    layer = SelfAttention(dim, heads, dtype=DT, device=device)
    with torch.no_grad():
        for lin in (layer.q, layer.k, layer.v, layer.o):
            lin.weight.normal_(0, dim ** -0.5)
        layer.q_norm.copy_(1 + 0.1 * torch.randn(dim))
        layer.k_norm.copy_(1 + 0.1 * torch.randn(dim))
    cos, sin = (t.to(device) for t in rope_table(torch.arange(rows) + 83, dim // heads))
    caches = [KVCache(1, 1, 300, heads, dim // heads, device, DT) for _ in range(2)]
    hist = _setup(1, 83, dim, heads, dim // heads, seed=21)[0]
    for c in caches:  # the same history through the unfused path
        layer(hist, cos, sin, c, 0, write=True, fused_qkv=False)
        c.commit(rows)
    x = torch.randn(1, rows, dim, device=device).to(DT)
    fused = layer(x, cos, sin, caches[0], 0, write=write, fused_qkv=True)
    plain = layer(x, cos, sin, caches[1], 0, write=write, fused_qkv=False)
    assert_parity_scaled(fused, plain.float(), what=f"write={write}")
    if write:
        assert_parity_scaled(caches[0].cache[0][:, :, 83:166], caches[1].cache[0][:, :, 83:166].float(),
                             what="appended rows")
