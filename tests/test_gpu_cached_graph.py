"""Device-resident cache cursor and graph replay of cache-writing steps (MI355X).

The ``dx_*_dev`` entry points read the cache length (attention) or start row
(appends) from an int32 in device memory when the kernels run. Checked here:

* each device-cursor op against its host-length form: appends bit-exact,
  attention against the oracle (its launch is planned for the whole capacity,
  so its split count, and with it the last bits, may differ);
* out-of-range cursors: attention clamps to [0, capacity]; an append that
  would not fit writes nothing and sets the status word;
* ``CachedStepGraph``: one capture of a cache-writing step of three
  self-attention layers, replayed over an episode, against the same layers run
  eagerly with host lengths: caches bit-exact, outputs at the parity bar, and
  the host-side overflow error when the episode fills the cache.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.bench.workloads import rope_table
from dexter_amd.models import KVCache, SelfAttention
from dexter_amd.runtime import CachedStepGraph, capture
from oracle import attention as oatt

from _util import assert_parity

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _rand(shape, device, scale=1.0, seed=0, dtype=DT):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def _cursor(v, device):
    return torch.tensor([v], dtype=torch.int32, device=device)


def _oracle(q, k, v, cache, cache_len):
    return oatt.blockwise_causal_attention(q.cpu(), k.cpu(), v.cpu(), cache.cpu(), cache_len,
                                           None, None, False, keep_fp32=True)


@pytest.mark.parametrize("length", [0, 1, 700, 1245, 1600])
def test_attention_device_cursor(device, built_lib, length):
    cap = 1600
    cache = _rand((2, 1, cap, 24, 128), device, 0.5, seed=1)
    q = _rand((1, 83, 24, 128), device, 0.3, seed=2)
    k, v = _rand((1, 83, 24, 128), device, seed=3), _rand((1, 83, 24, 128), device, seed=4)
    got = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=_cursor(length, device))
    assert_parity(got, _oracle(q, k, v, cache, length), what=f"cursor {length}")
    host = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=length)
    assert_parity(got, host.float(), what=f"cursor {length} vs host length")


def test_attention_device_cursor_clamps(device, built_lib):
    cap = 300
    cache = _rand((2, 2, cap, 4, 128), device, 0.5, seed=5)
    q = _rand((2, 40, 4, 128), device, 0.3, seed=6)
    k, v = _rand((2, 40, 4, 128), device, seed=7), _rand((2, 40, 4, 128), device, seed=8)
    bb = torch.tensor([0, 20], device=device)
    high = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=_cursor(10**6, device),
                                          block_boundaries=bb)
    full = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cap,
                                          block_boundaries=bb)
    assert_parity(high, full.float(), what="cursor above capacity")
    low = ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=_cursor(-5, device),
                                         block_boundaries=bb)
    none = ops.blockwise_causal_attention(q, k, v, block_boundaries=bb)
    assert_parity(low, none.float(), what="negative cursor")


def test_attention_device_cursor_rejects_other_dtypes(device, built_lib):
    cache = _rand((2, 1, 64, 2, 128), device)
    q = _rand((1, 8, 2, 128), device)
    with pytest.raises(ValueError, match="int32"):
        ops.blockwise_causal_attention(q, q, q, kv_cache=cache,
                                       cache_len=torch.tensor([3], device=device))
    with pytest.raises(ValueError, match="needs kv_cache"):
        ops.blockwise_causal_attention(q, q, q, cache_len=_cursor(3, device))


def test_kv_append_device_cursor(device, built_lib):
    cap = 64
    k, v = _rand((2, 9, 4, 128), device, seed=9), _rand((2, 9, 4, 128), device, seed=10)
    a = torch.zeros(2, 2, cap, 4, 128, dtype=DT, device=device)
    b = torch.zeros_like(a)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.kv_cache_append(a, k, v, _cursor(17, device), status)
    ops.kv_cache_append(b, k, v, 17)
    assert torch.equal(a, b) and int(status.item()) == 0
    before = a.clone()
    ops.kv_cache_append(a, k, v, _cursor(cap - 5, device), status)  # 9 rows do not fit
    assert torch.equal(a, before) and int(status.item()) == 1
    ops.kv_cache_append(a, k, v, _cursor(cap - 9, device))  # exactly fits; no status given
    assert torch.equal(a[:, :, cap - 9:], torch.stack((k, v)))


def test_prologue_append_device_cursor(device, built_lib):
    b_, l_, h, d, cap = 1, 83, 24, 128, 200
    q, k, v = (_rand((b_, l_, h, d), device, seed=s) for s in (11, 12, 13))
    w = (1 + 0.1 * torch.randn(h * d, generator=torch.Generator().manual_seed(14))).to(DT).to(device)
    cos, sin = (t.to(device) for t in rope_table(torch.arange(l_) + 40, d))
    a = torch.zeros(2, b_, cap, h, d, dtype=DT, device=device)
    b = torch.zeros_like(a)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    qa, ka = ops.qk_norm_rope_append(q, k, v, w, w, cos, sin, a, _cursor(40, device), 1e-6,
                                     True, status)
    qb, kb = ops.qk_norm_rope_append(q, k, v, w, w, cos, sin, b, 40)
    assert torch.equal(qa, qb) and torch.equal(ka, kb) and torch.equal(a, b)
    assert int(status.item()) == 0
    before = a.clone()
    qc, kc = ops.qk_norm_rope_append(q, k, v, w, w, cos, sin, a, _cursor(cap - 10, device), 1e-6,
                                     True, status)
    assert torch.equal(a, before) and int(status.item()) == 1
    assert torch.equal(qc, qa) and torch.equal(kc, ka)  # q and k are still produced


def _layers(n, dim, heads, device, seed=0):
    torch.manual_seed(seed)
    layers = [SelfAttention(dim, heads, device=device) for _ in range(n)]
    for layer in layers:
        with torch.no_grad():
            for lin in (layer.q, layer.k, layer.v, layer.o):
                lin.weight.normal_(0, dim ** -0.5)
            layer.q_norm.normal_(1, 0.1)
            layer.k_norm.normal_(1, 0.1)
    return layers


def test_cached_step_graph_replays_an_episode(device, built_lib):
    """One capture of a cache-writing step, replayed for every block of an episode."""
    n_layers, dim, heads, rows, cap = 3, 1024, 8, 83, 83 * 6
    layers = _layers(n_layers, dim, heads, device)
    cos, sin = (t.to(device) for t in rope_table(torch.arange(rows), dim // heads))
    kv_dev = KVCache(n_layers, 1, cap, heads, dim // heads, device, DT, device_cursor=True)
    kv_host = KVCache(n_layers, 1, cap, heads, dim // heads, device, DT)

    def step(kv):
        def fn(x):
            outs = [layer(x, cos, sin, kv, i, write=True) for i, layer in enumerate(layers)]
            kv.commit(rows)
            return torch.stack(outs)
        return fn

    xs = [_rand((1, rows, dim), device, seed=100 + t) for t in range(6)]
    graph = CachedStepGraph(step(kv_dev), (xs[0],), [kv_dev], rows)
    assert kv_dev.length == 0 and int(kv_dev.cursor.item()) == 0
    for t, x in enumerate(xs):
        (got,) = graph(x)
        want = step(kv_host)(x)
        assert kv_dev.length == kv_host.length == rows * (t + 1)
        assert int(kv_dev.cursor.item()) == kv_dev.length
        for i in range(n_layers):
            assert torch.equal(kv_dev.cache[i], kv_host.cache[i]), f"step {t} layer {i} cache"
        assert_parity(got.float(), want.float(), what=f"step {t}")
    assert not kv_dev.overflowed()
    with pytest.raises(RuntimeError, match="KV cache full"):
        graph(xs[0])


def test_cache_reading_graph_follows_the_cursor(device, built_lib):
    """A captured read-only step (the denoising steps) after the cursor has moved."""
    n_layers, dim, heads, rows, cap = 2, 512, 4, 40, 200
    layers = _layers(n_layers, dim, heads, device, seed=1)
    cos, sin = (t.to(device) for t in rope_table(torch.arange(rows), dim // heads))
    kv = KVCache(n_layers, 1, cap, heads, dim // heads, device, DT, device_cursor=True)

    def read_step(x):
        return torch.stack([layer(x, cos, sin, kv, i, write=False)
                            for i, layer in enumerate(layers)])

    x = _rand((1, rows, dim), device, seed=7)
    runner = capture(read_step, (x,))
    for t in range(3):
        # Eagerly write and commit a block, then replay the captured read.
        blk = _rand((1, rows, dim), device, seed=20 + t)
        for i, layer in enumerate(layers):
            layer(blk, cos, sin, kv, i, write=True)
        kv.commit(rows)
        (got,) = runner(x)
        want = read_step(x)
        assert_parity(got.float(), want.float(), what=f"after {t + 1} blocks")
