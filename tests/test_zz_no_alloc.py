"""The no-allocation attention entry point (dx_blockwise_causal_attention_noalloc)
against the workspace entry point (dx_blockwise_causal_attention), both called
through the C ABI on the same inputs (MI355X).

Both run the same kernels with the same plan, so the outputs must be equal bit
for bit. Two calls in a row, the second smaller, on the default plan and on
the one-launch decode kernel with its in-kernel merge (the plan that uses the
scratch's arrival counters, which every call must leave zero); plus a call
too large for the static scratch, refused before any launch.
"""

from __future__ import annotations

import pytest
import torch

from dexter_amd.ops.gfx950 import _lib

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _rand(shape, device, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(DT).to(device)


def _strides(t):
    return list(t.stride()[:3])


def _call(lib, noalloc, q, k, v, cache, cache_len):
    """One call through the C ABI; returns (rc, out)."""
    b, lq, h, d = q.shape
    out = torch.empty_like(q)
    common = [q.data_ptr(), *_strides(q), k.data_ptr(), *_strides(k), v.data_ptr(), *_strides(v),
              cache.data_ptr(), cache.stride(0), cache.stride(1), cache.stride(2), cache.stride(3),
              out.data_ptr(), *_strides(out), _lib.DX_BF16, b, lq, k.shape[1], h, k.shape[2], d,
              cache_len, None, _lib.DX_I32, 0, 0, float(d) ** -0.5]
    stream = _lib.stream_handle(q.device)
    if noalloc:
        rc = lib.dx_blockwise_causal_attention_noalloc(*common, stream)
    else:
        ws_bytes = lib.dx_attention_workspace_bytes(b, lq, k.shape[1], h, d, cache_len, None)
        assert ws_bytes >= 0
        ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
        rc = lib.dx_blockwise_causal_attention(*common, ws.data_ptr(), ws_bytes, stream)
    return rc, out


def _case(device, b, lq, h, d, cache_len, seed):
    q, k, v = (_rand((b, lq, h, d), device, seed + i) for i in range(3))
    cache = _rand((2, b, cache_len + lq, h, d), device, seed + 3)
    return q, k, v, cache, cache_len


@pytest.mark.parametrize("plan", ["default", "decode in-kernel merge"])
def test_noalloc_matches_workspace_entry(device, built_lib, plan):
    lib = _lib.load()
    kernel, merge = (0, 0) if plan == "default" else (4, 1)
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, kernel), _lib.tuning(_lib.TUNE_ATTN_MERGE, merge):
        # C1's shape (split-KV: the scratch holds partials), then a smaller call.
        for shape, seed in (((1, 83, 24, 128, 1245), 500), ((1, 40, 8, 128, 300), 510)):
            q, k, v, cache, c = _case(device, *shape, seed)
            print(f"no-alloc {plan}: shape {shape}", flush=True)
            rc_ref, ref = _call(lib, False, q, k, v, cache, c)
            _lib.check(rc_ref, "attention")
            rc, got = _call(lib, True, q, k, v, cache, c)
            _lib.check(rc, "attention no-alloc")
            torch.cuda.synchronize()
            assert torch.isfinite(got.float()).all()
            assert torch.equal(got, ref), f"{plan} {shape}: no-alloc differs from the workspace call"
        # The same call again (the scratch keeps the last call's contents).
        rc, again = _call(lib, True, q, k, v, cache, c)
        _lib.check(rc, "attention no-alloc")
        torch.cuda.synchronize()
        assert torch.equal(again, ref)


def test_noalloc_refuses_a_call_beyond_the_scratch(device, built_lib):
    """128 heads x 16 forced splits need ~71 MB of partials: refused with
    DX_EWORKSPACE before any launch (the output is left untouched)."""
    lib = _lib.load()
    q, k, v, cache, c = _case(device, 1, 128, 128, 128, 4096, 520)
    with _lib.tuning(_lib.TUNE_ATTN_SPLITS, 16):
        need = lib.dx_attention_workspace_bytes(1, 128, 128, 128, 128, c, None)
        assert need > (64 << 20)
        out_before = torch.full_like(q, 7.0)
        b, lq, h, d = q.shape
        rc = lib.dx_blockwise_causal_attention_noalloc(
            q.data_ptr(), *_strides(q), k.data_ptr(), *_strides(k), v.data_ptr(), *_strides(v),
            cache.data_ptr(), cache.stride(0), cache.stride(1), cache.stride(2), cache.stride(3),
            out_before.data_ptr(), *_strides(out_before), _lib.DX_BF16, b, lq, lq, h, h, d, c,
            None, _lib.DX_I32, 0, 0, 0.088, _lib.stream_handle(device))
    assert rc == _lib.DX_EWORKSPACE
    assert "static scratch" in lib.dx_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out_before == 7.0).all())


def test_noalloc_first_call_under_graph_capture(device, built_lib, tmp_path):
    """The entry point's first call on a device sets its scratch up (the symbol
    lookup and a counter-clearing kernel on the caller's stream). Here that first
    call is made under graph capture: a private copy of the library is loaded,
    whose static scratch and per-device set-up are its own, so its first call is
    a first call whatever ran before in this process. The graph is replayed
    several times, with eager calls in between, and every replay must equal the
    workspace entry point bit for bit (the one-launch decode kernel, which keeps
    its arrival counters in the scratch)."""
    import ctypes
    import shutil

    copy = tmp_path / "libdexter_gfx950_capture_copy.so"
    shutil.copyfile(built_lib, copy)
    fresh = ctypes.CDLL(str(copy))
    for name, (res, args) in _lib._SIGNATURES.items():
        fn = getattr(fresh, name)
        fn.restype, fn.argtypes = res, args
    lib = _lib.load()
    q, k, v, cache, c = _case(device, 1, 83, 24, 128, 1245, 530)
    b, lq, h, d = q.shape
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, 4), _lib.tuning(_lib.TUNE_ATTN_MERGE, 1):
        fresh.dx_set_tuning(_lib.TUNE_ATTN_KERNEL, 4)
        fresh.dx_set_tuning(_lib.TUNE_ATTN_MERGE, 1)
        rc, ref = _call(lib, False, q, k, v, cache, c)
        _lib.check(rc, "attention")
        out = torch.zeros_like(q)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        print("no-alloc: first call of a fresh library copy under capture", flush=True)
        with torch.cuda.graph(graph, stream=s):
            rc = fresh.dx_blockwise_causal_attention_noalloc(
                q.data_ptr(), *_strides(q), k.data_ptr(), *_strides(k), v.data_ptr(),
                *_strides(v), cache.data_ptr(), cache.stride(0), cache.stride(1),
                cache.stride(2), cache.stride(3), out.data_ptr(), *_strides(out), _lib.DX_BF16,
                b, lq, lq, h, h, d, c, None, _lib.DX_I32, 0, 0, float(d) ** -0.5, s.cuda_stream)
        assert rc == 0, fresh.dx_last_error().decode()
        torch.cuda.synchronize()
        for rep in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {rep} differs from the workspace entry point"
            rc, again = _call(lib, False, q, k, v, cache, c)  # eager work between replays
            _lib.check(rc, "attention")
        fresh.dx_set_tuning(_lib.TUNE_ATTN_KERNEL, 0)
        fresh.dx_set_tuning(_lib.TUNE_ATTN_MERGE, 0)
