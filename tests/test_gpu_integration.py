"""The reference-side binding that INTEGRATION.md gives a dexter maintainer, run
as written, and the package's own workspace cache under graph capture (MI355X).

The binding's code block is read from INTEGRATION.md and executed unchanged,
except for the library path. Its two dexter imports resolve to stand-in
modules: ``register`` returns the function it decorates, and the platform
types are this package's mirror of ``python/dexter/platform.py``. The call
replaces ``ops/gfx1151/attention/blockwise_causal.py:146-173`` and is checked
against the oracle (``ops/reference/attention.py:50-77``).

At C3's shape (913 queries over 7,304 cached + 913 new keys, 40 heads) the
planner picks the paired prefill kernel with its key splits merged in the
launch, which needs the workspace's arrival counters at zero. Before the call
a block of the same size, filled with 0xFF, is allocated and freed on the same
stream, so a binding that took an uninitialised buffer would get those bytes
back from torch's caching allocator, and rows would go unwritten.
"""

from __future__ import annotations

import re
import sys
import types
from pathlib import Path

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd import platform as dx_platform
from dexter_amd.ops.gfx950 import _lib
from oracle import attention as oatt

from _util import assert_parity

pytestmark = pytest.mark.gpu
DT = torch.bfloat16
ROOT = Path(__file__).resolve().parents[1]


def _binding_source() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    src = [b for b in blocks if "def attention(" in b and "lib = ctypes.CDLL" in b]
    assert len(src) == 1, "INTEGRATION.md holds one attention binding"
    return src[0]


def _load_binding():
    """Execute the binding's text; returns its namespace."""
    class Priority:  # the reference's ordering (registry.py); only SPECIALISED is read
        REFERENCE, PORTABLE, PERFORMANT, SPECIALISED = 0, 10, 20, 30

    def register(*_args, **_kwargs):
        return lambda fn: fn

    pkg = types.ModuleType("dexter")
    reg = types.ModuleType("dexter.registry")
    reg.Priority, reg.register = Priority, register
    plat = types.ModuleType("dexter.platform")
    plat.ArchVersion, plat.Capability = dx_platform.ArchVersion, dx_platform.Capability
    saved = {k: sys.modules.get(k) for k in ("dexter", "dexter.registry", "dexter.platform")}
    sys.modules.update({"dexter": pkg, "dexter.registry": reg, "dexter.platform": plat})
    try:
        src = _binding_source().replace("/path/to/libdexter_gfx950.so", str(_lib.LIB_PATH))
        ns: dict = {"__name__": "integration_binding"}
        exec(compile(src, "INTEGRATION.md#binding", "exec"), ns)
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v
    return ns


def _rand(shape, device, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(DT).to(device)


def test_integration_binding_at_c3_shape(device, built_lib):
    ns = _load_binding()
    b, lq, h, d, c = 1, 913, 40, 128, 7304
    q, k, v = (_rand((b, lq, h, d), device, 900 + i) for i in range(3))
    cache = _rand((2, b, c + lq, h, d), device, 903)
    ws_n = ns["lib"].dx_attention_workspace_bytes(b, lq, lq, h, d, c, None)
    assert ws_n > 0, "C3 splits its key range, so it needs a workspace"
    # The planted garbage: same size, same stream, freed before the call.
    junk = torch.full((ws_n,), 0xFF, dtype=torch.uint8, device=device)
    del junk
    got = ns["attention"](q, k, v, cache, c, None, None)
    torch.cuda.synchronize()
    ref = oatt.blockwise_causal_attention(q.cpu(), k.cpu(), v.cpu(), cache.cpu(), c, None, None,
                                          keep_fp32=True)
    assert_parity(got, ref, what="INTEGRATION.md binding at C3")
    # A second call on the same (now reused) workspace, and the package's own op.
    again = ns["attention"](q, k, v, cache, c, None, None)
    torch.cuda.synchronize()
    assert torch.equal(again, got)
    assert torch.equal(ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=c), got)


def _paired_call(device, lq, cache_len, seed):
    """A chunk over a cache on the paired kernel with 3 key splits merged in the
    launch: the plan whose correctness depends on the workspace's counters."""
    h, d = 8, 128
    q, k, v = (_rand((1, lq, h, d), device, seed + i) for i in range(3))
    cache = _rand((2, 1, cache_len + lq, h, d), device, seed + 3)
    out = torch.empty_like(q)

    def run():
        out.copy_(ops.blockwise_causal_attention(q, k, v, kv_cache=cache, cache_len=cache_len))
        return out
    return run, out


def test_outgrown_workspace_stays_valid_for_captured_graphs(device, built_lib):
    """Graph A is captured on stream s with s's workspace; then an eager call on s
    (and a second capture) needs a larger one. The old buffer must stay allocated:
    A replays with its address. Blocks of its size filled with 0xFF are taken
    from s's pool before each replay, which would land on it had it been freed."""
    s = torch.cuda.Stream()
    with _lib.tuning(_lib.TUNE_ATTN_KERNEL, 3), _lib.tuning(_lib.TUNE_ATTN_SPLITS, 3):
        small, small_out = _paired_call(device, 200, 2000, 950)
        big, _ = _paired_call(device, 900, 30000, 960)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            small()
            want = small_out.clone()
            key = (device.index or 0, s.cuda_stream)
            ws_small = _lib._workspaces[key]
            graph_a = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_a, stream=s):
            small()
        with torch.cuda.stream(s):
            big()  # grows s's workspace
            assert _lib._workspaces[key].numel() > ws_small.numel()
            graph_b = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_b, stream=s):
            big()
        torch.cuda.synchronize()
        junk = []
        for rep in range(4):
            with torch.cuda.stream(s):
                junk.append(torch.full((ws_small.numel(),), 0xFF, dtype=torch.uint8,
                                       device=device))
                small_out.zero_()
                graph_a.replay()
                got = small_out.clone()
                graph_b.replay()
                big()
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"replay {rep} of the first graph differs"


def test_integration_binding_in_fp32_and_at_head_dim_256(device, built_lib):
    """The same binding with fp32 inputs (C0, the reference's own fp32 case, and
    a decode chunk over a cache that splits its keys) and with bf16 at head
    dim 256: the general kernel behind the same entry point."""
    ns = _load_binding()
    from dexter_amd.bench.workloads import CONFIGS, make_inputs
    cfg = CONFIGS["C0"]
    inp = make_inputs(cfg)
    bb = torch.tensor(cfg.block_starts)
    got = ns["attention"](inp.q.to(device), inp.k.to(device), inp.v.to(device), None, 0,
                          bb.to(device), None)
    ref = oatt.blockwise_causal_attention(inp.q, inp.k, inp.v, None, 0, bb, None, keep_fp32=True)
    assert got.dtype == torch.float32
    assert_parity(got, ref, 1e-4, 1e-5, what="binding, C0 fp32")
    for dt, d, c in ((torch.float32, 128, 1245), (torch.bfloat16, 256, 700)):
        g = torch.Generator().manual_seed(d)
        q, k, v = (torch.randn((1, 83, 4, d), generator=g).to(dt) for _ in range(3))
        cache = torch.randn((2, 1, c + 83, 4, d), generator=g).to(dt)
        got = ns["attention"](q.to(device), k.to(device), v.to(device), cache.to(device), c,
                              None, None)
        torch.cuda.synchronize()
        ref = oatt.blockwise_causal_attention(q, k, v, cache, c, None, None, keep_fp32=True)
        bar = (1e-4, 1e-5) if dt == torch.float32 else (2e-2, 2e-3)
        assert_parity(got, ref, *bar, what=f"binding, {dt} D={d}")
