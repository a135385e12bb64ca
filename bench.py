#!/usr/bin/env python3
"""Benchmark of the blockwise-causal attention path on one MI355X.

Headline (BASELINE.json ``metric``): block-causal attention TFLOP/s and its
fraction of the dense bf16 MFMA peak at the Wan-5B shape, and ms per 83-token
chunk. A *step* is one 83-token chunk through the path for all 30 layers of
Wan2.2-TI2V-5B (config C1): per layer, QK-RMSNorm+RoPE of the chunk's q/k and
blockwise-causal attention over that layer's 1,245 cached keys plus the 83
new ones. The 30 per-layer caches (16.3 MB each, 489 MB in all) exceed the
256 MB MALL, so the cache really streams from HBM. Inputs are synthetic,
seeded (C1 recipe), resident in HBM before timing. Steps are replayed from a
HIP graph; K steps are timed with synchronisation on both sides.

``value`` = 30 x 1.354 GFLOP (visible pairs only) / step time. Alongside:
``roofline`` for the attention kernel at C1 (HBM-bound: algorithmic bytes
per launch / event-timed launch duration), ``cpu_baseline`` (the torch fp32
oracle timed on this host), and ``extra`` with the prologue, the fused
prologue+append, and attention at C2 (8K prefill, MFMA-bound), C3 and C4.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "dexter-labs_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
PEAK_HBM_GBPS = 8000.0
LAYERS_5B = 30
DEFAULT_METRIC = "block-causal attn TFLOP/s + % bf16 MFMA peak @Wan-5B; ms per 83-token chunk"


def _metric_name() -> str:
    try:
        return json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    except Exception:
        return DEFAULT_METRIC


def _profile_traffic() -> dict | None:
    """HBM bytes per attention launch at C1 from the committed rocprof counter summary."""
    path = ROOT / "profiles" / "attn_fwd_C1_hbm_traffic.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text())
    return {"bytes": float(m.group(1)), "source": str(path.relative_to(ROOT))} if m else None


def _profiled_call_us() -> dict | None:
    """Per-call time of the C1 attention kernels under rocprof (committed kernel summary)."""
    path = ROOT / "profiles" / "attn_fwd_C1_kernel_stats.md"
    if not path.exists():
        return None
    text = path.read_text()
    m = re.search(r"profiled_us_per_call:\s*([0-9.eE+]+)", text)
    if not m:
        return None
    out = {"us": float(m.group(1)), "source": str(path.relative_to(ROOT))}
    # HIP-event time of the same call in the same profiled run: the two agree when
    # the event method counts what the kernel trace counts.
    e = re.search(r"event_us_same_run:\s*([0-9.eE+]+)", text)
    if e:
        out["event_us_same_run"] = float(e.group(1))
        out["method_gap"] = out["event_us_same_run"] / out["us"] - 1.0
    # The same command without the profiler, as committed: the figure this line's
    # live launch_us is checked against.
    u = re.search(r"unprofiled_us_per_call:\s*([0-9.eE+]+)", text)
    if u:
        out["unprofiled_us_committed"] = float(u.group(1))
    return out


def _per_layer_inputs(inp, device, layers: int, cache_len: int):
    """Per-layer chunk activations and per-layer caches holding the rotated history."""
    import torch

    import dexter_amd.ops as ops


    cfg = inp.cfg
    c = cache_len
    q, k, v = inp.q.to(device), inp.k.to(device), inp.v.to(device)
    qw, kw = inp.q_weight.to(device), inp.k_weight.to(device)
    cos, sin = inp.cos.to(device), inp.sin.to(device)
    _, kr = ops.qk_norm_rope(q[:, :c], k[:, :c], qw, kw, cos[:c], sin[:c])
    caches = []
    for _ in range(layers):  # the model's per-layer caches
        cache = torch.zeros(2, cfg.batch, c + cfg.q_len, cfg.heads, cfg.head_dim,
                            device=device, dtype=cfg.dtype)
        ops.kv_cache_append(cache, kr, v[:, :c], 0)
        caches.append(cache)
    chunk = [tuple(t[:, c:].clone() for t in (q, k, v)) for _ in range(layers)]
    tables = (cos[c:].contiguous(), sin[c:].contiguous())
    torch.cuda.synchronize()
    return caches, chunk, (qw, kw), tables


def run_headline(args, device):
    import time

    import torch

    import dexter_amd.ops as ops
    from dexter_amd.bench import harness
    from dexter_amd.bench.workloads import CONFIGS, make_inputs

    cfg = CONFIGS["C1"]
    L = args.layers
    c = cfg.cache_lens[0]
    inp = make_inputs(cfg)
    caches, chunk, (qw, kw), (cos, sin) = _per_layer_inputs(inp, device, L, c)

    def step():
        for layer in range(L):
            qi, ki, vi = chunk[layer]
            qc, kc = ops.qk_norm_rope(qi, ki, qw, kw, cos, sin)
            ops.blockwise_causal_attention(qc, kc, vi, kv_cache=caches[layer], cache_len=c)

    # Eager (Python dispatch per op) for reference, then the graph that is timed.
    for _ in range(max(1, args.warmup)):
        step()
    eager_ms = harness.wall_time_ms(step, reps=max(3, args.steps // 5))
    graph = harness.capture(step)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # Attention alone, per launch (event-timed graph of L launches).
    rot = []
    for layer in range(L):
        qi, ki, vi = chunk[layer]
        rot.append(ops.qk_norm_rope(qi, ki, qw, kw, cos, sin) + (vi,))
    attn_graph = harness.capture(lambda: [
        ops.blockwise_causal_attention(rot[i][0], rot[i][1], rot[i][2], kv_cache=caches[i],
                                       cache_len=c) for i in range(L)])
    attn_ms = harness.event_time_ms(attn_graph.replay, reps=max(5, args.steps // 2)) / L
    pro_graph = harness.capture(lambda: [ops.qk_norm_rope(chunk[i][0], chunk[i][1], qw, kw, cos,
                                                          sin) for i in range(L)])
    pro_ms = harness.event_time_ms(pro_graph.replay, reps=max(5, args.steps // 2)) / L

    # The same step with the cache length read from device memory (a graph
    # captured once and replayed as the cache grows), per step.
    cursor = torch.tensor([c], dtype=torch.int32, device=device)

    def step_dev():
        for layer in range(L):
            qi, ki, vi = chunk[layer]
            qc, kc = ops.qk_norm_rope(qi, ki, qw, kw, cos, sin)
            ops.blockwise_causal_attention(qc, kc, vi, kv_cache=caches[layer], cache_len=cursor)

    dev_graph = harness.capture(step_dev)
    for _ in range(args.warmup):
        dev_graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dev_graph.replay()
    torch.cuda.synchronize()
    dev_ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    del dev_graph

    # Fused prologue + append (the priming pass's form), per launch.
    def prime():
        for i in range(L):
            ops.qk_norm_rope_append(chunk[i][0], chunk[i][1], chunk[i][2], qw, kw, cos, sin,
                                    caches[i], c)
    prime_graph = harness.capture(prime)
    prime_ms = harness.event_time_ms(prime_graph.replay, reps=max(5, args.steps // 2)) / L

    flops = cfg.flops()
    attn_bytes = cfg.bytes()
    tok = cfg.q_len * cfg.heads * cfg.head_dim * 2
    pro_bytes = 4 * tok + 2 * cfg.heads * cfg.head_dim * 2 + 2 * cfg.q_len * cfg.head_dim // 2 * 4
    value = L * flops / (ms_per_step * 1e-3) / 1e12
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    traffic = _profile_traffic()
    profiled = _profiled_call_us()
    if profiled:
        # The same call's kernels timed by rocprof (begin to end of each dispatch,
        # lengthened by the profiler's instrumentation): the frac the committed
        # profile gives, beside the live HIP-event one.
        profiled["frac"] = attn_bytes / (profiled["us"] * 1e-6) / 1e9 / PEAK_HBM_GBPS
        if "unprofiled_us_committed" in profiled:
            profiled["live_vs_committed"] = attn_ms * 1e3 / profiled["unprofiled_us_committed"] - 1.0
    return {
        "ms_per_step": ms_per_step,
        "value": value,
        "eager_ms_per_step": eager_ms,
        "device_cursor_ms_per_step": dev_ms_per_step,
        "attn_ms": attn_ms,
        "roofline": {
            "bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBPS,
            "traffic": traffic["bytes"] if traffic else None,
            "kernel": ("one attention call at C1 = attn_fwd_kernel<128,bf16_t,2> (split-KV, "
                       "dual-stream, partials stored blocked) + "
                       "attn_combine_kernel<128,bf16_t,8,true>"),
            "profiled": profiled,
            "algorithmic_bytes_per_launch": attn_bytes,
            "launch_us": attn_ms * 1e3,
            "tflops": flops / (attn_ms * 1e-3) / 1e12,
        },
        "prologue": {"us": pro_ms * 1e3, "gbps": pro_bytes / (pro_ms * 1e-3) / 1e9,
                     "bytes": pro_bytes},
        "prologue_append_fused": {"us": prime_ms * 1e3,
                                  "gbps": (pro_bytes + 2 * tok) / (prime_ms * 1e-3) / 1e9,
                                  "bytes": pro_bytes + 2 * tok},
        "inputs": inp,
    }


def _config_graph(name: str, device):
    """A captured graph of n attention calls at one config on n distinct copies of the
    inputs (n chosen so that they exceed the 256 MB MALL, as a model's per-layer caches
    do). Returns (config, graph, n)."""
    import math

    import torch

    import dexter_amd.ops as ops
    from dexter_amd.bench import harness
    from dexter_amd.bench.workloads import CONFIGS, block_tensor, make_inputs

    cfg = CONFIGS[name]
    inp = make_inputs(cfg)
    bb = block_tensor(cfg, device)
    if name == "C4":
        lens = list(cfg.cache_lens)
        b, h, d = cfg.batch, cfg.heads, cfg.head_dim
        cache = torch.zeros(2, b, max(lens), h, d, device=device, dtype=cfg.dtype)
        kq = torch.zeros(b, cfg.q_len, h, d, dtype=cfg.dtype)
        vq = torch.zeros_like(kq)
        for i, c in enumerate(lens):
            cache[0, i, :c] = inp.k[i, :c].to(device)
            cache[1, i, :c] = inp.v[i, :c].to(device)
            kq[i], vq[i] = inp.k[i, c:c + cfg.q_len], inp.v[i, c:c + cfg.q_len]
        q, kq, vq = (t.to(device) for t in (inp.q, kq, vq))
        args = (q, kq, vq, cache)

        def one(q, kq, vq, cache):
            ops.blockwise_causal_attention_varlen(q, kq, vq, kv_cache=cache, cache_lens=lens,
                                                  block_boundaries=bb)
    else:
        c = cfg.cache_lens[0]
        q, k, v = inp.q.to(device), inp.k.to(device), inp.v.to(device)
        qw, kw = inp.q_weight.to(device), inp.k_weight.to(device)
        cos, sin = inp.cos.to(device), inp.sin.to(device)
        qr, kr = ops.qk_norm_rope(q, k, qw, kw, cos, sin)
        cache = None
        if c:
            cache = torch.zeros(2, cfg.batch, c + cfg.q_len, cfg.heads, cfg.head_dim,
                                device=device, dtype=cfg.dtype)
            ops.kv_cache_append(cache, kr[:, :c], v[:, :c], 0)
        qc, kc, vc = qr[:, c:].contiguous(), kr[:, c:].contiguous(), v[:, c:].contiguous()
        del q, k, qr, kr
        args = (qc, kc, vc, cache)

        def one(qc, kc, vc, cache):
            ops.blockwise_causal_attention(qc, kc, vc, kv_cache=cache, cache_len=c,
                                           block_boundaries=bb)
    footprint = sum(t.numel() * t.element_size() for t in args if t is not None)
    n = max(2, min(16, math.ceil(300e6 / footprint)))
    copies = [args] + [tuple(None if t is None else t.clone() for t in args)
                       for _ in range(n - 1)]
    graph = harness.capture(lambda: [one(*a) for a in copies])
    return cfg, graph, n


def run_config(name: str, device, reps: int) -> dict:
    """Attention alone at one config, per call: event-timed replays of a graph of n calls
    on n distinct copies of the inputs (the replay overhead is shared by the n calls)."""
    from dexter_amd.bench import harness

    cfg, graph, n = _config_graph(name, device)
    ms = harness.event_time_ms(graph.replay, reps=reps) / n
    del graph
    return {
        "us": ms * 1e3,
        "tflops": cfg.flops() / (ms * 1e-3) / 1e12,
        "pct_mfma_peak": 100 * cfg.flops() / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "gbps": cfg.bytes() / (ms * 1e-3) / 1e9,
        "pct_hbm_peak": 100 * cfg.bytes() / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
        "gflop": cfg.flops() / 1e9,
        "bytes": cfg.bytes(),
        "calls_per_graph": n,
    }


def run_timeline(name: str, device, reps: int) -> dict:
    """Phase timeline of the decode kernel's last call in one replay of the config's graph
    (`_config_graph`), from the timeline build's per-workgroup s_memrealtime stamps (100 MHz;
    the words are listed at g_timeline in csrc/attn_fwd.hip). Medians per (sequence, split
    count) over the workgroups, in us from the call's first workgroup start; the merge
    kernel's blocks (if any) as one span. Stamps mark instructions issued: a store's
    completion is not in them."""
    import ctypes
    import statistics

    import torch

    from dexter_amd.bench import harness
    from dexter_amd.ops.gfx950 import _lib

    lib = _lib.load()
    if not hasattr(lib, "dx_timeline_read"):
        raise RuntimeError(f"{_lib.LIB_PATH.name} has no stamps: build it with "
                           "`python dexter-labs_amd/csrc/build.py --timeline`")
    lib.dx_timeline_words.restype = ctypes.c_int64
    cfg, graph, n = _config_graph(name, device)
    per_call_us = harness.event_time_ms(graph.replay, reps=reps) / n * 1e3
    words = lib.dx_timeline_words()
    buf = (ctypes.c_uint64 * words)()
    if lib.dx_timeline_clear() != 0:
        raise RuntimeError("dx_timeline_clear failed")
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    if lib.dx_timeline_read(buf) != 0:
        raise RuntimeError("dx_timeline_read failed")
    slots, groups = 32, 2048  # kTimelineSlots, kTimelineGroups (csrc/attn_fwd.hip)
    if words != slots * groups + 2 * 8 * groups:
        raise RuntimeError(f"timeline library layout changed: {words} words")
    rows = [buf[w * slots:(w + 1) * slots] for w in range(groups)]
    rows = [r for r in rows if r[0]]
    merge = [(buf[slots * groups + 2 * i], buf[slots * groups + 2 * i + 1])
             for i in range(8 * groups)]
    merge = [m for m in merge if m[0]]
    t0 = min(r[0] for r in rows)
    us = lambda t: round((t - t0) / 100, 2)
    med = lambda v: round(statistics.median(v), 2) if v else None
    segs = {}
    for r in rows:
        segs.setdefault((r[8] >> 16 & 0xffff, r[8] >> 8 & 0xff), []).append(r)
    out = {"config": name, "per_call_us": round(per_call_us, 2), "calls_per_graph": n,
           "workgroups": len(rows), "span_us": us(max(r[7] for r in rows if r[7])),
           "segments": []}
    names = {1: "q_ready", 2: "loop_done", 3: "handover_done", 4: "stores_issued",
             5: "arrived", 7: "end"}
    for (b, ns), rs in sorted(segs.items()):
        seg = {"batch": b, "splits": ns, "workgroups": len(rs),
               "tiles": max(r[9] & 0xffff for r in rs), "rounds": max(r[9] >> 16 for r in rs),
               "start": med([us(r[0]) for r in rs]), "start_max": max(us(r[0]) for r in rs)}
        for k, label in names.items():
            seg[label] = med([us(r[k]) for r in rs if r[k]])
        seg["end_max"] = max((us(r[7]) for r in rs if r[7]), default=None)
        seg["round_tiles_in_lds"] = [med([us(r[16 + i]) for r in rs if r[16 + i]])
                                     for i in range(min(seg["rounds"], 16))]
        mergers = [r for r in rs if r[8] >> 32]
        if mergers:
            seg["mergers"] = {"n": len(mergers),
                              "arrived": med([us(r[5]) for r in mergers]),
                              "merge_loads_done": med([us(r[6]) for r in mergers]),
                              "end": med([us(r[7]) for r in mergers]),
                              "end_max": max(us(r[7]) for r in mergers)}
        out["segments"].append(seg)
    if merge:
        ends = [m[1] for m in merge if m[1]]
        out["merge_kernel"] = {"blocks": len(merge), "first_start": us(min(m[0] for m in merge)),
                               "median_start": med([us(m[0]) for m in merge]),
                               "last_end": us(max(ends)) if ends else None}
    del graph
    return out


def run_gemm_ceiling(device, reps: int = 10) -> dict:
    """The same box's bf16 GEMM rate through torch.matmul (hipBLASLt), 8192^3, timed
    like the attention configs: the practical MFMA ceiling of this GPU under its power
    cap, beside which the prefill configs' fraction of nominal peak is read."""
    import torch

    from dexter_amd.bench import harness

    n = 8192
    g = torch.Generator().manual_seed(0)
    a = torch.randn(n, n, generator=g).to(torch.bfloat16).to(device)
    b = torch.randn(n, n, generator=g).to(torch.bfloat16).to(device)
    for _ in range(3):
        torch.matmul(a, b)
    ms = harness.event_time_ms(lambda: torch.matmul(a, b), reps=reps)
    tflops = 2 * n ** 3 / (ms * 1e-3) / 1e12
    return {"shape": [n, n, n], "us": ms * 1e3, "tflops": tflops,
            "pct_mfma_peak": 100 * tflops / PEAK_BF16_TFLOPS, "library": "torch.matmul (hipBLASLt)"}


def run_norm(device, layers: int, reps: int) -> dict:
    """adaLN modulation and gated residual (the ops either side of attention in a Wan
    block) at the C1 activation (83 x 3072) and the C2 prefill activation
    (8,192 x 3072), bf16, [1, 1, C] modulation rows as the model passes them.
    Each figure is one launch, event-timed inside a graph of distinct inputs, next to
    the reference's unfused torch expression (``ops/reference/norm.py:20,25``) timed
    the same way, and to torch's own copy and add of the same activation (the
    streaming rate this GPU reaches at that size with the same read/write mix)."""
    import torch
    import torch.nn.functional as F

    import dexter_amd.ops as ops
    from dexter_amd.bench import harness

    out = {}
    g = torch.Generator(device=device).manual_seed(0)
    for name, rows, n in (("C1", 83, layers), ("C2", 8192, 4)):
        cols = 3072
        xs = [torch.randn(1, rows, cols, device=device, generator=g).to(torch.bfloat16)
              for _ in range(n)]
        ys = [torch.randn_like(x) for x in xs]
        mod = torch.randn(n, 6, 1, cols, device=device, generator=g).to(torch.bfloat16)
        parts = [m.unsqueeze(0).unbind(1) for m in mod]  # [1, 1, C] views, as the model's
        act = rows * cols * 2
        row = cols * 2
        cases = {
            "adaln": (lambda i: ops.adaln_modulate(xs[i], parts[i][1], parts[i][0], 1e-6),
                      lambda i: F.layer_norm(xs[i], (cols,), eps=1e-6) * (1 + parts[i][1])
                      + parts[i][0],
                      2 * act + 2 * row),
            "gated_residual": (lambda i: ops.gated_residual(xs[i], ys[i], parts[i][2]),
                               lambda i: xs[i] + ys[i] * parts[i][2],
                               3 * act + row),
        }
        for op, (fused, ref, nbytes) in cases.items():
            fg = harness.capture(lambda f=fused: [f(i) for i in range(n)])
            ms = harness.event_time_ms(fg.replay, reps=reps) / n
            rg = harness.capture(lambda f=ref: [f(i) for i in range(n)])
            rms = harness.event_time_ms(rg.replay, reps=reps) / n
            gbps = nbytes / (ms * 1e-3) / 1e9
            out[f"{op}_{name}"] = {
                "us": ms * 1e3, "gbps": gbps, "pct_hbm_peak": 100 * gbps / PEAK_HBM_GBPS,
                "bytes": nbytes, "torch_unfused_us": rms * 1e3, "speedup_vs_torch": rms / ms,
                "shape": [1, rows, cols]}
            del fg, rg
        # Streaming references at the same size: torch's copy (1 read + 1 write, what
        # adaLN moves) and add (2 reads + 1 write, what the gated residual moves).
        zs = [torch.empty_like(x) for x in xs]
        cg = harness.capture(lambda: [zs[i].copy_(xs[i]) for i in range(n)])
        cms = harness.event_time_ms(cg.replay, reps=reps) / n
        ag = harness.capture(lambda: [torch.add(xs[i], ys[i], out=zs[i]) for i in range(n)])
        ams = harness.event_time_ms(ag.replay, reps=reps) / n
        out[f"stream_ref_{name}"] = {
            "copy_us": cms * 1e3, "copy_gbps": 2 * act / (cms * 1e-3) / 1e9,
            "add_us": ams * 1e3, "add_gbps": 3 * act / (ams * 1e-3) / 1e9}
        del xs, ys, zs, mod, parts, cg, ag
    return out


def run_cross(device, layers: int, reps: int) -> dict:
    """Cross-attention of the C1 chunk (83 queries, 24 heads x 128, bf16) onto the Wan-5B
    i2v conditioning: 512 text keys and 257 CLIP image keys, each layer with its own
    context K/V (``models/dreamzero/model.py:234-241``). One call per stream per layer,
    event-timed inside a graph over the 30 layers."""
    import torch

    import dexter_amd.ops as ops
    from dexter_amd.bench import harness

    h, d, lq = 24, 128, 83
    g = torch.Generator(device=device).manual_seed(0)
    rnd = lambda *s: torch.randn(*s, device=device, generator=g).to(torch.bfloat16)  # noqa: E731
    out = {}
    q = [rnd(1, lq, h, d) for _ in range(layers)]
    for name, ctx in (("text", 512), ("image", 257)):
        k = [rnd(1, ctx, h, d) for _ in range(layers)]
        v = [rnd(1, ctx, h, d) for _ in range(layers)]
        graph = harness.capture(lambda: [ops.blockwise_causal_attention(q[i], k[i], v[i])
                                         for i in range(layers)])
        ms = harness.event_time_ms(graph.replay, reps=reps) / layers
        flops = 4 * d * lq * ctx * h
        nbytes = (2 * lq + 2 * ctx) * h * d * 2
        out[f"cross_{name}_C1"] = {
            "us": ms * 1e3, "keys": ctx, "tflops": flops / (ms * 1e-3) / 1e12,
            "gbps": nbytes / (ms * 1e-3) / 1e9,
            "pct_hbm_peak": 100 * nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, "bytes": nbytes}
        del graph, k, v
    return out


def run_qkv(device, layers: int, reps: int) -> dict:
    """The C1 chunk's q/k/v projections (83 tokens x 3072 -> 3 x 3072, bf16, with bias)
    fused with the QK-norm + rotary prologue (``ops.qkv_norm_rope``), each of 30 layers
    with its own weights, against three ``F.linear`` (hipBLASLt) plus the HIP prologue:
    the path it replaces (``models/dreamzero/model.py:162-175``)."""
    import torch
    import torch.nn.functional as F

    import dexter_amd.ops as ops
    from dexter_amd.bench import harness
    from dexter_amd.bench.workloads import rope_table

    c, heads, dim, tokens = 3072, 24, 128, 83
    g = torch.Generator(device=device).manual_seed(0)
    rnd = lambda *s: torch.randn(*s, device=device, generator=g).to(torch.bfloat16)  # noqa: E731
    x = [rnd(1, tokens, c) for _ in range(layers)]
    w = [[rnd(c, c).mul_(c ** -0.5) for _ in range(3)] for _ in range(layers)]
    b = [[rnd(c).mul_(0.1) for _ in range(3)] for _ in range(layers)]
    nq, nk = rnd(c).add_(1.0), rnd(c).add_(1.0)
    cos, sin = (t.to(device) for t in rope_table(torch.arange(tokens) + 1245, dim))

    def fused():
        for i in range(layers):
            ops.qkv_norm_rope(x[i], w[i][0], b[i][0], w[i][1], b[i][1], w[i][2], b[i][2],
                              nq, nk, cos, sin, heads)

    def unfused():
        for i in range(layers):
            q, k, _ = (F.linear(x[i], w[i][j], b[i][j]).view(1, tokens, heads, dim)
                       for j in range(3))
            ops.qk_norm_rope(q, k, nq, nk, cos, sin)

    out = {}
    for name, fn in (("fused", fused), ("linear_x3_plus_prologue", unfused)):
        graph = harness.capture(fn)
        out[f"{name}_us"] = harness.event_time_ms(graph.replay, reps=reps) / layers * 1e3
        del graph
    wbytes = 3 * c * c * 2
    out["weight_bytes"] = wbytes
    out["fused_weight_gbps"] = wbytes / (out["fused_us"] * 1e-6) / 1e9
    out["fused_pct_hbm_peak"] = 100 * out["fused_weight_gbps"] / PEAK_HBM_GBPS
    out["speedup"] = out["linear_x3_plus_prologue_us"] / out["fused_us"]
    return out


def run_cpu_baseline(inp, budget_s: float) -> dict:
    """The torch fp32 oracle on this host's cores, C1 attention per layer (a bounded sample)."""
    import platform as pyplatform

    import torch

    from dexter_amd.bench import harness
    from oracle import attention as oatt
    from oracle import rope as orope

    # All of the host's cores, as the baseline plan says; the affinity set
    # (the CPUs this process may actually run on) is reported beside it.
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    cfg = inp.cfg
    c = cfg.cache_lens[0]
    rq, rk = orope.qk_norm_rope(inp.q, inp.k, inp.q_weight, inp.k_weight, inp.cos, inp.sin, 1e-6)
    cache = torch.stack((rk[:, :c], inp.v[:, :c]))
    qc, kc, vc = rq[:, c:], rk[:, c:], inp.v[:, c:]

    def call():
        oatt.blockwise_causal_attention(qc, kc, vc, cache, c, None, None)

    ms, runs = harness.cpu_median_ms(call, budget_s)
    return {
        "value": cfg.flops() / (ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"C1 attention (one layer: 83 q x 1,328 keys x 24 heads), torch fp32 oracle "
                   f"(oracle/attention.py), median of {runs} calls in ~{budget_s:.0f} s; "
                   f"ms per 30-layer chunk = {LAYERS_5B * ms:.2f}"),
        "ms_per_call": ms,
        "cpu": _cpu_model() or pyplatform.processor() or pyplatform.machine(),
        "os_cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
    }


def _cpu_model() -> str | None:
    """The host CPU's model name (/proc/cpuinfo), or None where unavailable."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=LAYERS_5B)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU work for the cpu_baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip C2/C3/C4")
    ap.add_argument("--only", choices=["C1", "C2", "C3", "C4", "norm", "cross", "qkv", "gemm"],
                    default=None,
                    help="time one config's attention only (for profiling runs)")
    ap.add_argument("--timeline", choices=["C1", "C4"], default=None,
                    help="phase timeline of one config's decode call (needs the library that "
                         "`csrc/build.py --timeline` builds)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="first run a plain device copy of this size (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); attention heads shard across GPUs with no collective, "
              "so the one-GPU number is the per-GPU figure.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    device = torch.device("cuda", 0)
    import dexter_amd.ops  # noqa: F401
    from dexter_amd.ops.gfx950 import _lib

    if args.timeline:
        _lib.LIB_PATH = _lib.LIB_PATH.with_name("libdexter_gfx950_timeline.so")
    _lib.load()  # fail loudly if the HIP library is missing

    if args.copy_mb:
        n = args.copy_mb * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy calibration: {n} bytes read, {n} bytes written", file=sys.stderr, flush=True)
        del src, dst

    if args.timeline:
        print(json.dumps({"timeline": args.timeline,
                          **run_timeline(args.timeline, device, reps=max(10, args.steps))}),
              flush=True)
        return 0
    if args.only == "gemm":
        print(json.dumps({"only": "gemm", **run_gemm_ceiling(device, reps=max(10, args.steps))}),
              flush=True)
        return 0
    if args.only in ("norm", "cross", "qkv"):
        run = {"norm": run_norm, "cross": run_cross, "qkv": run_qkv}[args.only]
        res = run(device, args.layers, reps=max(10, args.steps))
        print(json.dumps({"only": args.only, **res}), flush=True)
        return 0
    if args.only:
        res = run_config(args.only, device, reps=max(10, args.steps))
        print(json.dumps({"only": args.only, **res}), flush=True)
        return 0

    head = run_headline(args, device)
    print(f"headline done: {head['ms_per_step']:.4f} ms/step", file=sys.stderr, flush=True)
    extra = {"eager_ms_per_step": head["eager_ms_per_step"],
             "device_cursor_ms_per_step": head["device_cursor_ms_per_step"],
             "prologue_C1": head["prologue"],
             "prologue_append_fused_C1": head["prologue_append_fused"]}
    if not args.no_extra:
        extra["gemm_ceiling"] = run_gemm_ceiling(device)
        print(f"gemm ceiling: {extra['gemm_ceiling']['tflops']:.0f} TFLOP/s", file=sys.stderr,
              flush=True)
        for name, reps in (("C2", 20), ("C3", 20), ("C4", 50)):
            extra[name] = run_config(name, device, reps)
            extra[name]["pct_of_gemm_ceiling"] = (100 * extra[name]["tflops"]
                                                  / extra["gemm_ceiling"]["tflops"])
            print(f"{name} done: {extra[name]['us']:.1f} us", file=sys.stderr, flush=True)
        extra["norm"] = run_norm(device, args.layers, reps=20)
        print("norm done: " + ", ".join(f"{k} {v['us']:.2f} us" for k, v in extra["norm"].items()
                                        if "us" in v), file=sys.stderr, flush=True)
        extra["qkv"] = run_qkv(device, args.layers, reps=20)
        print(f"qkv done: fused {extra['qkv']['fused_us']:.2f} us", file=sys.stderr, flush=True)
        extra["cross"] = run_cross(device, args.layers, reps=20)
        print("cross done: " + ", ".join(f"{k} {v['us']:.2f} us" for k, v in extra["cross"].items()),
              file=sys.stderr, flush=True)
    cpu = None if args.no_cpu else run_cpu_baseline(head["inputs"], args.cpu_budget)

    line = {
        "metric": _metric_name(),
        "value": head["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded C1 recipe; random q/k/v, norm weights 1+0.1N(0,1), theta=1e4 RoPE)",
        "config": {"workload": "C1 Wan-5B closed-loop chunk: 83 queries over 1,245 cached + 83 "
                               "new keys, 24 heads x 128, x 30 layers (prologue + attention)",
                   "layers": args.layers, "q_len": 83, "cache_len": 1245, "heads": 24,
                   "head_dim": 128, "batch": 1},
        "pct_mfma_peak": 100 * head["value"] / PEAK_BF16_TFLOPS,
        "ms_per_83_token_chunk": head["ms_per_step"],
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
