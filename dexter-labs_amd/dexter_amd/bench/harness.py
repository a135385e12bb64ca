"""Timing helpers: HIP-graph replay and HIP-event timing on the launch stream.

The reference times small kernels with many back-to-back calls behind one
sync, minimum over trials (``python/dexter/bench/harness.py:35-62``). On
MI355X the same intent -- take the launch path out of a microsecond-scale
measurement -- is met by capturing the calls in a HIP graph and timing graph
replays with HIP events recorded on the stream the kernels run on.
"""

from __future__ import annotations

import statistics
import time
from typing import Callable

import torch


def capture(fn: Callable[[], object], warmup: int = 2) -> torch.cuda.CUDAGraph:
    """Run ``fn`` eagerly ``warmup`` times on a side stream, then capture it once
    on that same stream, so per-stream state the calls set up while warming up
    (the attention workspace) is what the graph records, not a new allocation
    and its zero fill inside the graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        fn()
    torch.cuda.synchronize()
    return graph


def event_time_ms(run: Callable[[], object], reps: int, trials: int = 5) -> float:
    """Minimum over trials of (event-timed ``reps`` calls of ``run``) / reps, in ms.

    Events are recorded on torch's current stream, which is where ``run``
    launches (graph replays and the ops both use it).
    """
    stream = torch.cuda.current_stream()
    best = float("inf")
    for _ in range(trials):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            run()
        end.record(stream)
        end.synchronize()
        best = min(best, start.elapsed_time(end) / reps)
    return best


def wall_time_ms(run: Callable[[], object], reps: int) -> float:
    """Host wall time per call of ``reps`` back-to-back calls behind one sync."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / reps


def cpu_median_ms(run: Callable[[], object], budget_s: float, warmup: int = 2,
                  min_runs: int = 5) -> tuple[float, int]:
    """Median wall time of ``run`` on the CPU: ``warmup`` runs, then at least
    ``min_runs`` runs and as many more as fit in ``budget_s`` seconds."""
    for _ in range(warmup):
        run()
    samples: list[float] = []
    t_end = time.perf_counter() + budget_s
    while len(samples) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        run()
        samples.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(samples), len(samples)
