"""HIP-graph capture of a control step, including the steps that write the KV cache.

Mirrors ``python/dexter/runtime/graph.py``: ``GraphRunner`` replays a captured
forward against fixed input buffers (:28-47), and ``capture`` warms up on a
side stream before recording, so allocator and library set-up stay out of the
graph (:50-74).

The reference captures only the cache-free denoising steps: the final step of
a control step writes the KV cache at a length that grows between control
steps, and a graph records that length as a constant (:57-60). With a
``KVCache(device_cursor=True)`` the cursor lives in device memory and the
kernels read it when they run (``dx_*_dev`` entry points), so
``CachedStepGraph`` captures the cache-writing step once and replays it for
every control step of an episode:

* before each replay it checks on the host that the block fits, with the
  reference's ``RuntimeError("KV cache full: ...")``;
* the captured step appends at the device cursor and commits, which advances
  the cursor on the device; after the replay the host mirror advances too.

On MI355X a Wan-5B control step is 30 layers x (prologue, attention, and the
block's other launches); replaying it from one graph removes the per-launch
host cost that otherwise exceeds the ~15 us kernels.
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch

from ..models.kv_cache import KVCache


class GraphRunner:
    """A captured forward, replayed against fixed input buffers.

    Callers pass ordinary tensors; they are copied into the buffers the graph
    was captured with, so the static-address requirement stays hidden.
    """

    def __init__(self, graph: torch.cuda.CUDAGraph, inputs: tuple[torch.Tensor, ...],
                 outputs: tuple[torch.Tensor, ...]) -> None:
        self.graph = graph
        self.inputs = inputs
        self.outputs = outputs

    def __call__(self, *args: torch.Tensor) -> tuple[torch.Tensor, ...]:
        if len(args) != len(self.inputs):
            raise ValueError(f"graph takes {len(self.inputs)} inputs, got {len(args)}")
        for buffer, arg in zip(self.inputs, args):
            buffer.copy_(arg)
        self.graph.replay()
        return self.outputs


def _as_tuple(out) -> tuple[torch.Tensor, ...]:
    return tuple(out) if isinstance(out, (tuple, list)) else (out,)


def capture(fn: Callable[..., object], sample_inputs: Sequence[torch.Tensor],
            warmup: int = 3) -> GraphRunner:
    """Capture ``fn(*inputs)`` into a graph, after ``warmup`` eager runs on a side stream.

    ``fn`` must be shape-stable and must not synchronise with the host.
    """
    static = tuple(t.clone() for t in sample_inputs)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn(*static)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = _as_tuple(fn(*static))
    return GraphRunner(graph, static, outputs)


class CachedStepGraph:
    """A captured step that appends ``rows`` rows to device-cursor KV caches and commits them.

    ``fn(*inputs)`` runs one step: its layers append at each cache's cursor
    (``KVCache.append`` / ``append_fused``) and read ``cache_len`` from it, and it
    calls ``commit(rows)`` on every cache in ``caches`` once, at its end. The
    eager warm-up and the capture leave the caches' cursors, host lengths and
    statuses as they found them; rows the warm-up wrote past the cursor are
    rewritten by the first replay.
    """

    def __init__(self, fn: Callable[..., object], sample_inputs: Sequence[torch.Tensor],
                 caches: Sequence[KVCache], rows: int, warmup: int = 2) -> None:
        if not caches or any(c.cursor is None for c in caches):
            raise ValueError("CachedStepGraph needs KVCache(device_cursor=True) caches")
        self.caches = list(caches)
        self.rows = int(rows)
        for c in self.caches:
            c._check_room(self.rows)
        saved = [(c.length, c.cursor.clone(), c.status.clone()) for c in self.caches]

        def restore():
            for c, (length, cursor, status) in zip(self.caches, saved):
                c.length = length
                c.cursor.copy_(cursor)
                c.status.copy_(status)

        static = tuple(t.clone() for t in sample_inputs)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                fn(*static)
                restore()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outputs = _as_tuple(fn(*static))
        # Capture ran fn's host code once (its commits moved the host lengths)
        # but no kernel: restore the host side only.
        for c, (length, _, _) in zip(self.caches, saved):
            c.length = length
        self.runner = GraphRunner(graph, static, outputs)

    def __call__(self, *args: torch.Tensor) -> tuple[torch.Tensor, ...]:
        for c in self.caches:
            c._check_room(self.rows)
        out = self.runner(*args)
        for c in self.caches:
            c.length += self.rows
        return out
