"""HIP-graph capture of a control step, including the steps that write the KV cache.

Covers what ``python/dexter/runtime/graph.py`` offers: a runner that replays a
recorded forward against fixed input buffers (``GraphRunner``, the interface of
:28-47), and ``capture``, which warms the step up on a side stream before
recording so allocator and library set-up stay out of the graph (:50-74).

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
    """A recorded step plus the tensors it reads and writes.

    A graph reads its inputs from the addresses it was recorded with, so each
    call copies the caller's tensors into those buffers (skipping a tensor that
    already is the buffer), replays, and returns the graph's own output
    tensors, which the next call overwrites. Shapes and dtypes must match the
    recording exactly: ``copy_`` would otherwise broadcast or cast without a
    word.
    """

    __slots__ = ("graph", "inputs", "outputs")

    def __init__(self, graph: torch.cuda.CUDAGraph, inputs: tuple[torch.Tensor, ...],
                 outputs: tuple[torch.Tensor, ...]) -> None:
        self.graph, self.inputs, self.outputs = graph, tuple(inputs), tuple(outputs)

    def _stage(self, args: Sequence[torch.Tensor]) -> None:
        if len(args) != len(self.inputs):
            raise ValueError(f"the recorded step reads {len(self.inputs)} input tensors; "
                             f"{len(args)} were passed")
        for i, (buf, arg) in enumerate(zip(self.inputs, args)):
            if arg.shape != buf.shape or arg.dtype != buf.dtype:
                raise ValueError(f"input {i} was recorded as {tuple(buf.shape)} {buf.dtype}, "
                                 f"got {tuple(arg.shape)} {arg.dtype}")
            if arg.data_ptr() != buf.data_ptr():
                buf.copy_(arg)

    def __call__(self, *args: torch.Tensor) -> tuple[torch.Tensor, ...]:
        self._stage(args)
        self.graph.replay()
        return self.outputs


def _as_tuple(out) -> tuple[torch.Tensor, ...]:
    return tuple(out) if isinstance(out, (tuple, list)) else (out,)


def _record(fn: Callable[..., object], static: tuple[torch.Tensor, ...], warmup: int,
            after_each_warmup: Callable[[], None] | None = None) -> GraphRunner:
    """Run ``fn(*static)`` ``warmup`` times on a side stream (so module loads and
    allocator growth happen outside the recording), then record one call on
    that same stream (per-stream state set up while warming up, such as the
    attention workspace, is then reused rather than allocated and zero-filled
    inside the graph).

    ``after_each_warmup`` runs after every eager call, still on the side stream.
    """
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn(*static)
            if after_each_warmup is not None:
                after_each_warmup()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outputs = _as_tuple(fn(*static))
    return GraphRunner(graph, static, outputs)


def capture(fn: Callable[..., object], sample_inputs: Sequence[torch.Tensor],
            warmup: int = 3) -> GraphRunner:
    """Record ``fn(*inputs)`` (shape-stable, no host synchronisation) into a graph.

    The recorded inputs are copies of ``sample_inputs``.
    """
    return _record(fn, tuple(t.clone() for t in sample_inputs), warmup)


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

        self.runner = _record(fn, tuple(t.clone() for t in sample_inputs), warmup,
                              after_each_warmup=restore)
        # Recording ran fn's host code once (its commits moved the host lengths)
        # but no kernel: restore the host side only.
        for c, (length, _, _) in zip(self.caches, saved):
            c.length = length

    def __call__(self, *args: torch.Tensor) -> tuple[torch.Tensor, ...]:
        for c in self.caches:
            c._check_room(self.rows)
        out = self.runner(*args)
        for c in self.caches:
            c.length += self.rows
        return out
