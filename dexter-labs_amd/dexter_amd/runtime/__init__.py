"""Host-side runtime around the kernels: HIP-graph capture of control steps."""

from .graph import CachedStepGraph, GraphRunner, capture

__all__ = ["CachedStepGraph", "GraphRunner", "capture"]
