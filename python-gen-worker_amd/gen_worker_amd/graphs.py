"""HIP graph capture shared by the benchmarks, the lane gates and the DiT step timer."""

from __future__ import annotations

import gc
from typing import Any, Callable, Optional

import torch


def capture_graph(fn: Callable[[], Any], stream: Optional["torch.cuda.Stream"] = None
                  ) -> tuple["torch.cuda.CUDAGraph", Any]:
    """``fn()`` captured into a new HIP graph on ``stream`` (default: a fresh stream), which first waits for
    the current one; returns (graph, fn's result), synchronized. Garbage is collected before the capture and
    Python's cyclic collector stays off during it, so no tensor held by a dead reference cycle is released
    while the graph is captured (torch's capture no longer collects first)."""
    gc.collect()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        s = stream if stream is not None else torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                out = fn()
        torch.cuda.synchronize()
    finally:
        if was_enabled:
            gc.enable()
    return g, out


__all__ = ["capture_graph"]
