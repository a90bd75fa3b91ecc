"""Whole-forward hipGraph capture.

Mirrors the reference's graph layer (tjkernels/graphs.py:30-91): one captured
forward per (shape, dtype, mask mode); every call copies the live input (and
mask) into the captured static buffers, replays, and returns a clone of the
static output, so results are correct for any input and the caller always
gets a fresh tensor.  On ROCm ``torch.cuda.CUDAGraph`` is a hipGraph; the
tjk kernels launch on torch's current stream, which is the capture stream
inside ``torch.cuda.graph``.  Every tjk entry point is capture-safe (no
allocation, no host sync, no memset).
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Callable, Optional, Tuple

import torch

_WARNED = False


def _warn_once(msg: str) -> None:
    global _WARNED
    if not _WARNED:
        _WARNED = True
        print(f"[tjkernels] {msg}")


class CapturedGraph:
    """One captured forward bound to one input shape / dtype / mask mode."""

    def __init__(self, fn: Callable[[torch.Tensor, Optional[torch.Tensor]], torch.Tensor],
                 x: torch.Tensor, mask: Optional[torch.Tensor], warmup: int = 2) -> None:
        self.static_x = x.clone()
        self.static_mask = None if mask is None else mask.clone()
        # Warm up on a side stream (default priority) so lazily created
        # state exists before capture, as torch requires.
        side = torch.cuda.Stream(device=x.device)
        side.wait_stream(torch.cuda.current_stream(x.device))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn(self.static_x, self.static_mask)
        torch.cuda.current_stream(x.device).wait_stream(side)
        torch.cuda.synchronize(x.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_out = fn(self.static_x, self.static_mask)

    def run(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
        self.static_x.copy_(x)
        if self.static_mask is not None and mask is not None:
            self.static_mask.copy_(mask)
        self.graph.replay()
        return self.static_out.clone()


class GraphCache:
    """Captured graphs keyed by everything that changes the captured work,
    least recently used first out beyond ``max_entries`` (keys include the
    prefix lengths of packed forwards, so distinct masks add entries)."""

    def __init__(self, max_entries: int = 16) -> None:
        self._graphs: "OrderedDict[Tuple, Optional[CapturedGraph]]" = OrderedDict()
        self.max_entries = max_entries

    def get(self, key: Tuple, fn, x: torch.Tensor, mask: Optional[torch.Tensor],
            keepalive: object = None) -> Optional[CapturedGraph]:
        if key in self._graphs:
            self._graphs.move_to_end(key)
            return self._graphs[key]
        try:
            graph = CapturedGraph(fn, x, mask)
            graph.keepalive = keepalive  # device buffers the captured kernels read
        except Exception as exc:  # capture is an optimisation; eager HIP still runs
            _warn_once(f"hipGraph capture failed ({exc}); running eager.")
            graph = None
        self._graphs[key] = graph
        while len(self._graphs) > self.max_entries:
            self._graphs.popitem(last=False)
        return graph

    def clear(self) -> None:
        self._graphs.clear()

    def __len__(self) -> int:
        return len(self._graphs)
