"""hipGraph capture of the forward's layer body.

Mirrors the reference's graph layer (tjkernels/graphs.py:30-91): one captured
graph per (shape, dtype, mask mode, prefix lengths, plan), replayed on every
call.  The reference captures the whole forward and copies the live input
into a static buffer and clones the static output (graphs.py:57-64); here
the engine runs the first LayerNorm (reading the caller's x) and the final
one (writing a fresh output) eagerly around the replay, so neither copy is
needed and the caller still always gets a fresh tensor.  On ROCm
``torch.cuda.CUDAGraph`` is a hipGraph; the tjk kernels launch on torch's
current stream, which is the capture stream inside ``torch.cuda.graph``.
Every tjk entry point is capture-safe (no allocation, no host sync, no
memset).
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
    """One captured launch sequence bound to fixed buffers.

    ``fn`` enqueues the work on the current stream and reads / writes only
    buffers that outlive the graph.  It runs once on a side stream (default
    priority) so lazily created state exists before capture, as torch
    requires, then is captured; ``replay`` launches it on the current stream.
    """

    def __init__(self, fn: Callable[[], None], device: torch.device, warmup: int = 1) -> None:
        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn()
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            fn()
        self.keepalive = None

    def replay(self) -> None:
        self.graph.replay()


class GraphCache:
    """Captured graphs keyed by everything that changes the captured work,
    least recently used first out beyond ``max_entries`` (keys include the
    prefix lengths of packed forwards, so distinct masks add entries)."""

    def __init__(self, max_entries: int = 16) -> None:
        self._graphs: "OrderedDict[Tuple, Optional[CapturedGraph]]" = OrderedDict()
        self.max_entries = max_entries

    def get(self, key: Tuple, fn: Callable[[], None], device: Optional[torch.device] = None,
            keepalive: object = None) -> Optional[CapturedGraph]:
        if key in self._graphs:
            self._graphs.move_to_end(key)
            return self._graphs[key]
        try:
            if device is None:
                device = torch.device("cuda", torch.cuda.current_device())
            graph = CapturedGraph(fn, device)
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
