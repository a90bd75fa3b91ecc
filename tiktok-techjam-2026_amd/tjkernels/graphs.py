"""hipGraph capture of the forward's layer body (the reference's graph layer,
tjkernels/graphs.py:30-91).

One captured graph per (shape, dtype, mask mode, prefix lengths, plan),
replayed on every later call with that key.  The reference captures the
whole forward and copies the live input into a static buffer, then clones
the static output (graphs.py:57-64).  Here the engine launches the first
LayerNorm (which reads the caller's x) and the final one (which writes a
fresh output tensor) on the stream around the replay, so neither copy
exists and the caller still always receives a new tensor.

On ROCm ``torch.cuda.CUDAGraph`` is a hipGraph.  The tjk kernels launch on
torch's current stream, which is the capture stream inside
``torch.cuda.graph``, and every tjk entry point is capture-safe (no
allocation, no host sync, no memset).
"""

from __future__ import annotations

import warnings
from collections import OrderedDict
from typing import Callable, Hashable, Optional, Tuple

import torch


class CaptureFailed(UserWarning):
    """A hipGraph capture raised; the forward runs eagerly instead."""


class CapturedGraph:
    """A launch sequence recorded once and replayed on the current stream.

    ``body`` must enqueue its work on the current stream and touch only
    buffers that outlive the graph.  It runs ``warmup`` times on a side
    stream first (default priority), so that everything created lazily
    (library handles, caches) exists before capture, as torch requires."""

    def __init__(self, body: Callable[[], None], device: torch.device, warmup: int = 1,
                 keepalive: object = None) -> None:
        origin = torch.cuda.current_stream(device)
        side = torch.cuda.Stream(device=device)
        side.wait_stream(origin)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                body()
        origin.wait_stream(side)
        torch.cuda.synchronize(device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            body()
        # device buffers the recorded kernels read or write (row maps,
        # schedules, workspaces): held for as long as the graph can replay
        self.keepalive = keepalive

    def replay(self) -> None:
        self.graph.replay()


class GraphCache:
    """Captured graphs by key, least recently used dropped beyond
    ``max_entries``.  A failed capture is remembered as None, so the caller
    runs eagerly for that key without trying again."""

    def __init__(self, max_entries: int = 16) -> None:
        self.max_entries = max_entries
        self._entries: "OrderedDict[Hashable, Optional[CapturedGraph]]" = OrderedDict()

    def get(self, key: Hashable, body: Callable[[], None], device: Optional[torch.device] = None,
            keepalive: object = None) -> Optional[CapturedGraph]:
        if key in self._entries:
            self._entries.move_to_end(key)
            return self._entries[key]
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        try:
            entry: Optional[CapturedGraph] = CapturedGraph(body, dev, keepalive=keepalive)
        except Exception as exc:  # capture is an optimisation: the eager launches stay correct
            warnings.warn(f"[tjkernels] hipGraph capture failed ({exc}); running eagerly",
                          CaptureFailed, stacklevel=2)
            entry = None
        self._entries[key] = entry
        if len(self._entries) > self.max_entries:
            self._entries.popitem(last=False)
        return entry

    def lookup(self, key: Hashable) -> Tuple[bool, Optional[CapturedGraph]]:
        """(key present, its graph or None for a failed capture), marking the
        key as the most recently used; no capture happens."""
        if key not in self._entries:
            return False, None
        self._entries.move_to_end(key)
        return True, self._entries[key]

    def __contains__(self, key: Hashable) -> bool:
        return key in self._entries

    def clear(self) -> None:
        self._entries.clear()

    def __len__(self) -> int:
        return len(self._entries)
