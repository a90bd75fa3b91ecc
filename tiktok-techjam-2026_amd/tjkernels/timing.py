"""GPU-side timing of short launches.

A launch through the C-ABI costs the host some tens of microseconds
(argument checks, ctypes), comparable with the kernels being timed (an
out-projection GEMM of a C4 forward runs ~20 us).  Timed back to back from
an idle GPU, such launches run at the host's issue rate, and HIP events
between them measure the host, not the kernel.  ``queue_ahead`` first puts a
spin kernel of a chosen length on the stream, so the launches that follow
are queued while it runs and then execute back to back; the events around
them then read GPU time only.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch

_cycles_per_ms: Optional[float] = None


def _rate() -> float:
    global _cycles_per_ms
    if _cycles_per_ms is None:
        torch.cuda._sleep(1000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        e1.synchronize()
        _cycles_per_ms = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    return _cycles_per_ms


def queue_ahead(ms: float) -> None:
    """Occupy the current stream for about ``ms`` milliseconds."""
    torch.cuda._sleep(max(1, int(ms * _rate())))


def launch_ms(fn: Callable[[], object], reps: int, host_us_per_launch: float = 60.0) -> float:
    """Average GPU time of one ``fn()`` over ``reps`` queued launches."""
    queue_ahead(0.2 + reps * host_us_per_launch * 1e-3)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / reps
