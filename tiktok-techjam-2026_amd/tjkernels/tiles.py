"""Measured GEMM tile choice per (M, N, K, dtype, epilogue).

With packed prefix-masked tokens the row count M of every projection is
the number of valid tokens, which changes with the input lengths, and the
best tile shape depends on how the tile count falls onto the 256 CUs (a
launch whose last round holds a handful of tiles costs nearly a full
round).  No fixed table covers that, so the first time a projection shape is
seen its candidate tile plans are timed on scratch operands of that exact
shape (HIP events on the current stream) and the fastest is kept for the
rest of the process.  Every candidate accumulates each output element over
K in the same order, so the choice changes speed, not results.  (The
K-split plans 16 / 17 add two half-K partial sums instead; they measured
no faster on the BASELINE shapes and are only used when a Plan forces them.)

This replaces the reference's static per-shape table lookup for the GEMM
part of a plan (tjkernels/plans.py:147-170); plan ids >= 0 in a ``Plan``
still force a specific tile.  ``TJ_GEMM_TUNE=0`` falls back to the
library's own rule (plan -1).
"""

from __future__ import annotations

import os
from typing import Dict, Tuple

import torch

from . import _lib, ops, timing

# Direct-to-LDS tile plans worth timing (2-byte types): 128x128, 256x256,
# 64x64, 192x128, 192x256, 192x384, 96x128, 192x128 in a 4-slot ring,
# 64x64 / 128x64 in 8- / 6-slot rings, and 64x64 / 128x64 with K split
# between 2 or 4 wave groups.  fp32 uses its own list.
CANDIDATES_16 = (7, 8, 9, 12, 13, 14, 15, 26, 27, 28, 29, 30, 31)
CANDIDATES_32 = (2, 3, 4)

_choice: Dict[Tuple, int] = {}


def _time_plan(a, w, bias, out, epi, plan, reps) -> float:
    return timing.launch_ms(lambda: ops.gemm(a, w, bias, out, epi, plan), reps)


def gemm_plan(m: int, n: int, k: int, dtype: torch.dtype, epilogue: int, forced: int = -1) -> int:
    """Tile plan for out[m, n] = epi(a[m, k] w[n, k]^T + b); ``forced`` >= 0 wins."""
    if forced >= 0 or m == 0:
        return forced
    if os.environ.get("TJ_GEMM_TUNE") == "0" or torch.cuda.is_current_stream_capturing():
        return _choice.get((m, n, k, dtype, epilogue), -1)
    key = (m, n, k, dtype, epilogue)
    plan = _choice.get(key)
    if plan is not None:
        return plan
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator(device=dev)
    g.manual_seed(m * 7919 + n * 31 + k)
    a = torch.randn(m, k, device=dev, generator=g).to(dtype)
    w = (torch.randn(n, k, device=dev, generator=g) * k ** -0.5).to(dtype)
    bias = torch.zeros(n, device=dev, dtype=dtype)
    out = torch.empty(m, n, device=dev,
                      dtype=torch.float32 if epilogue == ops.EPI_BIAS_RESIDUAL else dtype)
    # about 0.4 ms of GPU work per measurement (estimated at 500 TFLOP/s)
    reps = max(3, min(24, int(0.4e-3 / (2.0 * m * n * k / 500e12))))
    cands = []
    for cand in (CANDIDATES_32 if dtype == torch.float32 else CANDIDATES_16):
        try:
            ops.gemm(a, w, bias, out, epilogue, cand)  # warm; rejects shapes it does not take
        except _lib.TjkError:  # e.g. K % 64 != 0
            continue
        cands.append(cand)
    # Three interleaved rounds, best time per candidate: the clock drifts
    # (power / thermal) while this runs, and a single pass in order would
    # hand the early candidates the cooler chip.
    times = {c: float("inf") for c in cands}
    for rnd in range(3):
        order = cands if rnd % 2 == 0 else cands[::-1]
        for cand in order:
            times[cand] = min(times[cand], _time_plan(a, w, bias, out, epilogue, cand, reps))
    best, best_ms = -1, float("inf")
    for cand in cands:  # earlier (larger-reuse) candidates win near ties
        if times[cand] < best_ms * 0.98:
            best, best_ms = cand, times[cand]
    _choice[key] = best
    return best


def reset() -> None:
    _choice.clear()
