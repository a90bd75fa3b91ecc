"""Measured GEMM tile choice per projection shape, deterministic in its results.

With packed prefix-masked tokens the row count M of every projection is the
number of valid tokens, which follows the input lengths, and the best tile
depends on how the tile count falls onto the 256 CUs (a launch whose last
round holds a handful of tiles costs nearly a full round).  No fixed table
covers that, so the first time a projection shape is seen the candidate
tiles are timed on scratch operands and the fastest is kept.

Timing noise must not change results.  The tile plans fall into classes by
the order in which they add up the K dimension:

* class 1: one accumulator per output element, K tiles in order;
* class 2: two wave groups take alternate K tiles and their two sums are
  added at the end (the in-workgroup K split);
* class 4: four wave groups take every 4th K tile, their sums added in group
  order at the end.

Every plan of a class produces the same bits for the same inputs, so the
class is fixed by the shape (``k_class``) and only tiles within it are
timed.  Two processes, or two boxes, therefore compute identical outputs
whatever the timing picks.  ``k_class`` chooses the K split when a launch of
128 x 64 tiles fits in one round of the CUs and K is long enough for the
split to shorten the serial chain of K tiles (the launch-bound projections
of C2 and C3's FFN2: 10.6 -> 8.5 us and 26.1 -> 23.0 us measured on MI355X),
and the four-way split when one round of 32 x 64 tiles covers the launch and
K >= 2048 (C2's FFN2).

The LayerNorm-prologue GEMM (``tjk_gemm_ln``, LayerNorm computed inside
the GEMM for launch-bound row counts) has its own plans, 32-row tiles of
32 / 64 / 128 columns that all sum K in one chain: ``gemm_ln_plan`` times
them the same way (any pick gives the same bits).

The table is keyed by M rounded up to a multiple of 64 (the timing runs at
that M), so ragged lengths reuse a measurement, and it holds at most
``MAX_ENTRIES`` shapes.  This replaces the reference's static per-shape
table lookup for the GEMM part of a plan (tjkernels/plans.py:147-170); tile
ids >= 0 in a ``Plan`` still force a tile, at the row bucket
``Plan.tile_rows`` names (the autotuner's tiles, timed inside whole
forwards, where the ranking of near-equal tiles differs from this timing
of lone launches) or at every row count when it is 0.  ``TJ_GEMM_TUNE=0``
uses the library's own rule (tile -1) instead of timing.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from typing import Tuple

import torch

from . import _lib, ops, timing

# Direct-to-LDS plans of the 2-byte table by K order (ids of tjk_gemm_plan_info):
# class 1: 128x128, 256x256 (8 waves), 64x64, 192x128, 192x256, 192x384,
#          96x128, 192x128 in a 4-slot ring, 64x64 / 128x64 in 8- / 6-slot rings,
#          and the wave-specialized tiles (compute waves + DMA-only loader
#          waves): 192x128 with 4 compute waves in a 4-slot ring, with 8 in 3-
#          and 4-slot rings, 192x256 with 8 in 2 slots, 128x256 with 8 in 3;
# class 2: 192x128, 128x128, 64x64 (4-slot ring), 128x64 (3-slot ring), each
#          with K split between two groups of 4 waves; 32x64 and 32x32
#          (4-slot rings) with K split between two groups of 2 / 1 waves;
# class 4: 64x64 (2-slot rings), 32x32 (4-slot) and 32x64 (3-slot) with K split
#          between four groups of 4 / 1 / 2 waves.
CLASS_TILES_16 = {1: (7, 8, 9, 12, 13, 14, 15, 18, 19, 20, 28, 29, 30, 31, 32), 2: (16, 17, 22, 23, 24, 25),
                  4: (21, 26, 27)}
CANDIDATES_32 = (2, 3, 4)  # fp32: class 1 only
MAX_ENTRIES = 256
M_BUCKET = 64

_choice: "OrderedDict[Tuple, int]" = OrderedDict()


def k_class(m: int, n: int, k: int, dtype: torch.dtype) -> int:
    """K-summation class of the tile used for out[m, n] = a[m, k] w[n, k]^T."""
    if dtype == torch.float32:
        return 1
    if ((m + 31) // 32) * ((n + 63) // 64) <= 256 and k >= 2048:
        return 4
    one_round = ((m + 127) // 128) * ((n + 63) // 64) <= 256
    return 2 if one_round and k >= 512 else 1


def candidates(m: int, n: int, k: int, dtype: torch.dtype) -> Tuple[int, ...]:
    if dtype == torch.float32:
        return CANDIDATES_32
    return CLASS_TILES_16[k_class(m, n, k, dtype)]


def _measure(m: int, n: int, k: int, dtype: torch.dtype, epilogue: int, ln: bool = False) -> int:
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator(device=dev)
    g.manual_seed(m * 7919 + n * 31 + k)
    a = torch.randn(m, k, device=dev, generator=g)  # fp32: the LayerNorm GEMM's residual
    if not ln:
        a = a.to(dtype)
    w = (torch.randn(n, k, device=dev, generator=g) * k ** -0.5).to(dtype)
    bias = torch.zeros(n, device=dev, dtype=dtype)
    gamma, beta = torch.ones(k, device=dev), torch.zeros(k, device=dev)
    out = torch.empty(m, n, device=dev,
                      dtype=torch.float32 if epilogue == ops.EPI_BIAS_RESIDUAL else dtype)
    if ln:
        def run(plan):
            ops.gemm_ln(a, gamma, beta, 1e-5, w, bias, out, epilogue, plan)
        plans = tuple(range(ops.gemm_ln_plan_count()))
    else:
        def run(plan):
            ops.gemm(a, w, bias, out, epilogue, plan)
        plans = candidates(m, n, k, dtype)
    # about 1.5 ms of GPU work per measurement (estimated at 500 TFLOP/s):
    # with 0.4 ms and three rounds the packed C4 FFN1 / FFN2 picks moved
    # between tiles 2-5% apart from one process to the next
    reps = max(3, min(64, int(1.5e-3 / (2.0 * m * n * k / 500e12))))
    cands = []
    for cand in plans:
        try:
            run(cand)  # warm; rejects shapes it does not take
        except _lib.TjkError:  # e.g. K % 64 != 0
            continue
        cands.append(cand)
    if not cands:
        return -1
    # Five interleaved rounds, best time per candidate: the clock drifts
    # (power / thermal) while this runs, and a single pass in order would
    # hand the early candidates the cooler chip.
    times = {c: float("inf") for c in cands}
    for rnd in range(5):
        for cand in (cands if rnd % 2 == 0 else cands[::-1]):
            times[cand] = min(times[cand], timing.launch_ms(lambda: run(cand), reps))
    best, best_ms = cands[0], times[cands[0]]
    for cand in cands[1:]:  # earlier (larger-reuse) candidates win near ties
        if times[cand] < best_ms * 0.98:
            best, best_ms = cand, times[cand]
    return best


def gemm_plan(m: int, n: int, k: int, dtype: torch.dtype, epilogue: int, forced: int = -1) -> int:
    """Tile plan for out[m, n] = epi(a[m, k] w[n, k]^T + b); ``forced`` >= 0 wins."""
    if forced >= 0 or m == 0:
        return forced
    mb = -(-m // M_BUCKET) * M_BUCKET
    key = (mb, n, k, dtype, epilogue)
    plan = _choice.get(key)
    if plan is not None:
        _choice.move_to_end(key)
        return plan
    if os.environ.get("TJ_GEMM_TUNE") == "0" or torch.cuda.is_current_stream_capturing():
        return -1
    plan = _measure(mb, n, k, dtype, epilogue)
    _choice[key] = plan
    while len(_choice) > MAX_ENTRIES:
        _choice.popitem(last=False)
    return plan


def gemm_ln_plan(m: int, n: int, k: int, dtype: torch.dtype, epilogue: int, forced: int = -1) -> int:
    """Column-tile plan of tjk_gemm_ln for out[m, n] = epi(LN(res[m, k]) w[n, k]^T + b)."""
    if forced >= 0 or m == 0:
        return forced
    mb = -(-m // M_BUCKET) * M_BUCKET
    key = ("ln", mb, n, k, dtype, epilogue)
    plan = _choice.get(key)
    if plan is not None:
        _choice.move_to_end(key)
        return plan
    if os.environ.get("TJ_GEMM_TUNE") == "0" or torch.cuda.is_current_stream_capturing():
        return -1
    plan = _measure(mb, n, k, dtype, epilogue, ln=True)
    _choice[key] = plan
    while len(_choice) > MAX_ENTRIES:
        _choice.popitem(last=False)
    return plan


def chosen() -> dict:
    """{(M bucket, N, K, dtype, epilogue): tile} measured so far (the
    LayerNorm GEMM's entries keyed ("ln", M bucket, N, K, dtype, epilogue))."""
    return dict(_choice)


def describe() -> dict:
    """The choices as {"MxNxK/epiE": tile}, LayerNorm GEMM entries prefixed
    "ln:", in shape order."""
    out = {}
    for key, plan in sorted(_choice.items(), key=lambda kv: (kv[0][0] == "ln", kv[0][-5:-2])):
        m, n, k, _, e = key[-5:]
        out[f"{'ln:' if key[0] == 'ln' else ''}{m}x{n}x{k}/epi{e}"] = plan
    return out


def reset() -> None:
    _choice.clear()
