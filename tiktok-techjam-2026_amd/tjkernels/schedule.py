"""Work list of the scheduled attention kernel for packed sequences.

The reference launches one program per (query block, b*h) in a fixed grid
(tjkernels/kernels/attention.py:199-217).  With packed ragged sequences a
causal query block's cost is its number of key tiles, which ranges from 1 to
len/64: launched in grid order, the longest blocks set the kernel's length
while most of the GPU idles at the end.  Here, from the host-known lengths:

* every (b, h, query block of 128) is an item costing its key tiles (64 keys);
* items are issued longest first (ties broken by (b, h, block) so the list,
  and hence the result, is a pure function of the lengths);
* an item costing more than ``split_factor`` times the average work per
  resident workgroup (and at least ``min_split`` tiles) is split into two
  halves over its key range: the first (the larger, so it is issued first)
  publishes an fp32 partial, the second merges it into its own result and
  writes the output rows.

Measured on MI355X at the packed C4 lengths (bf16, hd 64): grid order
45.6 us, longest first 39.4 us; splitting every item above 1.0 / 1.2 / 1.5
times the average (192 / 80 / 16 splits) 45.3 / 40.6 / 39.5 us.  The kernel
is throughput-bound (the softmax VALU work of a 64-key tile is about twice
its MFMA time) and each half pays its own Q load and pipeline fill, so the
default ``split_factor`` = 2 only splits lists dominated by a few very long
items.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence, Tuple

import torch

BMQ, BNK = 128, 64


@dataclass
class AttentionSchedule:
    work: torch.Tensor      # int32 [n_work, 4]: (b*H + h, qb, t_lo | t_hi << 16, slot)
    n_slots: int            # split items (partial slots)
    partials: torch.Tensor  # fp32 partial slots + error word + flags (zero-filled)
    max_item: int           # largest item, in key tiles
    total: int              # key tiles over all items
    error_index: int = 0    # int32 index of the kernel's error word in `partials`


def _key_tiles(n: int, qb: int, causal: bool) -> int:
    kend = min((qb + 1) * BMQ, n) if causal else n
    return (kend + BNK - 1) // BNK


def validate_work(work: Sequence[Tuple[int, int, int, int]], lengths: Sequence[int], heads: int,
                  causal: bool, n_slots: int) -> None:
    """Raise ValueError unless ``work`` [(b*H + h, qb, t_lo, t_hi, slot)] --
    in issue order -- is a list the scheduled kernel can run: every item
    inside the launch, every (b, h, query block) covered by exactly one
    whole item or by one split pair whose halves tile its key range, first
    half (slot s) before second half (slot -2 - s), every slot in
    [0, n_slots) used by exactly one pair."""
    cover = {}
    first_at, second_at = {}, {}
    for pos, (bh, qb, lo, hi, slot) in enumerate(work):
        if not 0 <= bh < len(lengths) * heads:
            raise ValueError(f"item {pos}: (b, h) index {bh} outside the launch")
        n = lengths[bh // heads]
        nqb = (n + BMQ - 1) // BMQ
        if not 0 <= qb < nqb:
            raise ValueError(f"item {pos}: query block {qb} outside a sequence of {n}")
        if not 0 <= lo < hi <= _key_tiles(n, qb, causal) or hi >= 1 << 15:
            raise ValueError(f"item {pos}: key tiles [{lo}, {hi}) outside [0, {_key_tiles(n, qb, causal)})")
        if slot >= 0:
            if slot >= n_slots or slot in first_at:
                raise ValueError(f"item {pos}: first-half slot {slot} invalid or repeated")
            first_at[slot] = (pos, bh, qb)
        elif slot <= -2:
            s = -2 - slot
            if s >= n_slots or s in second_at:
                raise ValueError(f"item {pos}: second-half slot {s} invalid or repeated")
            second_at[s] = (pos, bh, qb)
        elif slot != -1:
            raise ValueError(f"item {pos}: bad slot {slot}")
        cover.setdefault((bh, qb), []).append((lo, hi, slot))
    for s in range(n_slots):
        if s not in first_at or s not in second_at:
            raise ValueError(f"slot {s} lacks a first or second half")
        if first_at[s][0] > second_at[s][0] or first_at[s][1:] != second_at[s][1:]:
            raise ValueError(f"slot {s}: halves out of order or of different query blocks")
    for b, n in enumerate(lengths):
        for h in range(heads):
            for qb in range((n + BMQ - 1) // BMQ):
                got = sorted(cover.pop((b * heads + h, qb), []))
                nkt = _key_tiles(n, qb, causal)
                ok = (len(got) == 1 and got[0][:3] == (0, nkt, -1)) or (
                    len(got) == 2 and got[0][0] == 0 and got[0][1] == got[1][0] and got[1][1] == nkt
                    and got[0][2] >= 0 and got[1][2] == -2 - got[0][2])
                if not ok:
                    raise ValueError(f"(b={b}, h={h}, qb={qb}) covered by {got}, expected [0, {nkt})")
    if cover:
        raise ValueError(f"items for query blocks outside the sequences: {sorted(cover)[:4]}")


def error_count(schedule: "AttentionSchedule") -> int:
    """The kernel's error word (items it could not run as listed; a host
    sync).  Zero unless a wait timed out or the list was corrupted."""
    return int(schedule.partials.view(torch.int32)[schedule.error_index].item())


def build_items(lengths: Sequence[int], heads: int, causal: bool, slots: int, min_split: int = 6,
                split_factor: float = 2.0) -> Tuple[List[Tuple[int, int, int, int, int, int]], int]:
    """[(cost, b*H + h, qb, t_lo, t_hi, slot)] in issue order, and the number
    of partial slots.  slot -1: whole item; s >= 0: first half of split item
    s; -2 - s: its second half."""
    items = []
    for b, n in enumerate(lengths):
        for qb in range((n + BMQ - 1) // BMQ):
            kend = min((qb + 1) * BMQ, n) if causal else n
            nkt = (kend + BNK - 1) // BNK
            for h in range(heads):
                items.append((nkt, b * heads + h, qb))
    total = sum(c for c, _, _ in items)
    target = max(split_factor * total / max(slots, 1), float(min_split))
    work, n_slots = [], 0
    for nkt, bh, qb in items:
        if nkt > target:
            mid = (nkt + 1) // 2
            work.append((mid, bh, qb, 0, mid, n_slots))
            work.append((nkt - mid, bh, qb, mid, nkt, -2 - n_slots))
            n_slots += 1
        else:
            work.append((nkt, bh, qb, 0, nkt, -1))
    # the first half of a split item is at least as long and starts at key
    # tile 0, so it sorts before its second half
    work.sort(key=lambda w: (-w[0], w[1], w[2], w[3]))
    return work, n_slots


def build_schedule(lengths: Sequence[int], heads: int, head_dim: int, causal: bool,
                   dtype: torch.dtype, device: torch.device, slots: int = 0,
                   min_split: int = 6, split_factor: float = 2.0) -> AttentionSchedule:
    """``slots`` (resident workgroups) defaults to CUs x the kernel's occupancy."""
    from . import _lib
    lib = _lib.load()
    if slots <= 0:
        occ = lib.tjk_flash_sched_occupancy(head_dim, _lib.DTYPE_CODES[dtype])
        _lib.check(0 if occ > 0 else (occ or -1), "tjk_flash_sched_occupancy")
        slots = occ * torch.cuda.get_device_properties(device).multi_processor_count
    work, n_slots = build_items(lengths, heads, causal, slots, min_split, split_factor)
    validate_work([(bh, qb, lo, hi, slot) for _, bh, qb, lo, hi, slot in work], lengths, heads, causal, n_slots)
    w = torch.tensor([(bh, qb, lo | (hi << 16), slot) for _, bh, qb, lo, hi, slot in work] or [(0, 0, 0, -1)],
                     dtype=torch.int32)[:len(work)]
    nbytes = lib.tjk_flash_partial_bytes(head_dim, n_slots)
    hdp = 32 if head_dim <= 32 else 64 if head_dim <= 64 else 128
    return AttentionSchedule(work=w.contiguous().to(device), n_slots=n_slots,
                             partials=torch.zeros((nbytes + 15) // 4, dtype=torch.float32, device=device),
                             max_item=max((c for c, *_ in work), default=0),
                             total=sum(c for c, *_ in work), error_index=n_slots * BMQ * (hdp + 2))
