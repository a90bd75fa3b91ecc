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

With more items than resident workgroups, one workgroup per item leaves
the last items to start when the first ones end: at the C4 lengths (720
items, 512 resident workgroups) a per-workgroup timeline showed the
shortest items dispatched ~21 us into a 33 us launch, each paying ~2 us
of Q load and ring fill before its first tile, and finishing last.  So
``pack_lists`` can deal the items into at most as many lists as workgroups
are resident (largest cost first, each to the list with the least cost so
far, a cost being its key tiles plus ``ITEM_OVERHEAD``); the kernel then
runs one list per workgroup, its items back to back, and every list starts
at once.  First halves of split items go first, one at the head of each of
as many lists, so a second half never waits on an item queued behind it.
That pays where one workgroup fills a CU (head_dim 128: a CU otherwise
idles from one item's end to the next one's first tile); with two
workgroups per CU (head_dim <= 64) it measured slower than one workgroup
per item, and balancing the lists per CU (the two workgroups of a CU, the
older one faster, K/V of a head kept on one XCD's L2) did not change that:
the cost is each item's start (Q load and ring fill, ~2-3 us), which a list
runs in series like a new workgroup does (``build_schedule``).
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

BMQ, BNK = 128, 64
# An item's fixed cost (Q load, K/V ring fill, output store) in key tiles,
# for balancing lists: ~2 us against ~1.2 us per tile at C4.
ITEM_OVERHEAD = 2
HOLE = (-1, 0, 0, 0, -1)  # (b*H + h, qb, t_lo, t_hi, slot) padding a shorter list


@dataclass
class AttentionSchedule:
    work: torch.Tensor      # int32 [n_work, 4]: (b*H + h, qb, t_lo | t_hi << 16, slot)
    n_slots: int            # split items (partial slots)
    partials: torch.Tensor  # fp32 partial slots + error word + flags (zero-filled)
    max_item: int           # largest item, in key tiles
    total: int              # key tiles over all items
    error_index: int = 0    # int32 index of the kernel's error word in `partials`
    n_lists: int = 0        # workgroups: list w is items w, w + n_lists, ...; 0 = one per item


def _key_tiles(n: int, qb: int, causal: bool) -> int:
    kend = min((qb + 1) * BMQ, n) if causal else n
    return (kend + BNK - 1) // BNK


def validate_work(work: Sequence[Tuple[int, int, int, int]], lengths: Sequence[int], heads: int,
                  causal: bool, n_slots: int, n_lists: int = 0) -> None:
    """Raise ValueError unless ``work`` [(b*H + h, qb, t_lo, t_hi, slot)] --
    in array order, workgroup w running items w, w + n_lists, ... (n_lists
    0: one item per workgroup, in issue order) -- is a list the scheduled
    kernel can run: every item a ``HOLE`` or inside the launch, every
    (b, h, query block) covered by exactly one whole item or by one split
    pair whose halves tile its key range, every slot in [0, n_slots) used by
    exactly one pair, and each first half (slot s) ahead of its second half
    (slot -2 - s): before it in issue order, or at the head of a list when
    workgroups run lists."""
    lists = n_lists > 0 and n_lists < len(work)
    if n_lists < 0 or n_lists > max(len(work), 1):
        raise ValueError(f"n_lists={n_lists} outside [0, {len(work)}]")
    cover = {}
    first_at, second_at = {}, {}
    for pos, (bh, qb, lo, hi, slot) in enumerate(work):
        if (bh, qb, lo, hi, slot) == HOLE:
            continue
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
            if lists and pos >= n_lists:
                raise ValueError(f"item {pos}: first half of slot {slot} not at the head of a list")
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
        if (not lists and first_at[s][0] > second_at[s][0]) or first_at[s][1:] != second_at[s][1:]:
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


def pack_lists(work: Sequence[Tuple[int, int, int, int, int, int]], n_lists: int
               ) -> List[Tuple[int, int, int, int, int]]:
    """Deal ``work`` [(cost, b*H + h, qb, t_lo, t_hi, slot)] (build_items'
    order) into ``n_lists`` lists and lay them out for the kernel: item j of
    list w at position j * n_lists + w, shorter lists padded with ``HOLE``.
    First halves of split items are dealt first, one at the head of each of
    as many lists (there must be at most n_lists of them); then every other
    item, largest cost first, goes to the list with the least cost so far
    (ties: the lower list), a cost being tiles + ITEM_OVERHEAD.  A pure
    function of its input."""
    firsts = [w for w in work if w[5] >= 0]
    if len(firsts) > n_lists:
        raise ValueError(f"{len(firsts)} split items need as many lists (got {n_lists})")
    rest = sorted((w for w in work if w[5] < 0), key=lambda w: (-w[0], w[1], w[2], w[3]))
    lists: List[List[Tuple[int, int, int, int, int]]] = [[] for _ in range(n_lists)]
    heap = [(0, i) for i in range(n_lists)]
    for i, w in enumerate(firsts):
        lists[i].append(w[1:])
        heap[i] = (w[0] + ITEM_OVERHEAD, i)
    heapq.heapify(heap)
    for w in rest:
        load, i = heapq.heappop(heap)
        lists[i].append(w[1:])
        heapq.heappush(heap, (load + w[0] + ITEM_OVERHEAD, i))
    depth = max((len(li) for li in lists), default=0)
    return [lists[i][j] if j < len(lists[i]) else HOLE for j in range(depth) for i in range(n_lists)]


def build_schedule(lengths: Sequence[int], heads: int, head_dim: int, causal: bool,
                   dtype: torch.dtype, device: torch.device, slots: int = 0,
                   min_split: int = 6, split_factor: float = 2.0,
                   lists: Optional[bool] = None) -> AttentionSchedule:
    """``slots`` (resident workgroups) defaults to CUs x the kernel's
    occupancy.  ``lists``: run the items as per-workgroup lists when there
    are more than ``slots`` of them (None: only where one workgroup fills a
    CU, head_dim 128).  Measured on MI355X: 2 x 4096 tokens at head_dim 128
    (256 lists) 193 -> 184 us; at head_dim 64 with two workgroups per CU the
    packed C4 lengths ran 34.1 us as one workgroup per item against 35.0 as
    lists -- there the CU's other workgroup already covers a new one's start,
    and the hardware hands the next item to whichever workgroup ends first."""
    from . import _lib
    lib = _lib.load()
    occ = lib.tjk_flash_sched_occupancy(head_dim, _lib.DTYPE_CODES[dtype])
    _lib.check(0 if occ > 0 else (occ or -1), "tjk_flash_sched_occupancy")
    if slots <= 0:
        slots = occ * torch.cuda.get_device_properties(device).multi_processor_count
    if lists is None:
        lists = occ == 1
    work, n_slots = build_items(lengths, heads, causal, slots, min_split, split_factor)
    items = [(bh, qb, lo, hi, slot) for _, bh, qb, lo, hi, slot in work]
    n_lists = 0
    if lists and len(work) > slots and n_slots <= slots:
        n_lists = slots
        items = pack_lists(work, n_lists)
    validate_work(items, lengths, heads, causal, n_slots, n_lists)
    w = torch.tensor([(bh, qb, (lo | (hi << 16)) if bh >= 0 else 0, slot) for bh, qb, lo, hi, slot in items]
                     or [(0, 0, 0, -1)], dtype=torch.int32)[:len(items)]
    nbytes = lib.tjk_flash_partial_bytes(head_dim, n_slots)
    hdp = 32 if head_dim <= 32 else 64 if head_dim <= 64 else 128
    return AttentionSchedule(work=w.contiguous().to(device), n_slots=n_slots,
                             partials=torch.zeros((nbytes + 15) // 4, dtype=torch.float32, device=device),
                             max_item=max((c for c, *_ in work), default=0),
                             total=sum(c for c, *_ in work), error_index=n_slots * BMQ * (hdp + 2),
                             n_lists=n_lists)
