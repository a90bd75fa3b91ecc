"""Per-kernel-class summary of a rocprofv3 run of ``bench.py``.

    python -m tjkernels.rocprof_summary TRACE.csv [--fetch FETCH.csv --write WRITE.csv]
                                        [--pmc PMC.csv ...] [--cus 256]
                                        [--layers 4] [--copy-calib-bytes 268435456]

TRACE.csv is ``*_kernel_trace.csv`` of ``rocprofv3 --kernel-trace``; FETCH /
WRITE are ``*_counter_collection.csv`` of two ``rocprofv3 --pmc FETCH_SIZE``
/ ``--pmc WRITE_SIZE`` runs.  Kernels are labelled by their position in the
forward: the forward's launch sequence is fixed (first LayerNorm, then per
layer QKV GEMM, attention, out-proj GEMM, and either LayerNorm + FFN1 GEMM +
FFN2 GEMM or the single-launch FFN, LayerNorm, and the final LayerNorm), so
every complete sequence that starts with the first LayerNorm (the one
reading the model-dtype input) is split into labelled launches.  Sequences
are grouped by the first LayerNorm's grid (the packed forward has fewer rows
than the all-rows one) and by their kernel names (a forward of the same rows
through other kernels, such as the bench's masked comparison run), and each
group is reported separately.  HBM bytes per launch are FETCH_SIZE and WRITE_SIZE
(KiB per dispatch) scaled by what the same counters read for the bench's
plain 256 MiB copy (``__amd_rocclr_copyBuffer`` of 268435456 bytes read and
written).  ``--pmc`` takes ``*_counter_collection.csv`` files of runs with
several counters each and tabulates the mean per dispatch of every counter
per label, with the derived figures:

* MFMA busy % = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x CUs x 4
  SIMDs): GRBM_GUI_ACTIVE is summed over the XCDs, SQ_VALU_MFMA_BUSY_CYCLES
  over the SIMDs (32 per v_mfma_f32_32x32x16 -- the C4 QKV GEMM's count is
  exactly 32 x its SQ_INSTS_MFMA, which is M N K / (32 32 16));
* LDS bank-conflict share = SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS;
* VALU instructions per MFMA instruction = SQ_INSTS_VALU / SQ_INSTS_MFMA
  (SQ_INSTS_VALU counts the MFMAs too; they are subtracted);
* transcendental share = SQ_INSTS_VALU_TRANS_F32 / (SQ_INSTS_VALU - SQ_INSTS_MFMA).
"""

from __future__ import annotations

import argparse
import collections
import csv
import re
from typing import Dict, List, Optional, Tuple

# add_layernorm_kernel and add_layernorm_parts_kernel (the split-delta sum
# after the single-launch FFN) both count as LayerNorm launches; a GEMM
# launch is the direct-to-LDS kernel or the wave-specialized one
GEMM, FLASH, LN, FFN = "gemm_dtl_kernel", "flash_", "add_layernorm", "ffn_fused_kernel"
GEMM_WS = "gemm_ws_kernel"


def _is_gemm(name: str) -> bool:
    return GEMM in name or GEMM_WS in name
COPY = "__amd_rocclr_copyBuffer"


def _is_first_ln(name: str) -> bool:
    # add_layernorm_kernel<TRes, TDelta, TOut, ...>: TRes is the model dtype
    # (bf16 / fp16) for the first LayerNorm, fp32 for every other one.
    return LN in name and ("add_layernorm_kernelIDF16b" in name or "add_layernorm_kernelIDF16_" in name)


def _labels(layers: int, fused: bool = False) -> List[str]:
    seq = ["ln_first"]
    for i in range(layers):
        if i:
            seq.append("add_layernorm")
        seq += ["gemm_qkv", "flash_attention", "gemm_out_residual"]
        seq += ["ffn_fused"] if fused else ["add_layernorm", "gemm_ffn1_gelu", "gemm_ffn2_residual"]
    seq.append("ln_final")
    return seq


def _gemm_epilogue(name: str) -> Optional[int]:
    """EPI template argument of a gemm_dtl_kernel<T, BM, BN, WM, WN, BKB,
    STAGES, EPI, KSPLIT> or gemm_ws_kernel<T, BM, BN, WM, WN, STAGES, L, EPI>
    name, the seventh integer in both (2: residual read-modify-write, 4:
    residual read from the input x, the first layer's out-proj)."""
    kern = GEMM if GEMM in name else GEMM_WS if GEMM_WS in name else None
    ints = re.findall(r"Li(\d+)E", name.split(kern, 1)[1]) if kern else []
    return int(ints[6]) if len(ints) >= 7 else None


def _relabel(label: str, name: str) -> str:
    # the out-proj / FFN2 of a deferred-residual plan write their output for
    # the next LayerNorm instead of adding into the residual
    if label.endswith("_residual") and _gemm_epilogue(name) not in (None, 2, 4):
        return label[:-len("_residual")]
    return label


def _kind_ok(label: str, name: str) -> bool:
    return (_is_gemm(name) == label.startswith("gemm") and (FLASH in name) == (label == "flash_attention")
            and (FFN in name) == (label == "ffn_fused"))


def _grid(r: dict) -> int:
    return int(r.get("Grid_Size") or r["Grid_Size_X"])


def _wg(r: dict) -> int:
    return int(r.get("Workgroup_Size") or r["Workgroup_Size_X"])


def _tjk(name: str) -> bool:
    return _is_gemm(name) or FLASH in name or LN in name or FFN in name


def _forwards(rows: List[dict], layers: int) -> Dict[Tuple, List[List[Tuple[str, dict]]]]:
    """{(first-LN grid, kernel names): [forward as [(label, row)]]} from
    dispatch-ordered rows.  The names split forwards of one grid that run
    different kernels (C5's timed forward and the bench's masked comparison
    run have the same rows)."""
    tjk = [r for r in rows if _tjk(r["Kernel_Name"])]
    out: Dict[Tuple, List[List[Tuple[str, dict]]]] = collections.defaultdict(list)
    i = 0
    while i < len(tjk):
        matched = False
        if _is_first_ln(tjk[i]["Kernel_Name"]):
            for labels in (_labels(layers), _labels(layers, fused=True)):
                seq = tjk[i:i + len(labels)]
                if (len(seq) == len(labels) and all(_kind_ok(lab, r["Kernel_Name"]) for lab, r in zip(labels, seq))
                        and not any(_is_first_ln(r["Kernel_Name"]) for r in seq[1:])):
                    out[(_grid(seq[0]), tuple(r["Kernel_Name"] for r in seq))].append(
                        [(_relabel(lab, r["Kernel_Name"]), r) for lab, r in zip(labels, seq)])
                    i += len(labels)
                    matched = True
                    break
        if not matched:
            i += 1
    return out


def _timed(groups: Dict[Tuple, list]) -> Tuple:
    """Key of the forward group the bench times: the one with the most
    forwards (its warm-up, breakdown and timed steps; the bench's masked
    comparison forward runs once or twice and may share the first grid)."""
    return max(groups, key=lambda k: (len(groups[k]), k))


def _dur_us(r: dict) -> float:
    return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3


# bench.py's traffic-calibration GEMM: 64 x 65536 x 1024 bf16 in 64 x 64
# tiles (1024 workgroups of 256 threads); bytes it must fetch: the weight
# once, plus the 128 KiB A and 128 KiB bias once per XCD
CALIB_GEMM_GRID = 1024 * 256
CALIB_GEMM_FETCH = 65536 * 1024 * 2 + 8 * (64 * 1024 * 2 + 65536 * 2)
CALIB_GEMM_WRITE = 64 * 65536 * 2


def _counter(path: str) -> Tuple[List[dict], Optional[float]]:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    copies = [float(r["Counter_Value"]) for r in rows if r["Kernel_Name"] == COPY]
    return rows, (max(copies) if copies else None)


def _calib_gemm_kib(rows: List[dict]) -> Optional[float]:
    """Counter value of the calibration GEMM: the first 64 x 64-tile GEMM
    dispatch of its grid after the calibration copy (rows in dispatch
    order; other launches of the same grid, e.g. 256 x 256 tiles of 8 waves,
    are not it)."""
    copies = [i for i, r in enumerate(rows) if r["Kernel_Name"] == COPY]
    if not copies:
        return None
    big = max(copies, key=lambda i: float(rows[i]["Counter_Value"]))
    for r in rows[big + 1:]:
        name = r["Kernel_Name"]
        if GEMM in name and _grid(r) == CALIB_GEMM_GRID and "Li64ELi64ELi2ELi2ELi128ELi2ELi0E" in name:
            return float(r["Counter_Value"])
    return None


def _pmc_by_label(paths: List[str], layers: int) -> Dict[str, Dict[str, float]]:
    """{label: {counter: mean per dispatch}} over the timed forward group of
    each multi-counter counter-collection file."""
    out: Dict[str, Dict[str, float]] = collections.defaultdict(dict)
    for path in paths:
        rows = list(csv.DictReader(open(path)))
        by_dispatch: Dict[int, Dict[str, float]] = collections.defaultdict(dict)
        meta: Dict[int, dict] = {}
        for r in rows:
            d = int(r["Dispatch_Id"])
            by_dispatch[d][r["Counter_Name"]] = by_dispatch[d].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            meta[d] = r
        disp = [dict(meta[d], _counters=by_dispatch[d]) for d in sorted(meta)]
        groups = _forwards(disp, layers)
        if not groups:
            continue
        acc: Dict[str, Dict[str, List[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
        for f in groups[_timed(groups)]:
            for lab, r in f:
                for name, v in r["_counters"].items():
                    acc[lab][name].append(v)
        for lab, counters in acc.items():
            for name, vals in counters.items():
                out[lab][name] = sum(vals) / len(vals)
    return out


def pmc_table(paths: List[str], layers: int = 4, cus: int = 256, xcds: int = 8) -> str:
    data = _pmc_by_label(paths, layers)
    if not data:
        return "no complete forward found in the counter files"
    names = sorted({n for c in data.values() for n in c})
    lines = ["Counters per dispatch (mean over the forward's launches of each label):",
             f"{'label':<20} " + " ".join(f"{n:>26}" for n in names)]
    for lab, c in data.items():
        lines.append(f"{lab:<20} " + " ".join(f"{c.get(n, float('nan')):>26.4g}" for n in names))
    lines.append("")
    lines.append(f"{'label':<20} {'MFMA busy %':>12} {'VALU/MFMA':>10} {'trans share':>12} {'LDS conflict':>13}")
    for lab, c in data.items():
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES")
        gui = c.get("GRBM_GUI_ACTIVE")
        mf = c.get("SQ_INSTS_MFMA")
        va = c.get("SQ_INSTS_VALU")
        tr = c.get("SQ_INSTS_VALU_TRANS_F32")
        util = 100.0 * busy / (gui / xcds * cus * 4) if busy is not None and gui else None
        conf, lds = c.get("SQ_LDS_BANK_CONFLICT"), c.get("SQ_ACTIVE_INST_LDS")
        cshare = conf / lds if conf is not None and lds else None
        ratio = (va - mf) / mf if va is not None and mf else None
        trans = tr / (va - mf) if tr is not None and va is not None and mf is not None and va > mf else None
        fmt = lambda v, spec: "n/a" if v is None else format(v, spec)
        lines.append(f"{lab:<20} {fmt(util, '12.1f')} {fmt(ratio, '10.2f')} {fmt(trans, '12.3f')} {fmt(cshare, '13.3f')}")
    return "\n".join(lines)


def summarize(trace: str, layers: int = 4, fetch: Optional[str] = None,
              write: Optional[str] = None, calib_bytes: float = 268435456.0) -> str:
    rows = list(csv.DictReader(open(trace)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    groups = _forwards(rows, layers)
    lines = []
    for (grid, _), fwds in sorted(groups.items()):
        per: Dict[str, List[float]] = collections.defaultdict(list)
        totals = []
        for f in fwds:
            totals.append(sum(_dur_us(r) for _, r in f))
            for lab, r in f:
                per[lab].append(_dur_us(r))
        names = {lab: r["Kernel_Name"] for lab, r in fwds[-1]}
        grids = {lab: _grid(r) // _wg(r) for lab, r in fwds[-1]}
        lines.append(f"forward group: first LayerNorm grid {grid} threads, {len(fwds)} forwards, "
                     f"kernel time per forward {sorted(totals)[len(totals) // 2]:.1f} us (median)")
        lines.append(f"{'label':<20} {'launches/fwd':>12} {'avg us':>9} {'us/fwd':>9} {'WGs':>6}  kernel")
        for lab in dict.fromkeys(lab for lab, _ in fwds[-1]):
            v = per[lab]
            n = len(v) // len(fwds)
            lines.append(f"{lab:<20} {n:>12} {sum(v) / len(v):>9.2f} {sum(v) / len(fwds):>9.1f} "
                         f"{grids[lab]:>6}  {names[lab][:90]}")
        lines.append("")
    if fetch and write:
        lines.append(f"HBM traffic per launch (FETCH_SIZE / WRITE_SIZE, calibrated on the "
                     f"{calib_bytes / 2**20:.0f} MiB copy)")
        scaled = {}
        for tag, path in (("fetch", fetch), ("write", write)):
            crow, copy_kib = _counter(path)
            if not copy_kib:
                lines.append(f"  no calibration copy in {path}")
                return "\n".join(lines)
            factor = calib_bytes / (copy_kib * 1024.0)
            lines.append(f"  {tag}: calibration copy reads {copy_kib:.0f} KiB -> scale x{factor:.3f}")
            gemm_kib = _calib_gemm_kib(crow)
            if gemm_kib:
                want = CALIB_GEMM_FETCH if tag == "fetch" else CALIB_GEMM_WRITE
                got = gemm_kib * 1024.0 * factor
                lines.append(f"  {tag}: calibration GEMM reads {gemm_kib:.0f} KiB x{factor:.3f} = "
                             f"{got / 2**20:.1f} MiB against {want / 2**20:.1f} MiB known ({got / want:.3f})")
            gr = _forwards(crow, layers)
            grid = _timed(gr) if gr else None
            acc: Dict[str, List[float]] = collections.defaultdict(list)
            for f in gr.get(grid, []):
                for lab, r in f:
                    acc[lab].append(float(r["Counter_Value"]) * 1024.0 * factor)
            scaled[tag] = {lab: sum(v) / len(v) for lab, v in acc.items()}
        lines.append(f"{'label':<20} {'fetch MB':>9} {'write MB':>9} {'total MB':>9}")
        seen = list(dict.fromkeys(_labels(layers) + _labels(layers, fused=True)))
        for lab in [x for x in seen if x in scaled["fetch"] or x in scaled["write"]]:
            fb, wb = scaled["fetch"].get(lab, 0.0), scaled["write"].get(lab, 0.0)
            lines.append(f"{lab:<20} {fb / 1e6:>9.1f} {wb / 1e6:>9.1f} {(fb + wb) / 1e6:>9.1f}")
        for lab in [x for x in seen if x in scaled["fetch"] or x in scaled["write"]]:
            fb, wb = scaled["fetch"].get(lab, 0.0), scaled["write"].get(lab, 0.0)
            lines.append(f"traffic_bytes_per_launch[{lab}] {fb + wb:.0f}")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--copy-calib-bytes", type=float, default=268435456.0)
    ap.add_argument("--pmc", nargs="*", default=[])
    ap.add_argument("--cus", type=int, default=256)
    ap.add_argument("--xcds", type=int, default=8)
    args = ap.parse_args()
    print(summarize(args.trace, args.layers, args.fetch, args.write, args.copy_calib_bytes))
    if args.pmc:
        print()
        print(pmc_table(args.pmc, args.layers, args.cus, args.xcds))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
