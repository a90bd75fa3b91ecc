"""Sweep and ablation over the named workloads, with a markdown report.

    python -m tjkernels.sweep [--workloads C1,C2,C3,C4,C5] [--steps 100]
                              [--warmup 10] [--cpu] [--ablation C3,C4]
                              [--out DIR] [--tag main]

Counterpart of the reference's bench/run_all.py:41-217 (one subprocess per
case so an out-of-memory error or a crash cannot poison the rest of the
sweep, JSON + markdown table per run, OOM tagging) and bench/ablation.py:
30-130 (leave-one-out through the TJ_* environment knobs, with the tuned
plan table switched off so the knob is not overridden).  Each case runs
this repository's ``bench.py --workload NAME`` and keeps its JSON line:
latency, executed TFLOP/s and % of the dense peak, the padded-S equivalent
rate, the roofline of the dominant kernel, the accuracy check against the
CPU oracle and the CPU baseline (with ``--cpu``).

Ablation variants (each against the full stack on the same workloads):
  * without hipGraph capture             TJ_NO_GRAPH=1
  * deferred residual (reference scheme) TJ_DEFERRED_RESIDUAL=1
  * residual added in the GEMM epilogues  TJ_DEFERRED_RESIDUAL=0
  * library tile rule, no measured tiles TJ_GEMM_TUNE=0
  * padded rows computed (no packing)    TJ_NO_PACK=1
  * plain attention kernel (plan 1)      TJ_ATTN_PLAN=1
  * two-launch FFN (no single-launch)    TJ_FFN=gemm
  * fp32 compute (accuracy escalation)   TJ_COMPUTE_DTYPE=float32
  * one-launch attention block (opt-in)  TJ_ATTN_BLOCK=1
  * LayerNorm inside the GEMMs (opt-in)  TJ_LN_GEMM=1
  * fp16 residual stream (opt-in)        TJ_RESIDUAL_DTYPE=float16

The report opens with the system it ran on (GPU, its architecture and CU
count, ROCm / torch versions, host CPU and the cores the CPU baseline may
use), as the reference's report header does (bench/make_report.py:34-95).
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path
from typing import Dict, List, Optional

REPO = Path(__file__).resolve().parents[2]
BENCH = REPO / "bench.py"

LEAVE_ONE = [
    ("full stack (heuristic plan)", {}),
    ("without hipGraph capture", {"TJ_NO_GRAPH": "1"}),
    ("deferred residual", {"TJ_DEFERRED_RESIDUAL": "1"}),
    ("residual in the GEMM epilogues", {"TJ_DEFERRED_RESIDUAL": "0"}),
    ("library tile rule", {"TJ_GEMM_TUNE": "0"}),
    ("padded rows computed", {"TJ_NO_PACK": "1"}),
    ("plain attention kernel", {"TJ_ATTN_PLAN": "1"}),
    ("two-launch FFN", {"TJ_FFN": "gemm"}),
    ("fp32 compute", {"TJ_COMPUTE_DTYPE": "float32"}),
    ("one-launch attention block", {"TJ_ATTN_BLOCK": "1"}),
    ("LayerNorm inside the GEMMs", {"TJ_LN_GEMM": "1"}),
    ("fp16 residual stream", {"TJ_RESIDUAL_DTYPE": "float16"}),
]


_SYSTEM_PROBE = r"""
import json, os, platform, torch
info = {"torch": torch.__version__, "hip": getattr(torch.version, "hip", None),
        "host_cores": len(os.sched_getaffinity(0)), "host": platform.node()}
try:
    with open("/proc/cpuinfo") as f:
        info["cpu"] = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), None)
    with open("/proc/meminfo") as f:
        info["host_mem_gib"] = round(int(f.readline().split()[1]) / 2**20, 1)
except OSError:
    pass
if torch.cuda.is_available():
    p = torch.cuda.get_device_properties(0)
    info.update(gpu=p.name, arch=p.gcnArchName, cus=p.multi_processor_count,
                vram_gib=round(p.total_memory / 2**30, 1), gpus_visible=torch.cuda.device_count())
print(json.dumps(info))
"""


def system_info(timeout: float = 120.0) -> Dict[str, object]:
    """GPU and host facts, read in a child process (the caller never touches
    the GPU itself)."""
    try:
        proc = subprocess.run([sys.executable, "-c", _SYSTEM_PROBE], capture_output=True, text=True,
                              timeout=timeout, cwd=str(REPO))
        line = [ln for ln in proc.stdout.splitlines() if ln.startswith("{")]
        return json.loads(line[-1]) if line else {"error": proc.stderr.strip()[-200:]}
    except (subprocess.TimeoutExpired, ValueError) as exc:
        return {"error": str(exc)[:200]}


def system_header(info: Dict[str, object]) -> str:
    if "error" in info:
        return f"System: unknown ({info['error']})\n"
    gpu = (f"{info.get('gpu', 'no GPU')} ({info.get('arch', '?')}, {info.get('cus', '?')} CUs, "
           f"{info.get('vram_gib', '?')} GiB)")
    return (f"System: {gpu}; ROCm/HIP {info.get('hip')}, torch {info.get('torch')}; host "
            f"{info.get('cpu', '?')}, {info.get('host_cores', '?')} cores usable, {info.get('host_mem_gib', '?')} GiB\n")


def run_case(workload: str, steps: int, warmup: int, cpu: bool, env: Dict[str, str],
             timeout: float) -> Dict[str, object]:
    """One ``bench.py`` run in its own process; its JSON line plus status."""
    cmd = [sys.executable, str(BENCH), "--workload", workload, "--steps", str(steps),
           "--warmup", str(warmup)]
    if not cpu:
        cmd.append("--no-cpu-baseline")
    full_env = dict(os.environ)
    full_env.update(env)
    t0 = time.time()
    record: Dict[str, object] = {"workload": workload, "env": env, "cmd": " ".join(cmd[1:])}
    try:
        proc = subprocess.run(cmd, capture_output=True, text=True, env=full_env, cwd=str(REPO),
                              timeout=timeout)
        out, rc = proc.stdout + proc.stderr, proc.returncode
    except subprocess.TimeoutExpired as exc:
        out, rc = (exc.stdout or "") if isinstance(exc.stdout, str) else "", -1
        record["status"] = "TIMEOUT"
    record["returncode"] = rc
    record["wall_s"] = round(time.time() - t0, 1)
    line = None
    for ln in reversed(out.splitlines()):
        if ln.startswith("{") and '"metric"' in ln:
            line = ln
            break
    if line is not None:
        record["result"] = json.loads(line)
        acc = record["result"].get("accuracy") or {}
        record.setdefault("status", "PASS" if acc.get("passed", True) else "FAIL")
    else:
        tail = [ln for ln in out.strip().splitlines() if ln.strip()][-6:]
        record["error_tail"] = "\n".join(tail)
        record.setdefault("status", "OOM" if "out of memory" in out.lower() else "ERROR")
    return record


def _fmt(v: Optional[float], spec: str) -> str:
    return "n/a" if v is None else format(v, spec)


def sweep_table(records: List[Dict[str, object]]) -> str:
    lines = ["| workload | status | latency ms (p90) | executed TFLOP/s | % peak | padded-equiv TFLOP/s | "
             "dominant kernel: achieved / frac | max abs err | CPU baseline ms (cores) |",
             "|---|---|---:|---:|---:|---:|---|---:|---:|"]
    for r in records:
        res = r.get("result") or {}
        rf = res.get("roofline") or {}
        acc = res.get("accuracy") or {}
        cpu = res.get("cpu_baseline") or {}
        lines.append(
            f"| {r['workload']} | {r['status']} | {_fmt(res.get('value'), '.4f')} "
            f"({_fmt(res.get('p90_ms'), '.4f')}) | {_fmt(res.get('tflops'), '.1f')} | "
            f"{_fmt(res.get('pct_peak'), '.2f')} | {_fmt(res.get('tflops_padded_equiv'), '.1f')} | "
            f"{rf.get('kernel', 'n/a')}: {_fmt(rf.get('achieved'), '.1f')} / {_fmt(rf.get('frac'), '.3f')} | "
            f"{_fmt(acc.get('max_abs'), '.2e')} | "
            f"{_fmt(cpu.get('value'), '.1f')} ({cpu.get('cores', 'n/a')}) |")
    return "\n".join(lines)


def ablation_table(rows: List[Dict[str, object]], workloads: List[str]) -> str:
    variants: List[str] = []
    for r in rows:
        if r["variant"] not in variants:
            variants.append(r["variant"])
    base = {r["workload"]: (r.get("result") or {}).get("value") for r in rows if r["variant"] == variants[0]}
    lines = ["| variant | " + " | ".join(f"{w} ms (x full)" for w in workloads) + " |",
             "|---|" + "---:|" * len(workloads)]
    for v in variants:
        cells = []
        for w in workloads:
            m = [r for r in rows if r["variant"] == v and r["workload"] == w]
            ms = (m[0].get("result") or {}).get("value") if m else None
            if ms is None:
                cells.append(m[0]["status"] if m else "n/a")
            else:
                rel = f" ({ms / base[w]:.2f}x)" if base.get(w) else ""
                cells.append(f"{ms:.4f}{rel}")
        lines.append(f"| {v} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--workloads", default="C1,C2,C3,C4,C5")
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu", action="store_true", help="also time the CPU baseline (slow for C4/C5)")
    ap.add_argument("--ablation", default="", help="workloads for the leave-one-out ablation")
    ap.add_argument("--timeout", type=float, default=900.0, help="seconds per case")
    ap.add_argument("--out", default=str(REPO / "sweep_out"))
    ap.add_argument("--tag", default="main")
    args = ap.parse_args(argv)
    out = Path(args.out)
    out.mkdir(parents=True, exist_ok=True)

    info = system_info()
    records = []
    for w in [s for s in args.workloads.split(",") if s]:
        print(f"--- {w}", flush=True)
        r = run_case(w, args.steps, args.warmup, args.cpu, {}, args.timeout)
        res = r.get("result") or {}
        print(f"    {r['status']}  {res.get('value', 'n/a')} ms  ({r['wall_s']} s)", flush=True)
        if "error_tail" in r:
            print("    " + str(r["error_tail"]).replace("\n", "\n    "), flush=True)
        records.append(r)
    text = f"## Sweep ({args.tag})\n\n" + system_header(info) + "\n" + sweep_table(records) + "\n"

    abl_rows: List[Dict[str, object]] = []
    abl = [s for s in args.ablation.split(",") if s]
    if abl:
        print("=== leave-one-out ===", flush=True)
        for label, env in LEAVE_ONE:
            env = dict(env, TJ_IGNORE_PLANS="1")  # the tuned table would override the knob
            for w in abl:
                r = run_case(w, args.steps, args.warmup, False, env, args.timeout)
                r["variant"] = label
                abl_rows.append(r)
                res = r.get("result") or {}
                print(f"  {label:<32} {w}  {r['status']:<6} {res.get('value', 'n/a')} ms", flush=True)
        text += "\n## Leave-one-out ablation (heuristic plan, one knob changed)\n\n"
        text += ablation_table(abl_rows, abl) + "\n"

    stamp = time.strftime("%Y%m%d-%H%M%S")
    (out / f"{args.tag}-{stamp}.json").write_text(json.dumps({"tag": args.tag, "system": info, "records": records,
                                                              "ablation": abl_rows}, indent=2))
    (out / f"{args.tag}-{stamp}.md").write_text(text)
    print("\n" + text, flush=True)
    return 0 if all(r["status"] == "PASS" for r in records + abl_rows) else 1


if __name__ == "__main__":
    raise SystemExit(main())
