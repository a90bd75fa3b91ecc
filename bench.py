"""Headline benchmark: the 4-layer fused forward at C4 on one MI355X.

    python bench.py [--gpus 1] [--steps 300] [--warmup 20] [--workload C4]

Prints ONE JSON line.  A "step" is one forward of the drop-in hook
(``UserOptimizedTransformer``) over the workload's synthetic batch, inputs
already resident in HBM; each step is bracketed by HIP events on torch's
current stream (the harness's method, torch_transformer_benchmark.py:
491-504) and ``value`` is the median step latency in ms.  Prefix-padded tokens are not computed
(the engine packs the valid tokens), so TFLOP/s and % of the dense bf16
MFMA peak use the FLOPs of the work executed -- the valid tokens' GEMM rows
and causal attention pairs; the full-padded-S figure is reported beside it
as an equivalent rate, with the eager packed / unpacked latencies.

Also reported:
* ``roofline``: the dominant kernel (largest share of one eager forward,
  measured per launch with HIP events on the stream it runs on), its
  algorithmic FLOPs per launch over its average launch time, against the
  MI355X dense peak; ``traffic`` from the committed rocprofv3 FETCH_SIZE /
  WRITE_SIZE summary when present;
* ``breakdown``: per-kernel-class kernel time of one eager forward: every
  launch of the forward replayed on its own, back to back behind a spin
  kernel, HIP events on the launch stream (so no inter-launch gap or host
  launch cost enters), summed over the class's launches;
* ``cpu_baseline``: the CPU oracle (fp32 restatement of the reference
  forward) timed on the host's cores on a bounded sample (one sequence:
  one warmup run, then the median of three, scaled to a whole forward);
* ``accuracy``: every sequence of the GPU output against the CPU oracle,
  with the worst per-element budget use |d| / max(atol, rtol |ref|);
* ``wait_timeouts``: the scheduled attention's error word after the timed
  steps (timed-out split waits or invalid work items; 0 expected).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "tiktok-techjam-2026_amd")]

PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}
HBM_GBPS = 8000.0


def _percentile(vals, q):
    s = sorted(vals)
    pos = (len(s) - 1) * q
    lo, hi = int(pos), min(int(pos) + 1, len(s) - 1)
    return s[lo] * (1 - (pos - lo)) + s[hi] * (pos - lo)


def _time_steps(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return [s.elapsed_time(e) for s, e in zip(starts, ends)], wall


def _attn_flops(qkv, causal, cu_seqlens=None):
    """Algorithmic attention FLOPs of one launch: 2*hd per (query, key) pair
    for QK^T and again for PV, over the pairs it computes (causal: j <= i)."""
    if cu_seqlens is not None:
        h, hd = qkv.shape[2], qkv.shape[3]
        lens = (cu_seqlens[1:] - cu_seqlens[:-1]).tolist()
    else:
        b, s, _, h, hd = qkv.shape
        lens = [s] * b
    pairs = sum(n * (n + 1) // 2 if causal else n * n for n in lens)
    return 4.0 * h * hd * pairs


# The traffic-calibration GEMM (see _breakdown): M x N x K bf16, tile plan 9
# (64 x 64, direct-to-LDS).  tjkernels.rocprof_summary finds it by its grid.
GEMM_CALIB_M, GEMM_CALIB_N, GEMM_CALIB_K, GEMM_CALIB_PLAN = 64, 65536, 1024, 9


def _breakdown(engine, x, mask):
    """Per-kernel-class kernel time of one eager forward.  The forward runs
    once with every tjk launch recorded (its exact call); each recorded call
    is then replayed on its own, back to back behind a spin kernel
    (``_kernel_avg_ms``), and its average launch time is summed into its
    class.  Events bracketing the launches inside the forward would also
    count the gaps between launches.  Also returns, per class, the call of
    its last launch."""
    import torch
    from tjkernels import ops
    classes, calls = {}, {}
    orig = {name: getattr(ops, name) for name in ("gemm", "gemm_residual_from", "flash_attention",
                                                  "flash_attention_sched", "add_layernorm", "ffn")}
    events = []

    def wrap(name, fn):
        def inner(*a, **k):
            label = name
            if name == "gemm":
                a0, w = a[0], a[1]
                epi = a[4] if len(a) > 4 else k.get("epilogue", 0)
                d = engine.d_model
                if epi == 1:
                    label = "gemm_ffn1_gelu"
                elif w.shape[0] == 3 * d:
                    label = "gemm_qkv"
                else:
                    label = ("gemm_out" if w.shape[1] == d else "gemm_ffn2") + ("_residual" if epi == 2 else "")
                flops = 2.0 * a0.shape[0] * w.shape[0] * w.shape[1]
            elif name == "gemm_residual_from":  # the first layer's out-proj, adding the input rows
                label = "gemm_out_residual"
                flops = 2.0 * a[0].shape[0] * a[1].shape[0] * a[1].shape[1]
            elif name == "flash_attention":
                flops = _attn_flops(a[0], k.get("causal", True), k.get("cu_seqlens"))
            elif name == "flash_attention_sched":
                label = "flash_attention"
                flops = _attn_flops(a[0], k.get("causal", True), a[2])
            elif name == "ffn":
                label = "ffn_fused"
                flops = 4.0 * a[0].shape[0] * a[1].shape[0] * a[1].shape[1]
            else:
                flops = 0.0
            r = fn(*a, **k)
            events.append((label, flops, (fn, a, k)))
            calls[label] = (fn, a, k)
            return r
        return inner

    mode, lens = engine._mask_info(mask)
    packing = engine._packing(lens, x.shape[1]) if lens is not None else None
    for name, fn in orig.items():
        setattr(ops, name, wrap(name, fn))
    try:
        for _ in range(2):  # warm, then keep the last pass
            events.clear()
            engine._forward_impl(x, mask, mode, packing)
        torch.cuda.synchronize()
    finally:
        for name, fn in orig.items():
            setattr(ops, name, fn)
    # Replays write the forward's workspaces again (a residual epilogue adds
    # into the residual once more per replay); the forward's output was read
    # before, and every later forward recomputes them from x.
    timed = [(label, flops, _kernel_avg_ms(call, reps=20)) for label, flops, call in events]
    # A plain copy of known size (256 MiB read + 256 MiB written): its rocprof
    # FETCH_SIZE / WRITE_SIZE readings calibrate the HBM-traffic counters.
    src = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device=x.device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    # A GEMM of known traffic checks that scale on the GEMMs' own access
    # pattern (LDS DMA of 128-byte row pieces): 64 rows against a 128 MiB
    # weight (65536 x 1024 bf16) that each 64-column tile reads once, so the
    # fetch is the weight plus one copy of the 128 KiB A (and its bias) per XCD.
    ga = torch.randn(GEMM_CALIB_M, GEMM_CALIB_K, device=x.device).to(torch.bfloat16)
    gw = torch.randn(GEMM_CALIB_N, GEMM_CALIB_K, device=x.device).to(torch.bfloat16)
    gb = torch.zeros(GEMM_CALIB_N, dtype=torch.bfloat16, device=x.device)
    gc = torch.empty(GEMM_CALIB_M, GEMM_CALIB_N, dtype=torch.bfloat16, device=x.device)
    torch.cuda.synchronize()
    ops.gemm(ga, gw, gb, gc, ops.EPI_BIAS, GEMM_CALIB_PLAN)
    torch.cuda.synchronize()
    del ga, gw, gb, gc
    for label, flops, ms in timed:
        c = classes.setdefault(label, {"ms": 0.0, "launches": 0, "flops": 0.0})
        c["ms"] += ms
        c["launches"] += 1
        c["flops"] += flops
    return classes, calls


def _kernel_avg_ms(call, reps=50):
    """Average duration of one launch of a kernel class: its recorded call
    replayed `reps` times back to back (queued behind a spin kernel, so the
    host's launch rate does not enter), HIP events on the launch stream."""
    import torch
    from tjkernels import timing
    fn, a, k = call
    for _ in range(5):
        fn(*a, **k)
    torch.cuda.synchronize()
    return timing.launch_ms(lambda: fn(*a, **k), reps)


def _traffic(label):
    """HBM bytes per launch of `label` from the committed rocprofv3 PMC summary."""
    path = ROOT / "profiles" / "traffic_c4.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 2 and parts[0] == f"traffic_bytes_per_launch[{label}]":
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


def _cpu_baseline(w, sd, x, mask, got):
    """Time the CPU oracle on one sequence (a bounded sample: one warmup run,
    then the median of three), scale it to the whole forward, and check
    every sequence of the GPU output against the oracle."""
    import torch
    from oracle import model as oracle
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    refs = [oracle.forward(sd, x[b:b + 1], mask[b:b + 1], w.heads, w.causal, torch.float32)
            for b in range(w.batch)]  # also the warmup of the timed runs
    samples = []
    for _ in range(3):
        t0 = time.perf_counter_ns()
        oracle.forward(sd, x[:1], mask[:1], w.heads, w.causal, torch.float32)
        samples.append((time.perf_counter_ns() - t0) / 1e6)
    per_forward = statistics.median(samples) * w.batch
    tol = 1e-4 if w.dtype == torch.float32 else 2e-2
    ref = torch.cat(refs)
    acc = oracle.compare_outputs(ref, got, rtol=tol, atol=tol)
    err = (got.double() - ref.double()).abs()
    acc["budget_used"] = float((err / ref.double().abs().mul(tol).clamp_min(tol)).max())
    acc["padded_rows_zero"] = bool((got[~mask] == 0).all())
    return ({"value": round(per_forward, 3), "unit": "ms", "cores": cores, "kind": "port",
             "sample": f"fp32 CPU oracle (oracle/model.py) on 1 of {w.batch} sequences, one warmup run, "
                       f"median of 3 runs, scaled x{w.batch} to one forward"},
            {"vs": f"CPU oracle fp32, all {w.batch} sequences", "tolerance": tol, **acc})


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="C4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-breakdown", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "sequences are independent, so N GPUs would each run this benchmark on B/N "
              "sequences with no communication.", file=sys.stderr)
        return 2

    import torch
    from tjkernels import UserOptimizedTransformer
    from tjkernels.workloads import (WORKLOADS, flops_per_forward, flops_valid_tokens, make_inputs,
                                     make_state_dict)

    w = WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    sd = make_state_dict(w, seed=0)
    model = UserOptimizedTransformer(w.config)
    model.load_state_dict(sd, strict=True)
    model = model.to(device=dev, dtype=w.dtype).eval()
    x, mask, lengths = make_inputs(w, seed=100001)
    xd, md = x.to(device=dev, dtype=w.dtype), mask.to(dev)

    with torch.inference_mode():
        samples, wall = _time_steps(lambda: model(xd, md), args.steps, args.warmup)
        got = model(xd, md).cpu()
        engine = model._tj_engine
        plan = engine.plan
        from tjkernels import schedule as sched_mod
        scheds = [pk.attn for pk in engine._packings.values() if pk.attn is not None]
        wait_timeouts = sum(sched_mod.error_count(sc) for sc in scheds)
        breakdown, calls = ({}, {}) if args.no_breakdown else _breakdown(engine, xd, md)
        # The same forward with every padded row computed (per-key mask
        # attention, the reference's way), eager, for the packing gain.
        from tjkernels.engine import MASK_GENERAL
        # (at most 20 forwards each; fewer when the run itself is short)
        n_eager, w_eager = max(1, min(20, args.steps)), min(3, args.warmup)
        eager_unpacked = statistics.median(_time_steps(
            lambda: engine._forward_impl(xd, md, MASK_GENERAL), n_eager, w_eager)[0])
        mode, lens = engine._mask_info(md)
        pk = engine._packing(lens, w.seq) if lens is not None else None
        eager_packed = statistics.median(_time_steps(
            lambda: engine._forward_impl(xd, md, mode, pk), n_eager, w_eager)[0])

    from tjkernels import tiles
    flops = flops_per_forward(w)
    flops_valid = flops_valid_tokens(w, lengths.tolist())
    med = statistics.median(samples)
    dtype_name = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[plan.compute_dtype]
    peak = PEAK_TFLOPS[dtype_name]
    tflops = flops_valid / (med * 1e-3) / 1e12

    roofline = None
    if breakdown:
        dom = max((k for k in breakdown if breakdown[k]["flops"] > 0), key=lambda k: breakdown[k]["ms"])
        one_ms = breakdown[dom]["ms"] / breakdown[dom]["launches"]
        with torch.inference_mode():  # about 0.2 s of replays, 3 to 50 launches
            avg_ms = _kernel_avg_ms(calls[dom], reps=max(3, min(50, int(200.0 / max(one_ms, 1e-3)))))
        per_launch = breakdown[dom]["flops"] / breakdown[dom]["launches"]
        achieved = per_launch / (avg_ms * 1e-3) / 1e12
        roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                    "flops_per_launch": per_launch, "avg_launch_ms": round(avg_ms, 5),
                    # the committed PMC summary covers the C4 workload only
                    "traffic": _traffic(dom) if args.workload == "C4" else None}
        for k, v in breakdown.items():
            v["ms"] = round(v["ms"], 4)
            if v["flops"]:
                v["tflops"] = round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 1)

    cpu, acc = (None, None)
    if not args.no_cpu_baseline and w.seq > 16384:
        # the oracle materializes [H, S, S] scores: 640 GB at S = 100000
        print(f"bench.py: no CPU baseline for S={w.seq} (the CPU oracle holds S x S scores)", file=sys.stderr)
    elif not args.no_cpu_baseline:
        cpu, acc = _cpu_baseline(w, sd, x, mask, got)

    line = {
        "metric": "4-layer fused fwd latency (ms) + % bf16 MFMA peak, d=1024 S=2048, 1 GPU",
        "value": round(med, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(med, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype_name, "data": "synthetic",
        "config": {"workload": w.describe(), "tokens": w.tokens, "plan": plan.label,
                   "hipgraph": plan.cuda_graph, "residual_epilogue": plan.residual_epilogue},
        "p90_ms": round(_percentile(samples, 0.9), 4), "min_ms": round(min(samples), 4),
        "wall_s": round(wall, 3),
        # MFMA rate on the work actually executed: valid-token FLOPs (padded
        # rows are not computed; see "packing").
        "tflops": round(tflops, 1), "pct_peak": round(100 * tflops / peak, 2),
        "gflop_executed": round(flops_valid / 1e9, 2),
        # The full-padded-S formula (every padded row counted, as if computed):
        # an equivalent rate, not an MFMA utilisation.
        "gflop_per_forward_padded": round(flops / 1e9, 2),
        "tflops_padded_equiv": round(flops / (med * 1e-3) / 1e12, 1),
        "packing": {"lengths": lengths.tolist(), "valid_token_frac": round(sum(lengths.tolist()) / w.tokens, 4),
                    "eager_packed_ms": round(eager_packed, 4),
                    "eager_unpacked_ms": round(eager_unpacked, 4)},
        "roofline": roofline, "cpu_baseline": cpu, "accuracy": acc, "breakdown": breakdown,
        "wait_timeouts": wait_timeouts,
        "ffn": plan.ffn,
        # measured tile plan per projection shape (M bucket x N x K, epilogue)
        "gemm_tiles": tiles.describe(),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
