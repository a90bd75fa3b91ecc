"""Accuracy-gated autotuner: writes tuned plans into ``plans.json``.

    python -m tjkernels.autotune --workloads C2,C3,C4,C5 [--margin 0.85] [--dry-run]

Mirrors the reference's tuner (bench/autotune.py:61-246): it searches for
the fastest plan whose outputs stay inside a tightened version of the
accuracy budget, and records it per shape key.  A plan is admitted only
if, over the trial seeds and two held-out seeds (777, 4242), no element uses
more than ``margin`` of its own budget ``max(atol, rtol*|ref|)``
(bench/autotune.py:61-68); if the heuristic plan is inadmissible the tuner
escalates to fp32 compute (:203-217); a knob change is kept only if the plan
stays admissible and gets at least 2% faster (:229-234).

MI355X specifics:

* the accuracy reference is what the caller passes: the outputs of an
  independent implementation of the baseline model on the gate's seeds
  (``gate_seeds``), as the reference gates against its baseline model
  (bench/autotune.py:120-131); the GPU tests pass the CPU oracle's.  A
  caller that passes none (the command line) gets this build's own IEEE fp32
  plan on the same inputs, which the tests pin to the oracle at 1e-4 -- far
  inside the 2e-2 budgets, but an error common to every plan (packing,
  layout, masking) is then invisible to the gate;
* GEMM tile plans are not part of the tuned table: the engine times the tile
  candidates once per projection shape at run time (``tjkernels.tiles``),
  because with packed prefix-masked tokens the row count M of every
  projection follows the input lengths; ``tune_gemm`` remains as a tool;
  the plan-level knobs (attention plan, residual epilogue, hipGraph, residual dtype) are
  tuned by coordinate descent on whole-forward latency measured as the
  harness does (events on the current stream around the module call).
"""

from __future__ import annotations

import argparse
import statistics
from dataclasses import replace
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import ops
from .modules import UserOptimizedTransformer
from .plans import (Plan, attn_block_ok, default_plan, device_arch, fused_ffn_ok, save_plans, set_override,
                    shape_key)
from .workloads import WORKLOADS, Workload, make_inputs, make_state_dict

HELD_OUT_SEEDS = [777, 4242]


def gate_seeds(trials: int) -> List[int]:
    """Input seeds of the accuracy gate, in order: the trial seeds 1 ..
    ``trials`` and the held-out seeds (bench/autotune.py:120-131)."""
    return list(range(1, trials + 1)) + HELD_OUT_SEEDS


def budget(dtype: torch.dtype) -> Tuple[float, float]:
    """(atol, rtol) of the per-element budget for a model dtype."""
    return (1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2)


def budget_usage(ref: torch.Tensor, got: torch.Tensor, atol: float, rtol: float) -> float:
    err = (got.float() - ref.float()).abs_()
    bud = ref.float().abs().mul_(rtol).clamp_min_(atol)
    return float(err.div_(bud).max())


def _time_ms(fn, iters: int, warmup: int = 3) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        samples.append((e0, e1))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in samples)


def tune_gemm(m: int, n: int, k: int, dtype: torch.dtype, epilogue: int,
              iters: int = 20) -> Tuple[int, Dict[int, float]]:
    """Fastest valid tile plan for one projection shape; returns (plan, {plan: ms})."""
    dev = torch.device("cuda", torch.cuda.current_device())
    a = torch.randn(m, k, device=dev).to(dtype)
    w = (torch.randn(n, k, device=dev) * 0.02).to(dtype)
    b = torch.zeros(n, device=dev, dtype=dtype)
    out = torch.zeros(m, n, device=dev, dtype=torch.float32 if epilogue == ops.EPI_BIAS_RESIDUAL else dtype)
    times: Dict[int, float] = {}
    for pid, *_ in ops.gemm_plans(dtype):
        try:
            ops.gemm(a, w, b, out, epilogue, pid)
        except ops.TjkError:
            continue  # plan does not take this K
        times[pid] = _time_ms(lambda: ops.gemm(a, w, b, out, epilogue, pid), iters)
    best = min(times, key=times.get)
    return best, times


class _Evaluator:
    """Runs candidate plans of one workload on the gate's inputs (weights
    from ``make_state_dict(w, seed=0)``, inputs from ``make_inputs`` at
    ``gate_seeds(trials)``) and measures their budget usage against
    ``references`` (one output per seed, in that order), or against this
    build's fp32 plan when none are given."""

    def __init__(self, w: Workload, trials: int, iters: int,
                 references: Optional[Sequence[torch.Tensor]] = None) -> None:
        self.w = w
        self.dev = torch.device("cuda", torch.cuda.current_device())
        self.sd = make_state_dict(w, seed=0)
        self.atol, self.rtol = budget(w.dtype)
        self.iters = iters
        seeds = gate_seeds(trials)
        self.inputs = []
        for s in seeds:
            x, mask, _ = make_inputs(w, seed=s)
            self.inputs.append((x.to(self.dev, w.dtype), mask.to(self.dev)))
        xb, mb, _ = make_inputs(w, seed=100001)
        self.bench_input = (xb.to(self.dev, w.dtype), mb.to(self.dev))
        if references is not None:
            if len(references) != len(seeds):
                raise ValueError(f"{len(references)} reference outputs for {len(seeds)} gate seeds")
            self.refs = [r.to(self.dev, torch.float32) for r in references]
        else:
            self.refs = [self._run(Plan(compute_dtype=torch.float32, cuda_graph=False,
                                        label="fp32-reference"), x, m)
                         for x, m in self.inputs]

    def _model(self) -> UserOptimizedTransformer:
        m = UserOptimizedTransformer(self.w.config)
        m.load_state_dict(self.sd, strict=True)
        return m.to(device=self.dev, dtype=self.w.dtype).eval()

    def _run(self, plan: Plan, x, mask) -> torch.Tensor:
        set_override(plan)
        try:
            with torch.inference_mode():
                return self._model()(x, mask)
        finally:
            set_override(None)

    def evaluate(self, plan: Plan) -> Dict[str, object]:
        set_override(plan)
        try:
            model = self._model()
            usage = 0.0
            with torch.inference_mode():
                for (x, m), ref in zip(self.inputs, self.refs):
                    got = model(x, m)
                    if not torch.isfinite(got).all():
                        return {"plan": plan, "admissible": False, "usage": float("inf")}
                    usage = max(usage, budget_usage(ref, got, self.atol, self.rtol))
                xb, mb = self.bench_input
                ms = _time_ms(lambda: model(xb, mb), self.iters)
        except (ops.TjkError, ValueError) as exc:
            return {"plan": plan, "admissible": False, "error": str(exc)[:160]}
        finally:
            set_override(None)
        return {"plan": plan, "latency_ms": ms, "usage": usage}


def tune_workload(w: Workload, trials: int = 2, margin: float = 0.85, iters: int = 30,
                  verbose: bool = True, references: Optional[Sequence[torch.Tensor]] = None,
                  log: Optional[List[Dict[str, object]]] = None) -> Optional[Tuple[str, Plan, Dict[str, object]]]:
    """The fastest admissible plan of workload ``w`` as (shape key, plan,
    its evaluation), or None when neither the heuristic plan nor its fp32
    escalation is admissible.  ``references``: the gate's reference outputs,
    one per ``gate_seeds(trials)`` seed (see the module docstring).
    ``log``, if given, receives every evaluation in order, tagged."""
    dev = torch.device("cuda", torch.cuda.current_device())
    base = replace(default_plan(w.batch, w.seq, w.d_model, w.heads, w.ffn_dim, w.layers,
                                w.causal, w.dtype, dev), label="autotuned")
    ev = _Evaluator(w, trials, iters, references)

    def admissible(r):
        return "latency_ms" in r and r["usage"] <= margin

    def show(tag, r):
        if log is not None:
            log.append(dict(r, tag=tag))
        if verbose:
            if "latency_ms" in r:
                flag = "ok " if admissible(r) else "REJ"
                print(f"    {tag:<28} {flag} {r['latency_ms']:8.3f} ms  budget={r['usage']:.0%}", flush=True)
            else:
                print(f"    {tag:<28} ERR {r.get('error', 'non-finite output')}", flush=True)

    cur = ev.evaluate(base)
    show("heuristic", cur)
    if not admissible(cur) and base.compute_dtype != torch.float32:
        # fp32 compute (IEEE fp32 MFMA, the reference's escalation with TF32
        # off, bench/autotune.py:203-217); the single-launch FFN only where
        # it has an fp32 kernel for the shape
        ffn = "fused" if base.ffn == "fused" and fused_ffn_ok(w.d_model, w.ffn_dim, torch.float32) else "gemm"
        esc = ev.evaluate(replace(base, compute_dtype=torch.float32, ffn=ffn, label="autotuned-fp32"))
        show("escalate-fp32", esc)
        if admissible(esc):
            cur = esc
    if not admissible(cur):
        return None

    # GEMM tile plans stay -1: the engine times the tile candidates once per
    # projection shape at run time (tjkernels.tiles), since with packed
    # prefix-masked tokens M follows the input lengths.

    # coordinate descent over the plan-level knobs
    attn_plans = [0, 1, 3] + ([4] if w.seq <= 128 else [])
    knobs = [("attn_plan", attn_plans), ("residual_epilogue", [True, False]), ("cuda_graph", [True, False])]
    if cur["plan"].compute_dtype != torch.float32:
        # an fp16 residual stream, the reference's candidate
        # (bench/autotune.py:88); not tried for fp32 compute, whose 1e-4
        # budget a 2-byte residual cannot hold
        knobs.append(("residual_dtype", [torch.float32, torch.float16]))
    if ops.gemm_ln_supported(w.d_model, cur["plan"].compute_dtype):
        # LayerNorms inside the QKV / FFN1 GEMMs (takes effect with the
        # two-launch FFN and residual epilogues)
        knobs.insert(0, ("ln_gemm", [False, True]))
    if fused_ffn_ok(w.d_model, w.ffn_dim, cur["plan"].compute_dtype):
        knobs.insert(0, ("ffn", ["gemm", "fused"]))
    if attn_block_ok(w.seq, w.d_model, w.heads, cur["plan"].compute_dtype):
        knobs.insert(0, ("attn_block", [True, False]))
    for knob, values in knobs:
        for v in values:
            if getattr(cur["plan"], knob) == v:
                continue
            probe = ev.evaluate(replace(cur["plan"], **{knob: v}))
            show(f"{knob}={v}", probe)
            if admissible(probe) and probe["latency_ms"] < cur["latency_ms"] * 0.98:
                cur = probe
    key = shape_key(w.batch, w.seq, w.d_model, w.heads, w.ffn_dim, w.layers, w.causal,
                    w.dtype, device_arch(dev))
    return key, cur["plan"], cur


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--workloads", default="C2,C3,C4,C5")
    ap.add_argument("--trials", type=int, default=2)
    ap.add_argument("--margin", type=float, default=0.85)
    ap.add_argument("--iters", type=int, default=30)
    ap.add_argument("--dry-run", action="store_true")
    ap.add_argument("--out", default=None, help="plans file to merge into (default: the package's plans.json)")
    args = ap.parse_args(argv)
    tuned: Dict[str, Plan] = {}
    for name in args.workloads.split(","):
        w = WORKLOADS[name]
        print(f"{w.describe()}", flush=True)
        out = tune_workload(w, args.trials, args.margin, args.iters)
        if out is None:
            print("    no admissible plan; heuristic left in place", flush=True)
            continue
        key, plan, res = out
        tuned[key] = plan
        print(f"    -> {res['latency_ms']:.3f} ms budget={res['usage']:.0%} {plan.to_json()}", flush=True)
    if tuned and not args.dry_run:
        from pathlib import Path
        save_plans(tuned, Path(args.out) if args.out else None)
        print(f"wrote {len(tuned)} plan(s) to {args.out or 'plans.json'}", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
