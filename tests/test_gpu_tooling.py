"""The accuracy-gated autotuner and the sweep, run on the GPU.

The autotuner mirrors the reference's bench/autotune.py:61-246: a plan is
admitted only if no element uses more than ``margin`` of its budget
max(atol, rtol |ref|) on the trial and held-out seeds; an inadmissible
heuristic escalates to fp32 compute (:203-217); a knob change is kept only
when it stays admissible and is at least 2% faster.  The sweep runs
``bench.py`` per workload in its own process (bench/run_all.py:41-112).
"""

from pathlib import Path

import pytest
import torch

from tjkernels import autotune, plans as plans_mod, sweep
from tjkernels.workloads import WORKLOADS

pytestmark = pytest.mark.gpu


def _select(w, tmp_table, monkeypatch):
    monkeypatch.setattr(plans_mod, "TUNED", plans_mod.PlanTable(tmp_table))
    return plans_mod.select_plan(w.batch, w.seq, w.d_model, w.heads, w.ffn_dim, w.layers, w.causal, w.dtype,
                                 torch.device("cuda", 0))


def test_autotune_admits_records_and_selects_a_plan(device, tmp_path, monkeypatch):
    w = WORKLOADS["C2"]
    out = autotune.tune_workload(w, trials=1, margin=0.85, iters=5, verbose=False)
    assert out is not None
    key, plan, res = out
    assert res["usage"] <= 0.85 and res["latency_ms"] > 0
    assert plan.compute_dtype == torch.float16 and plan.label == "autotuned"
    plan.validate()
    table = tmp_path / "plans.json"
    plans_mod.save_plans({key: plan}, table)
    assert _select(w, table, monkeypatch) == plan


def test_autotune_escalates_to_fp32_when_the_gate_rejects_fp16(device, tmp_path, monkeypatch):
    """A margin no fp16 plan can meet (1% of the budget: fp16 rounding alone
    uses more) but the fp32 plan can: the tuner escalates, records an fp32
    plan, and select_plan then picks it."""
    w = WORKLOADS["C2"]
    out = autotune.tune_workload(w, trials=1, margin=0.01, iters=5, verbose=False)
    assert out is not None, "the fp32 escalation was not admitted"
    key, plan, res = out
    assert plan.compute_dtype == torch.float32 and plan.label == "autotuned-fp32"
    assert res["usage"] <= 0.01
    table = tmp_path / "plans.json"
    plans_mod.save_plans({key: plan}, table)
    chosen = _select(w, table, monkeypatch)
    assert chosen.compute_dtype == torch.float32 and chosen == plan


def test_sweep_runs_bench_in_a_subprocess(device, tmp_path):
    """sweep.run_case on the real bench.py: PASS, with the dominant kernel's
    roofline and the CPU baseline in the record; the report names the GPU."""
    r = sweep.run_case("C1", 20, 5, True, {}, 600)
    assert r["status"] == "PASS", r.get("error_tail")
    res = r["result"]
    assert res["roofline"] and res["roofline"]["frac"] > 0
    assert res["cpu_baseline"] and res["cpu_baseline"]["cores"] >= 1
    assert res["accuracy"]["passed"] and res["accuracy"]["padded_rows_zero"]
    info = sweep.system_info()
    assert "gfx" in str(info.get("arch", "")), info
    assert "System:" in sweep.system_header(info)
    assert "| C1 | PASS |" in sweep.sweep_table([r])
