"""The accuracy-gated autotuner and the sweep, run on the GPU.

The autotuner mirrors the reference's bench/autotune.py:61-246: a plan is
admitted only if no element uses more than ``margin`` of its budget
max(atol, rtol |ref|) on the trial and held-out seeds, measured here
against the CPU oracle's outputs on those seeds (the reference measures
against its baseline model, :120-131); an inadmissible heuristic escalates
to fp32 compute (:203-217); a knob change is kept only when it stays
admissible and is at least 2% faster.  The sweep runs
``bench.py`` per workload in its own process (bench/run_all.py:41-112).
"""

from pathlib import Path

import pytest
import torch

from oracle import model as oracle
from tjkernels import autotune, ops as ops_mod, plans as plans_mod, sweep
from tjkernels.workloads import WORKLOADS, make_inputs, make_state_dict

pytestmark = pytest.mark.gpu


def _select(w, tmp_table, monkeypatch):
    monkeypatch.setattr(plans_mod, "TUNED", plans_mod.PlanTable(tmp_table))
    return plans_mod.select_plan(w.batch, w.seq, w.d_model, w.heads, w.ffn_dim, w.layers, w.causal, w.dtype,
                                 torch.device("cuda", 0))


def _oracle_refs(w, trials):
    """The CPU oracle's fp32 outputs on the gate's inputs, in gate_seeds
    order: the tuner's reference, independent of every plan it judges."""
    sd = make_state_dict(w, seed=0)
    refs = []
    for seed in autotune.gate_seeds(trials):
        x, mask, _ = make_inputs(w, seed=seed)
        refs.append(oracle.forward(sd, x, mask, w.heads, w.causal, torch.float32))
    return refs


def test_autotune_admits_records_and_selects_a_plan(device, tmp_path, monkeypatch):
    w = WORKLOADS["C2"]
    out = autotune.tune_workload(w, trials=1, margin=0.85, iters=5, verbose=False,
                                 references=_oracle_refs(w, 1))
    assert out is not None
    key, plan, res = out
    assert res["usage"] <= 0.85 and res["latency_ms"] > 0  # measured against the oracle
    assert plan.compute_dtype == torch.float16 and plan.label == "autotuned"
    plan.validate()
    table = tmp_path / "plans.json"
    plans_mod.save_plans({key: plan}, table)
    assert _select(w, table, monkeypatch) == plan


def test_autotune_escalates_to_fp32_when_the_gate_rejects_fp16(device, tmp_path, monkeypatch):
    """A margin of 3.3% of the budget, measured against the CPU oracle: the
    fp16 heuristic plan uses more (4.3% at C2 on the gate's seeds: fp16
    activations) and is rejected; the fp32 escalation uses less (2.4%: its
    output is still rounded to the model's fp16, which alone costs up to
    2^-11 |ref| against a budget of 2e-2 |ref|) and is admitted.  The tuner
    records the fp32 plan and select_plan then picks it."""
    w = WORKLOADS["C2"]
    margin = 0.033
    log = []
    out = autotune.tune_workload(w, trials=1, margin=margin, iters=5, verbose=False,
                                 references=_oracle_refs(w, 1), log=log)
    first, esc = log[0], log[1]
    assert first["tag"] == "heuristic" and first["plan"].compute_dtype == torch.float16
    assert first["usage"] > margin, f"the fp16 plan used only {first['usage']:.4f} of its budget"
    assert esc["tag"] == "escalate-fp32" and esc["usage"] <= margin, f"fp32 plan used {esc['usage']:.4f}"
    assert out is not None, "the fp32 escalation was not admitted"
    key, plan, res = out
    assert plan.compute_dtype == torch.float32 and plan.label == "autotuned-fp32"
    assert res["usage"] <= margin
    table = tmp_path / "plans.json"
    plans_mod.save_plans({key: plan}, table)
    chosen = _select(w, table, monkeypatch)
    assert chosen.compute_dtype == torch.float32 and chosen == plan


def test_autotune_gate_rejects_a_corrupted_plan(device, monkeypatch):
    """A planted error common to every plan -- every LayerNorm launched with
    eps = 0.5 instead of the module's 1e-5 -- is rejected by the gate
    measured against the oracle.  A gate referenced to this build's own
    fp32 plan (computed with the same planted error) admits it, which is
    why the tuner takes its reference from the caller."""
    w = WORKLOADS["C2"]
    plan = plans_mod.default_plan(w.batch, w.seq, w.d_model, w.heads, w.ffn_dim, w.layers, w.causal, w.dtype,
                                  torch.device("cuda", 0))
    ev = autotune._Evaluator(w, 1, 2, references=_oracle_refs(w, 1))
    good = ev.evaluate(plan)
    assert good["usage"] <= 0.85
    real = ops_mod.add_layernorm
    monkeypatch.setattr(ops_mod, "add_layernorm", lambda *a, **k: real(*a[:4], 0.5, *a[5:], **k))
    bad = ev.evaluate(plan)
    assert bad["usage"] > 1.0, f"the corrupted plan used only {bad['usage']:.2f} of its budget"
    self_ref = autotune._Evaluator(w, 1, 2)  # its fp32 reference carries the same error
    assert self_ref.evaluate(plan)["usage"] <= 0.85


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


def test_tile_step_pins_tiles_at_the_bench_rows_only(device):
    """The autotuner's tile step times each projection's tiles inside whole
    forwards on the bench input and pins the winners with tile_rows = that
    input's row bucket.  A forward on the bench input then runs exactly the
    pinned tiles and gives the bits of the run-time picks (same K-summation
    class); a forward with another row count times its own tiles."""
    from dataclasses import replace
    from tjkernels import UserOptimizedTransformer, tiles
    from tjkernels.engine import MASK_PREFIX, reset_engines
    w = WORKLOADS["C3"]
    base = plans_mod.default_plan(w.batch, w.seq, w.d_model, w.heads, w.ffn_dim, w.layers, w.causal, w.dtype,
                                  torch.device("cuda", 0))
    base = replace(base, cuda_graph=False)
    ev = autotune._Evaluator(w, 1, 3)
    best = autotune.tune_tiles(ev, ev.evaluate(base), w, rounds=1)
    pinned = best["plan"]
    rows = ev.bench_rows(pinned)
    mb = -(-rows // tiles.M_BUCKET) * tiles.M_BUCKET
    assert pinned.tile_rows == mb
    shapes = autotune._tile_shapes(w, pinned, rows)
    assert [s[0] for s in shapes] == ["gemm_qkv", "gemm_out", "gemm_ffn1", "gemm_ffn2"]
    for name, n, k, _ in shapes:
        assert getattr(pinned, name) in tiles.candidates(mb, n, k, pinned.compute_dtype), name

    model = UserOptimizedTransformer(w.config)
    model.load_state_dict(make_state_dict(w, seed=0), strict=True)
    model = model.to(device=device, dtype=w.dtype).eval()
    xb, maskb = ev.bench_input
    x2, mask2, len2 = make_inputs(w, seed=5)
    x2, mask2 = x2.to(device, w.dtype), mask2.to(device)
    rows2 = int(len2.sum())
    assert -(-rows2 // tiles.M_BUCKET) * tiles.M_BUCKET != mb  # another row bucket
    lens_b = tuple(int(n) for n in maskb.sum(1).tolist())
    outs = {}
    try:
        for tag, plan in (("pinned", pinned),
                          ("run-time", replace(pinned, tile_rows=0, gemm_qkv=-1, gemm_out=-1, gemm_ffn1=-1,
                                               gemm_ffn2=-1))):
            plans_mod.set_override(plan)
            reset_engines(model)
            with torch.inference_mode():
                outs[tag] = (model(xb, maskb).clone(), model(x2, mask2).clone())
            if tag == "pinned":
                eng = model._tj_engine  # its plan is the pinned one now

                def prepared(lengths):
                    return eng._prepare(w.batch, w.seq, MASK_PREFIX, eng._packing(lengths, w.seq), None).tiles

                t = prepared(lens_b)
                assert (t.qkv, t.out, t.fc1, t.fc2) == (pinned.gemm_qkv, pinned.gemm_out, pinned.gemm_ffn1,
                                                        pinned.gemm_ffn2)
                t2 = prepared(tuple(int(n) for n in len2.tolist()))  # another row count: run-time picks
                d, f = w.d_model, w.ffn_dim
                assert t2.qkv == tiles.gemm_plan(rows2, 3 * d, d, w.dtype, ops_mod.EPI_BIAS)
                assert t2.fc1 == tiles.gemm_plan(rows2, f, d, w.dtype, ops_mod.EPI_BIAS_GELU)
    finally:
        plans_mod.set_override(None)
    assert torch.equal(outs["pinned"][0], outs["run-time"][0])
    assert torch.equal(outs["pinned"][1], outs["run-time"][1])
