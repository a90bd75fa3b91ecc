"""End-to-end parity of the drop-in hook against the CPU oracle.

``UserOptimizedTransformer`` (HIP engine) and the oracle's restatement of
``BaselineTransformer`` run on the same seeded inputs and the same weights
(rounded to the model dtype; the oracle computes in fp32 on those values,
as bench/test_bf16_limit.py:73-77,88 does).  Per-element budget, OR rule of
torch_transformer_benchmark.py:313-320:
    fp16 / bf16 plans: |d| <= max(2e-2, 2e-2 |ref|)
    fp32 plans:        |d| <= max(1e-4, 1e-4 |ref|)
Padded rows must be exactly zero (bench/test_correctness.py:75-79).
"""

import pytest
import torch

from oracle import model as oracle
from tjkernels import Plan, TransformerConfig, UserOptimizedTransformer
from tjkernels import plans as plans_mod
from tjkernels.engine import MASK_NONE
from tjkernels.workloads import WORKLOADS, Workload, make_inputs, make_state_dict

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _module(cfg, sd, dtype, device):
    m = UserOptimizedTransformer(cfg)
    m.load_state_dict(sd, strict=True)
    return m.to(device=device, dtype=dtype).eval()


def _inputs(cfg, dtype, seed, padding=0.0, min_len=-2):
    """generate_random_case semantics (torch_transformer_benchmark.py:238-276)."""
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g)
    if min_len == -2:
        min_len = None if padding <= 0 else max(1, int(round(cfg.seq_len * (1.0 - padding))))
    if min_len is None:
        mask = torch.ones(cfg.batch_size, cfg.seq_len, dtype=torch.bool)
    else:
        lengths = torch.randint(min_len, cfg.seq_len + 1, (cfg.batch_size,), generator=g)
        mask = torch.arange(cfg.seq_len)[None, :] < lengths[:, None]
    x = x.masked_fill(~mask[..., None], 0).to(dtype)
    return x, mask


def _check(got, ref, mask, dtype):
    tol = TOL[dtype]
    r = oracle.compare_outputs(ref, got, rtol=tol, atol=tol)
    assert r["passed"], f"{r['failed']}/{r['total']} elements out of budget, max_abs={r['max_abs']:.3e}"
    if mask is not None and (~mask).any():
        assert (got.cpu()[~mask.cpu()] == 0).all(), "padded rows are not exactly zero"
    return r


def _run_workload(device, name, seeds=(1,), batch_subset=None, plan=None):
    w = WORKLOADS[name]
    sd = make_state_dict(w, seed=0)
    model = _module(w.config, sd, w.dtype, device)
    plans_mod.set_override(plan)
    try:
        for seed in seeds:
            x, mask, _ = make_inputs(w, seed=seed)
            xd = x.to(w.dtype).to(device)
            with torch.inference_mode():
                got = model(xd, mask.to(device)).cpu()
            sel = slice(None) if batch_subset is None else batch_subset
            ref = oracle.forward(sd, x[sel], mask[sel], w.heads, w.causal, torch.float32)
            _check(got[sel], ref, mask[sel], w.dtype)
    finally:
        plans_mod.set_override(None)


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4"])
def test_workload_parity(device, name):
    _run_workload(device, name, seeds=(1, 2))


def test_c5_parity_both_sequences(device):
    # the oracle costs seconds per C5 sequence; both are checked (the second
    # starts at packed row 4096, so its offsets are exercised too)
    _run_workload(device, "C5")


@pytest.mark.parametrize("name", ["C1", "C2"])
@pytest.mark.parametrize("ffn", ["gemm", "fused"])
def test_ffn_kinds_hold_the_budget(device, name, ffn):
    """Both FFN implementations -- two GEMM launches with the intermediate in
    HBM, and the single launch with it in LDS and LayerNorm 2 inside -- hold
    the workload's budget (C1: fp32 plan, 1e-4)."""
    w = WORKLOADS[name]
    cdt = torch.float32 if w.dtype == torch.float32 else w.dtype
    _run_workload(device, name, seeds=(1, 3),
                  plan=Plan(compute_dtype=cdt, ffn=ffn, cuda_graph=name == "C2", label=ffn))


def test_c5_fp32_escalation_plan(device):
    """The fp32 IEEE plan at the C5 shape holds the fp32 budget (1e-4):
    weights and x are the bf16-rounded values held in an fp32 model."""
    w = WORKLOADS["C5"]
    sd = make_state_dict(w, seed=0)
    model = _module(w.config, sd, torch.float32, device)
    x, mask, _ = make_inputs(w, seed=1)
    with torch.inference_mode():
        got = model(x.to(device), mask.to(device)).cpu()
    ref = oracle.forward(sd, x, mask, w.heads, w.causal, torch.float32)
    _check(got, ref, mask, torch.float32)


def test_c1_golden_fixture(device):
    """The committed C1 fixture (oracle fp64 output) is met by the fp32 plan."""
    from pathlib import Path
    fx = torch.load(Path(__file__).parent / "golden" / "c1_fixture.pt", weights_only=True)
    w = WORKLOADS["C1"]
    sd = make_state_dict(w, seed=int(fx["param_seed"]))
    model = _module(w.config, sd, w.dtype, device)
    with torch.inference_mode():
        got = model(fx["x"].to(device), fx["mask"].to(device)).cpu()
    _check(got, fx["out_fp64"], fx["mask"], torch.float32)


# ---- the reference's off-matrix cases (bench/test_correctness.py:132-156),
# with nn.Linear's default init under torch.manual_seed(1) as there.

CASES = [
    dict(id="baseline"),
    dict(id="padding0.3", padding=0.3),
    dict(id="padding0.6", padding=0.6),
    dict(id="non-causal", causal=False),
    dict(id="non-causal+padding", causal=False, padding=0.4),
    dict(id="fp16", dtype=torch.float16),
    dict(id="bf16", dtype=torch.bfloat16),
    dict(id="bf16+padding", dtype=torch.bfloat16, padding=0.5),
    dict(id="seq37", seq=37),
    dict(id="seq1", seq=1),
    dict(id="d96-h3", d_model=96, heads=3, ffn=96),
    dict(id="hd8", d_model=128, heads=16),
    dict(id="one-layer", layers=1),
    dict(id="ffn512", ffn=512),
    dict(id="batch1", batch=1),
]


@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_reference_cases(device, case):
    c = dict(batch=8, seq=64, d_model=128, heads=4, ffn=128, layers=2, causal=True,
             dtype=torch.float32, padding=0.0)
    c.update({k: v for k, v in case.items() if k != "id"})
    cfg = TransformerConfig(c["batch"], c["seq"], c["d_model"], c["heads"], c["ffn"],
                            c["layers"], c["causal"])
    torch.manual_seed(1)
    sd = {k: v.to(c["dtype"]).float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    model = _module(cfg, sd, c["dtype"], device)
    for trial in range(3):
        x, mask = _inputs(cfg, c["dtype"], seed=1 + trial, padding=c["padding"])
        with torch.inference_mode():
            got = model(x.to(device), mask.to(device)).cpu()
        ref = oracle.forward(sd, x.float(), mask, cfg.num_heads, cfg.causal, torch.float32)
        _check(got, ref, mask, c["dtype"])


def test_general_mask_and_lengths_input(device):
    """A non-prefix mask takes the per-key-mask attention path; int lengths
    are accepted in place of the bool mask (forward(x, lengths))."""
    cfg = TransformerConfig(4, 96, 128, 4, 256, 2, True)
    torch.manual_seed(1)
    sd = {k: v.float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    model = _module(cfg, sd, torch.float32, device)
    g = torch.Generator()
    g.manual_seed(3)
    x = torch.randn(4, 96, 128, generator=g)
    mask = torch.rand(4, 96, generator=g) > 0.3
    mask[:, 0] = True
    x = x.masked_fill(~mask[..., None], 0)
    with torch.inference_mode():
        got = model(x.to(device), mask.to(device)).cpu()
    ref = oracle.forward(sd, x, mask, 4, True, torch.float32)
    _check(got, ref, mask, torch.float32)

    lengths = torch.tensor([96, 1, 50, 95], dtype=torch.int32)
    pmask = torch.arange(96)[None, :] < lengths[:, None].long()
    x2 = x.masked_fill(~pmask[..., None], 0)
    with torch.inference_mode():
        got_l = model(x2.to(device), lengths.to(device)).cpu()
        got_m = model(x2.to(device), pmask.to(device)).cpu()
    assert torch.equal(got_l, got_m)
    _check(got_l, oracle.forward(sd, x2, pmask, 4, True, torch.float32), pmask, torch.float32)


@pytest.mark.parametrize("dtype,ffn,whole", [(torch.float32, "gemm", False), (torch.bfloat16, "gemm", False),
                                             (torch.bfloat16, "fused", False), (torch.float32, "fused", False),
                                             (torch.bfloat16, "fused", True), (torch.float32, "gemm", True)])
def test_graph_equals_eager(device, dtype, ffn, whole):
    """hipGraph replay == eager, bitwise, on fresh inputs, with eager work and
    synchronisations between replays (bench/test_correctness.py:94-125);
    ``whole``: the whole forward captured (static input copied in, output
    cloned), so every output must also be a fresh tensor."""
    cfg = TransformerConfig(4, 64, 128, 4, 256, 2, True)
    torch.manual_seed(1)
    eager = _module(cfg, UserOptimizedTransformer(cfg).state_dict(), dtype, device)
    graphed = _module(cfg, eager.state_dict(), dtype, device)
    cases = [_inputs(cfg, dtype, seed=50 + i, padding=0.3 * (i % 2)) for i in range(4)]
    # two non-prefix (GENERAL) masks: the captured attention reads the mask
    # from a static buffer the engine refreshes before every replay
    g = torch.Generator()
    g.manual_seed(7)
    for _ in range(2):
        m = torch.rand(cfg.batch_size, cfg.seq_len, generator=g) > 0.3
        m[:, 0] = True
        x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g).masked_fill(~m[..., None], 0)
        cases.append((x.to(dtype), m))
    plans_mod.set_override(Plan(compute_dtype=dtype, cuda_graph=False, ffn=ffn, label="eager"))
    try:
        with torch.inference_mode():
            expected = [eager(x.to(device), m.to(device)).cpu() for x, m in cases]
            # eager forwards add x into the residual in layer 0's out-proj
            # (the first LayerNorm writes no residual); graphed ones keep the
            # residual the first LayerNorm writes: the bits must agree
            fw = eager._tj_engine._prepare(cfg.batch_size, cfg.seq_len, MASK_NONE, None, None)
            assert fw.res_from_x
    finally:
        plans_mod.set_override(None)
    plans_mod.set_override(Plan(compute_dtype=dtype, cuda_graph=True, whole_graph=whole, ffn=ffn, label="graphed"))
    try:
        with torch.inference_mode():
            for rep in range(2):
                outs = []
                for (x, m), want in zip(cases, expected):
                    got = graphed(x.to(device), m.to(device))
                    torch.cuda.synchronize()
                    assert torch.equal(got.cpu(), want)
                    _ = (got * 2).sum().item()  # eager work between replays
                    outs.append(got)
                # earlier outputs are not overwritten by later replays
                for got, want in zip(outs, expected):
                    assert torch.equal(got.cpu(), want)
        assert len(graphed._tj_engine._graphs) >= 1
    finally:
        plans_mod.set_override(None)


def test_whole_graph_hot_key_survives_cache_churn(device):
    """Whole-forward capture: one key replayed between more new keys than
    the graph cache holds keeps the static input / output it was captured
    on, so each of its replays matches eager bit for bit (prefix lengths
    are part of the key, so every new lengths tuple is a new graph)."""
    cfg = TransformerConfig(2, 64, 128, 4, 256, 2, True)
    dtype = torch.float16
    torch.manual_seed(9)
    eager = _module(cfg, UserOptimizedTransformer(cfg).state_dict(), dtype, device)
    graphed = _module(cfg, eager.state_dict(), dtype, device)

    def case(lengths, seed):
        g = torch.Generator()
        g.manual_seed(seed)
        x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g)
        mask = torch.arange(cfg.seq_len)[None, :] < torch.tensor(lengths)[:, None]
        return x.masked_fill(~mask[..., None], 0).to(dtype), mask

    hot = case((64, 40), 1)
    others = [case((64, 10 + 3 * i), 2 + i) for i in range(7)]
    plans_mod.set_override(Plan(compute_dtype=dtype, cuda_graph=False, label="eager"))
    try:
        with torch.inference_mode():
            want_hot = eager(hot[0].to(device), hot[1].to(device)).cpu()
            want = [eager(x.to(device), m.to(device)).cpu() for x, m in others]
    finally:
        plans_mod.set_override(None)
    plans_mod.set_override(Plan(compute_dtype=dtype, cuda_graph=True, whole_graph=True, label="whole"))
    try:
        with torch.inference_mode():
            graphed(hot[0].to(device), hot[1].to(device))
            graphed._tj_engine._graphs.max_entries = 3
            for (x, m), w in zip(others, want):
                got = graphed(hot[0].to(device), hot[1].to(device)).cpu()
                assert torch.equal(got, want_hot)
                assert torch.equal(graphed(x.to(device), m.to(device)).cpu(), w)
            assert len(graphed._tj_engine._graphs) <= 3
    finally:
        plans_mod.set_override(None)


BLOCK_CASES = [
    dict(id="c2-graph", workload="C2"),
    dict(id="ragged-causal", cfg=(6, 128, 256, 4, 512, 2, True), dtype=torch.bfloat16, padding=0.7),
    dict(id="ragged-noncausal-graph", cfg=(5, 100, 384, 6, 768, 2, False), dtype=torch.float16, padding=0.5,
         graph=True, ffn="gemm"),
    dict(id="deferred-two-launch-ffn", cfg=(3, 64, 512, 8, 1024, 2, True), dtype=torch.bfloat16, padding=0.0,
         residual_epilogue=False, ffn="gemm"),
]


@pytest.mark.parametrize("case", BLOCK_CASES, ids=[c["id"] for c in BLOCK_CASES])
def test_attention_block_plan(device, case, monkeypatch):
    """Plan.attn_block: the QKV GEMM, attention and out-projection of each
    layer in one launch, the per-head partials summed into the residual by
    LayerNorm 2, holds the budget against the oracle -- at C2, on packed
    ragged sequences (causal and not, eager and graphed), and with the
    deferred residual and the two-launch FFN.  A non-prefix mask, which the
    block kernel does not take, runs the three launches on the same plan."""
    from tjkernels import ops as ops_mod
    calls = []
    real = ops_mod.attn_block
    monkeypatch.setattr(ops_mod, "attn_block", lambda *a, **k: calls.append(1) or real(*a, **k))
    if "workload" in case:
        w = WORKLOADS[case["workload"]]
        _run_workload(device, case["workload"], seeds=(1, 2),
                      plan=Plan(compute_dtype=w.dtype, ffn="fused", cuda_graph=True, attn_block=True,
                                label="block"))
        assert calls, "the attention block was not used"
        return
    cfg = TransformerConfig(*case["cfg"])
    dtype = case["dtype"]
    torch.manual_seed(3)
    sd = {k: v.to(dtype).float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    model = _module(cfg, sd, dtype, device)
    plan = Plan(compute_dtype=dtype, attn_block=True, cuda_graph=case.get("graph", False),
                residual_epilogue=case.get("residual_epilogue", True), ffn=case.get("ffn", "fused"),
                label="block")
    plans_mod.set_override(plan)
    try:
        for seed in (1, 2):
            x, mask = _inputs(cfg, dtype, seed=seed, padding=case["padding"])
            with torch.inference_mode():
                got = model(x.to(device), mask.to(device)).cpu()
            ref = oracle.forward(sd, x.float(), mask, cfg.num_heads, cfg.causal, torch.float32)
            _check(got, ref, mask, dtype)
        assert calls, "the attention block was not used"
        n_block = len(calls)
        # a non-prefix mask: per-key masked attention, three launches per layer
        g = torch.Generator()
        g.manual_seed(5)
        m = torch.rand(cfg.batch_size, cfg.seq_len, generator=g) > 0.4
        m[:, 0] = True
        x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g).masked_fill(~m[..., None], 0)
        x = x.to(dtype)
        with torch.inference_mode():
            got = model(x.to(device), m.to(device)).cpu()
        _check(got, oracle.forward(sd, x.float(), m, cfg.num_heads, cfg.causal, torch.float32), m, dtype)
        assert len(calls) == n_block, "the attention block ran on a general mask"
    finally:
        plans_mod.set_override(None)


def test_attention_block_graph_equals_eager(device):
    """With the attention block, hipGraph replay == eager bit for bit on
    fresh prefix-masked inputs, replayed twice with eager work between."""
    cfg = TransformerConfig(3, 96, 256, 4, 512, 2, True)
    dtype = torch.bfloat16
    torch.manual_seed(6)
    eager = _module(cfg, UserOptimizedTransformer(cfg).state_dict(), dtype, device)
    graphed = _module(cfg, eager.state_dict(), dtype, device)
    cases = [_inputs(cfg, dtype, seed=80 + i, padding=0.5 * (i % 2)) for i in range(3)]
    plans_mod.set_override(Plan(compute_dtype=dtype, attn_block=True, cuda_graph=False, ffn="fused", label="e"))
    try:
        with torch.inference_mode():
            expected = [eager(x.to(device), m.to(device)).cpu() for x, m in cases]
    finally:
        plans_mod.set_override(None)
    plans_mod.set_override(Plan(compute_dtype=dtype, attn_block=True, cuda_graph=True, ffn="fused", label="g"))
    try:
        with torch.inference_mode():
            for _ in range(2):
                for (x, m), want in zip(cases, expected):
                    got = graphed(x.to(device), m.to(device))
                    torch.cuda.synchronize()
                    assert torch.equal(got.cpu(), want)
                    _ = (got * 2).sum().item()
        assert len(graphed._tj_engine._graphs) >= 1
    finally:
        plans_mod.set_override(None)


def test_deferred_residual_plan_matches(device):
    """The reference's deferred-residual scheme (residual_epilogue=False)
    stays inside the budget too."""
    w = WORKLOADS["C3"]
    _run_workload(device, "C3", plan=Plan(compute_dtype=w.dtype, residual_epilogue=False,
                                          cuda_graph=False, label="deferred"))


LN_GEMM_CASES = [
    dict(id="c2-graph", workload="C2", plan=dict(ffn="gemm", cuda_graph=True)),
    dict(id="c2-eager", workload="C2", plan=dict(ffn="gemm", cuda_graph=False)),
    dict(id="ragged-bf16", cfg=(5, 96, 256, 4, 1024, 3, True), dtype=torch.bfloat16, padding=0.6),
    dict(id="ragged-noncausal-d768", cfg=(3, 64, 768, 12, 1536, 2, False), dtype=torch.float16, padding=0.5),
]


@pytest.mark.parametrize("case", LN_GEMM_CASES, ids=[c["id"] for c in LN_GEMM_CASES])
def test_layernorm_inside_gemm_plan(device, case, monkeypatch):
    """Plan.ln_gemm: LayerNorm 1 (after layer 0) and LayerNorm 2 computed
    inside the QKV and FFN1 GEMMs holds the budget against the oracle -- at
    C2 (graphed and eager) and on packed ragged sequences (causal and not) --
    and the fused GEMM is the one that runs."""
    from tjkernels import ops as ops_mod
    calls = []
    real = ops_mod.gemm_ln
    monkeypatch.setattr(ops_mod, "gemm_ln", lambda *a, **k: calls.append(1) or real(*a, **k))
    if "workload" in case:
        w = WORKLOADS[case["workload"]]
        _run_workload(device, case["workload"], seeds=(1, 2),
                      plan=Plan(compute_dtype=w.dtype, ln_gemm=True, label="ln", **case["plan"]))
        assert calls, "the LayerNorm GEMM was not used"
        return
    monkeypatch.setenv("TJ_GEMM_TUNE", "0")  # no tile timing: every counted call is the forward's
    cfg = TransformerConfig(*case["cfg"])
    dtype = case["dtype"]
    torch.manual_seed(11)
    sd = {k: v.to(dtype).float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    model = _module(cfg, sd, dtype, device)
    plans_mod.set_override(Plan(compute_dtype=dtype, ln_gemm=True, cuda_graph=False, ffn="gemm", label="ln"))
    try:
        for seed in (1, 2):
            x, mask = _inputs(cfg, dtype, seed=seed, padding=case["padding"])
            with torch.inference_mode():
                got = model(x.to(device), mask.to(device)).cpu()
            ref = oracle.forward(sd, x.float(), mask, cfg.num_heads, cfg.causal, torch.float32)
            _check(got, ref, mask, dtype)
        # 2 launches per layer, LayerNorm 1 of layer 0 excepted
        assert len(calls) == 2 * (2 * cfg.num_layers - 1)
    finally:
        plans_mod.set_override(None)


def test_layernorm_inside_gemm_graph_equals_eager(device):
    """With the LayerNorms inside the GEMMs, hipGraph replay == eager bit
    for bit, replayed twice with eager work between."""
    cfg = TransformerConfig(2, 128, 512, 8, 2048, 3, True)
    dtype = torch.float16
    torch.manual_seed(12)
    eager = _module(cfg, UserOptimizedTransformer(cfg).state_dict(), dtype, device)
    graphed = _module(cfg, eager.state_dict(), dtype, device)
    cases = [_inputs(cfg, dtype, seed=60 + i, padding=0.5 * (i % 2)) for i in range(3)]
    base = dict(compute_dtype=dtype, ln_gemm=True, ffn="gemm")
    plans_mod.set_override(Plan(cuda_graph=False, label="e", **base))
    try:
        with torch.inference_mode():
            expected = [eager(x.to(device), m.to(device)).cpu() for x, m in cases]
    finally:
        plans_mod.set_override(None)
    plans_mod.set_override(Plan(cuda_graph=True, label="g", **base))
    try:
        with torch.inference_mode():
            for _ in range(2):
                for (x, m), want in zip(cases, expected):
                    got = graphed(x.to(device), m.to(device))
                    torch.cuda.synchronize()
                    assert torch.equal(got.cpu(), want)
                    _ = (got * 2).sum().item()
    finally:
        plans_mod.set_override(None)


RESIDUAL_CASES = [
    dict(id="c2-fp16-graph-fused", workload="C2", residual=torch.float16,
         plan=dict(ffn="fused", cuda_graph=True)),
    dict(id="c2-fp16-block", workload="C2", residual=torch.float16,
         plan=dict(ffn="fused", cuda_graph=True, attn_block=True)),
    dict(id="c3-fp16", workload="C3", residual=torch.float16, plan=dict(cuda_graph=False)),
    dict(id="c4-fp16", workload="C4", residual=torch.float16, plan=dict(cuda_graph=False)),
    # f = 128 at 1024 rows: the single-launch FFN runs one f-slice, whose
    # output goes through the partials buffer since the residual is 2-byte
    dict(id="unsplit-fused-ffn", cfg=(8, 128, 256, 4, 128, 2, True), dtype=torch.bfloat16, padding=0.0,
         residual=torch.float16, plan=dict(ffn="fused", cuda_graph=True)),
]
# A bf16 residual stream is accepted by the plan but does not hold C4's
# budget: 1241 of 8.4M elements out, max |d| 0.058 on this kernel set, and a
# CPU restatement that rounds only the residual to bf16 already puts 132
# elements of one sequence out (max |d| 0.051; fp16: 0.0064).  That is what
# the autotuner's accuracy gate is for; its candidate is fp16.


@pytest.mark.parametrize("case", RESIDUAL_CASES, ids=[c["id"] for c in RESIDUAL_CASES])
def test_two_byte_residual_plans(device, case):
    """An fp16 residual stream (the reference's residual_dtype knob and its
    autotuner's fp16 candidate, plans.py:33-36, bench/autotune.py:88) holds
    the workload's budget against the oracle: the deferred scheme with the
    two-launch and the single-launch FFN, the attention block, packed ragged
    sequences (C3, C4) and graph replay (C2)."""
    if "workload" in case:
        w = WORKLOADS[case["workload"]]
        plan = Plan(compute_dtype=w.dtype, residual_dtype=case["residual"], label=case["id"], **case["plan"])
        _run_workload(device, case["workload"], seeds=(1, 2), plan=plan)
        return
    from tjkernels.engine import ffn_slices
    cfg = TransformerConfig(*case["cfg"])
    dtype = case["dtype"]
    assert ffn_slices(cfg.batch_size * cfg.seq_len, cfg.ffn_dim) == 1
    torch.manual_seed(13)
    sd = {k: v.to(dtype).float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    model = _module(cfg, sd, dtype, device)
    plans_mod.set_override(Plan(compute_dtype=dtype, residual_dtype=case["residual"], label=case["id"],
                                **case["plan"]))
    try:
        for seed in (1, 2):
            x, mask = _inputs(cfg, dtype, seed=seed, padding=case["padding"])
            with torch.inference_mode():
                got = model(x.to(device), mask.to(device)).cpu()
            ref = oracle.forward(sd, x.float(), mask, cfg.num_heads, cfg.causal, torch.float32)
            _check(got, ref, mask, dtype)
    finally:
        plans_mod.set_override(None)


def test_two_byte_residual_graph_equals_eager_and_env(device, monkeypatch):
    """With an fp16 residual stream, hipGraph replay == eager bit for bit;
    TJ_RESIDUAL_DTYPE=float16 selects the same plan on the heuristic path,
    and its residual workspace is fp16."""
    cfg = TransformerConfig(2, 128, 256, 4, 1024, 2, True)
    dtype = torch.bfloat16
    torch.manual_seed(8)
    eager = _module(cfg, UserOptimizedTransformer(cfg).state_dict(), dtype, device)
    graphed = _module(cfg, eager.state_dict(), dtype, device)
    cases = [_inputs(cfg, dtype, seed=40 + i, padding=0.4 * (i % 2)) for i in range(3)]
    base = dict(compute_dtype=dtype, residual_dtype=torch.float16, ffn="gemm")
    plans_mod.set_override(Plan(cuda_graph=False, label="e", **base))
    try:
        with torch.inference_mode():
            expected = [eager(x.to(device), m.to(device)).cpu() for x, m in cases]
    finally:
        plans_mod.set_override(None)
    plans_mod.set_override(Plan(cuda_graph=True, label="g", **base))
    try:
        with torch.inference_mode():
            for _ in range(2):
                for (x, m), want in zip(cases, expected):
                    got = graphed(x.to(device), m.to(device))
                    torch.cuda.synchronize()
                    assert torch.equal(got.cpu(), want)
                    _ = (got * 2).sum().item()
    finally:
        plans_mod.set_override(None)
    monkeypatch.setenv("TJ_IGNORE_PLANS", "1")
    monkeypatch.setenv("TJ_RESIDUAL_DTYPE", "float16")
    monkeypatch.setenv("TJ_NO_GRAPH", "1")
    monkeypatch.setenv("TJ_FFN", "gemm")
    plans_mod.TUNED._plans = None
    try:
        by_env = _module(cfg, eager.state_dict(), dtype, device)
        with torch.inference_mode():
            x, m = cases[0]
            got = by_env(x.to(device), m.to(device)).cpu()
        eng = by_env._tj_engine
        assert eng.plan.residual_dtype == torch.float16
        assert all(ws.res.dtype == torch.float16 for ws in eng._workspaces.values())
        assert torch.equal(got, expected[0])
    finally:
        plans_mod.TUNED._plans = None


@pytest.mark.parametrize("causal", [True, False])
def test_packed_forward_matches_unpacked(device, causal):
    """Prefix masks run packed (only the valid rows through every GEMM and
    LayerNorm, varlen attention); the valid rows must equal the unpacked
    forward that computes every row with a per-key mask (the reference's
    way, tjkernels/engine.py:184-203,267-268), and a zero-length sequence
    comes out as all-zero rows."""
    from tjkernels.engine import MASK_GENERAL
    cfg = TransformerConfig(4, 80, 128, 4, 256, 2, causal)
    torch.manual_seed(2)
    sd = {k: v.float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    model = _module(cfg, sd, torch.float32, device)
    lengths = torch.tensor([80, 0, 33, 1], dtype=torch.int32)
    mask = torch.arange(80)[None, :] < lengths[:, None].long()
    g = torch.Generator()
    g.manual_seed(9)
    x = torch.randn(4, 80, 128, generator=g).masked_fill(~mask[..., None], 0)
    plans_mod.set_override(Plan(compute_dtype=torch.float32, cuda_graph=False, label="eager"))
    try:
        with torch.inference_mode():
            packed = model(x.to(device), lengths.to(device)).cpu()
            eng = model._tj_engine
            unpacked = eng._forward_impl(x.to(device), mask.to(device), MASK_GENERAL).cpu()
    finally:
        plans_mod.set_override(None)
    # the same through the plan knob (TJ_NO_PACK / Plan.pack_prefix=False)
    plans_mod.set_override(Plan(compute_dtype=torch.float32, cuda_graph=False, pack_prefix=False,
                                label="unpacked"))
    try:
        with torch.inference_mode():
            by_plan = _module(cfg, sd, torch.float32, device)(x.to(device), mask.to(device)).cpu()
    finally:
        plans_mod.set_override(None)
    assert torch.equal(by_plan, unpacked)
    assert (packed[~mask] == 0).all() and (unpacked[~mask] == 0).all()
    diff = (packed[mask] - unpacked[mask]).abs().max().item()
    assert diff <= 1e-5, f"packed vs unpacked valid rows differ by {diff:.3e}"
    keep = lengths > 0
    ref = oracle.forward(sd, x[keep], mask[keep], cfg.num_heads, causal, torch.float32)
    _check(packed[keep], ref, mask[keep], torch.float32)


def test_long_sequence_prefix_property(device):
    """A 100000-token causal forward (case 14's length) runs in O(S) memory,
    and its first P rows equal the forward of the first P tokens alone: under
    causal attention no row sees a later token, and every other op is
    row-wise.  The short forward is checked against the CPU oracle, so the
    long one is pinned on those rows without an S x S reference."""
    w = Workload("long", 2, 256, 4, 512, 1, 100000, torch.bfloat16, None, 0.02)
    cfg = w.config
    sd = make_state_dict(w, seed=5)
    model = _module(cfg, sd, torch.bfloat16, device)
    g = torch.Generator()
    g.manual_seed(14)
    x = torch.randn(1, 100000, 256, generator=g).to(torch.bfloat16)
    p = 300
    short_cfg = TransformerConfig(1, p, 256, 4, 512, 2, True)
    short = _module(short_cfg, sd, torch.bfloat16, device)
    with torch.inference_mode():
        long_out = model(x.to(device)).cpu()
        short_out = short(x[:, :p].contiguous().to(device)).cpu()
    assert torch.isfinite(long_out).all()
    d = (long_out[:, :p].float() - short_out.float()).abs().max().item()
    assert d <= 2e-2, f"prefix rows differ from the short forward by {d:.3e}"
    full = torch.ones(1, p, dtype=torch.bool)
    ref = oracle.forward(sd, x[:, :p].float(), full, cfg.num_heads, True, torch.float32)
    _check(short_out, ref, full, torch.bfloat16)


@pytest.mark.parametrize("graph", [False, True])
def test_mask_updated_in_place_between_forwards(device, graph):
    """A mask buffer reused with new contents (written in place) is
    re-classified: each forward equals the forward of a fresh mask tensor
    with the same contents -- through the eager path and the hipGraph path
    (whose key holds the prefix lengths) -- for prefix masks of new
    lengths, a non-prefix mask and integer lengths updated in place."""
    cfg = TransformerConfig(3, 64, 128, 4, 256, 2, True)
    torch.manual_seed(4)
    sd = {k: v.float() for k, v in UserOptimizedTransformer(cfg).state_dict().items()}
    g = torch.Generator()
    g.manual_seed(21)
    x = torch.randn(3, 64, 128, generator=g).to(device)
    plans_mod.set_override(Plan(compute_dtype=torch.float32, cuda_graph=graph, label="inplace"))
    try:
        reused = _module(cfg, sd, torch.float32, device)
        fresh = _module(cfg, sd, torch.float32, device)
        buf = torch.ones(3, 64, dtype=torch.bool, device=device)
        lens_buf = torch.tensor([64, 64, 64], dtype=torch.int32, device=device)
        contents = []
        for lens in ([64, 10, 33], [5, 64, 20], [64, 64, 64], [40, 1, 64]):
            contents.append(torch.arange(64)[None, :] < torch.tensor(lens)[:, None])
        general = contents[0].clone()
        general[0, 5] = False
        contents.append(general)
        with torch.inference_mode():
            for want_mask in contents:
                buf.copy_(want_mask.to(device))  # in place: same tensor, new contents
                got = reused(x, buf)
                ref = fresh(x, want_mask.to(device).clone())
                torch.cuda.synchronize()
                assert torch.equal(got.cpu(), ref.cpu())
                assert (got.cpu()[~want_mask] == 0).all()
            for lens in ([64, 10, 33], [5, 64, 20]):
                lens_buf.copy_(torch.tensor(lens, dtype=torch.int32))
                got = reused(x, lens_buf)
                ref = fresh(x, (torch.arange(64)[None, :] < torch.tensor(lens)[:, None]).to(device))
                assert torch.equal(got.cpu(), ref.cpu())
    finally:
        plans_mod.set_override(None)


_TWO_PROCESS_SCRIPT = r"""
import hashlib, json, sys
import torch
from tjkernels import UserOptimizedTransformer, tiles
from tjkernels.workloads import WORKLOADS, make_inputs, make_state_dict
w = WORKLOADS["C4"]
m = UserOptimizedTransformer(w.config)
m.load_state_dict(make_state_dict(w, seed=0), strict=True)
m = m.to(device="cuda", dtype=w.dtype).eval()
x, mask, _ = make_inputs(w, seed=1)
with torch.inference_mode():
    out = m(x.to(w.dtype).cuda(), mask.cuda())
torch.cuda.synchronize()
raw = out.contiguous().view(torch.int16).cpu().numpy().tobytes()
print(json.dumps({"sha": hashlib.sha256(raw).hexdigest(),
                  "tiles": sorted(str(k) + ":" + str(v) for k, v in tiles.chosen().items())}))
"""


def test_two_processes_bitwise_identical(device, tmp_path):
    """Two fresh processes run the packed C4 forward, one choosing GEMM tiles
    by timing and one with the library's own tile rule (TJ_GEMM_TUNE=0):
    whatever tiles they run, every tile of a shape's K-summation class adds
    K in the same order, so the outputs are bitwise identical."""
    import json
    import os
    import subprocess
    import sys
    script = tmp_path / "c4_forward.py"
    script.write_text(_TWO_PROCESS_SCRIPT)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    pkg = os.path.join(root, "tiktok-techjam-2026_amd")
    res = []
    for extra in ({}, {"TJ_GEMM_TUNE": "0"}):
        env = dict(os.environ, PYTHONPATH=os.pathsep.join([pkg, root, os.environ.get("PYTHONPATH", "")]), **extra)
        r = subprocess.run([sys.executable, str(script)], env=env, capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-3000:]
        res.append(json.loads(r.stdout.strip().splitlines()[-1]))
    assert res[0]["tiles"] != res[1]["tiles"], "the two runs should have used different tile choices"
    assert res[0]["sha"] == res[1]["sha"], "outputs differ between processes"
