"""Host-side logic that runs without a GPU: the C-ABI library's exports, the
plan dispatcher, the module skeleton, the engine's guards, mask
classification, and graph-capture failure handling."""

import csv
import json
import re
from pathlib import Path

import pytest
import torch

import tjkernels
from tjkernels import Plan, TransformerConfig, UserOptimizedTransformer, _lib
from tjkernels import plans as plans_mod
from tjkernels.engine import MASK_GENERAL, MASK_NONE, MASK_PREFIX, Engine
from tjkernels.graphs import GraphCache

ROOT = Path(__file__).resolve().parents[1]


def test_library_exports_every_declared_symbol():
    header = (ROOT / "include" / "tjk.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|const char\*|size_t)\s+(tjk_\w+)\(", header, re.M))
    assert declared, "no declarations parsed"
    lib = _lib.load()
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in tjk.h but not exported"
    assert declared == set(_lib.EXPORTED_SYMBOLS)
    assert lib.tjk_abi_version() == _lib.ABI_VERSION


def test_abi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    # null pointers / bad shapes return a negative status and set the message
    assert lib.tjk_gemm_bias(None, 8, None, 8, None, None, 8, 4, 4, 8, _lib.BF16, 0, -1, None) < 0
    assert b"null" in lib.tjk_last_error_string()
    assert lib.tjk_flash_fwd(None, 0, 0, 0, 0, None, 0, 1, 4, 1, 12, 0.5, 1, None, None,
                             None, _lib.BF16, -1, None) < 0
    assert lib.tjk_add_layernorm(None, 0, 8, None, 0, 0, 1, 0, None, 0, 0, None, 0, 8, None, None,
                                 2, 6, 1e-5, None, 0, None, None, None) < 0
    assert b"null pointer" in lib.tjk_last_error_string()
    # split deltas need a stride that keeps the slices apart
    fake = 1 << 20  # never dereferenced: the call is rejected first
    assert lib.tjk_add_layernorm(fake, 0, 8, fake, 0, 8, 4, 8, None, 0, 0, fake, 0, 8, fake, fake,
                                 2, 8, 1e-5, None, 0, None, None, None) == _lib.EINVAL
    # the residual is written in place only in its own dtype and leading dimension
    assert lib.tjk_add_layernorm(fake, _lib.F32, 8, None, 0, 0, 1, 0, fake, _lib.F16, 8, fake, 0, 8, fake,
                                 fake, 2, 8, 1e-5, None, 0, None, None, None) == _lib.EINVAL
    assert b"alias" in lib.tjk_last_error_string()
    assert lib.tjk_add_layernorm(fake, _lib.F16, 8, None, 0, 0, 1, 0, fake, 7, 8, fake, 0, 8, fake,
                                 fake, 2, 8, 1e-5, None, 0, None, None, None) == _lib.EINVAL  # bad res_out dtype
    # a row_index needs a source-row count it is bounded by
    assert lib.tjk_add_layernorm(fake, _lib.F32, 8, None, 0, 0, 1, 0, None, 0, 0, fake, 0, 8, fake,
                                 fake, 2, 8, 1e-5, fake, -1, None, None, None) == _lib.EINVAL
    assert b"src_rows" in lib.tjk_last_error_string()
    # the single-launch FFN's shape gate (f / splits must be 128; d in {128, 256, 512})
    assert lib.tjk_ffn_supported(512, 2048, 16, _lib.F16) == 1
    assert lib.tjk_ffn_supported(128, 512, 4, _lib.F32) == 1
    assert lib.tjk_ffn_supported(512, 2048, 32, _lib.BF16) == 1  # 64-column slices
    assert lib.tjk_ffn_supported(512, 2048, 8, _lib.F16) == 0
    assert lib.tjk_ffn_supported(512, 2048, 16, _lib.F32) == 0
    assert lib.tjk_ffn_supported(1024, 4096, 32, _lib.BF16) == 0
    assert lib.tjk_ffn(fake, _lib.F16, 768, None, None, 0.0, fake, None, fake, None, fake, 768, 0, 24, 0,
                       16, 768, 3072, _lib.F16, None) == _lib.EUNSUPPORTED
    assert lib.tjk_ffn(fake, _lib.F16, 512, None, None, 0.0, fake, None, fake, None, fake, 512, 0, 16, 1,
                       16, 512, 2048, _lib.F16, None) == _lib.EINVAL  # accumulate with 16 splits
    # scheduled attention: split slots without enough partials bytes
    assert lib.tjk_flash_fwd_sched(fake, 192, 64, 64, fake, 64, 1, 128, 1, 64, 0.125, 1, fake, fake, 2, 2,
                                   fake, 16, 1, _lib.BF16, None) == _lib.EINVAL
    # the lists of a work list: 1 .. n_work of them
    for n_lists in (0, 3, -1):
        assert lib.tjk_flash_fwd_sched(fake, 192, 64, 64, fake, 64, 1, 128, 1, 64, 0.125, 1, fake, fake, 2,
                                       n_lists, None, 0, 0, _lib.BF16, None) == _lib.EINVAL
    # the residual GEMM reading x: x is required, bounded and aligned like the residual
    from_x = lib.tjk_gemm_bias_residual_from
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, None, 8, 4, None, None, _lib.BF16, -1, None) \
        == _lib.EINVAL
    assert b"null" in lib.tjk_last_error_string()
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, fake, 4, 4, None, None, _lib.BF16, -1, None) \
        == _lib.EINVAL  # ld_x < n
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, fake, 8, -1, None, None, _lib.BF16, -1, None) \
        == _lib.EINVAL  # negative x_rows
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, fake + 2, 8, 4, None, None, _lib.BF16, -1, None) \
        == _lib.EUNSUPPORTED  # x not aligned to 4 elements
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, fake, 8, 4, fake + 2, None, _lib.BF16, -1, None) \
        == _lib.EUNSUPPORTED  # misaligned row map
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, fake, 10, 4, None, None, _lib.BF16, -1, None) \
        == _lib.EUNSUPPORTED  # ld_x % 4
    assert from_x(None, 8, None, 8, None, None, 8, 0, 8, 8, None, 8, 0, None, None, _lib.BF16, -1, None) == 0
    # x may be NULL only when it has no rows (then nothing of it is read)
    assert from_x(fake, 8, fake, 8, None, fake, 8, 4, 8, 8, None, 8, 1, None, None, _lib.BF16, -1, None) \
        == _lib.EINVAL
    # empty work is a successful no-op
    assert lib.tjk_gemm_bias(None, 8, None, 8, None, None, 8, 0, 4, 8, _lib.BF16, 0, -1, None) == 0
    assert lib.tjk_gemm_plan_count(_lib.BF16) >= 4
    assert lib.tjk_flash_plan_count(_lib.F32) == 5
    # plan 4 takes sequences of at most 128 tokens (checked before any launch)
    assert lib.tjk_flash_fwd(fake, 0, 3 * 64, 64, 64, fake, 64, 1, 129, 1, 64, 0.125, 1, None, None,
                             None, _lib.BF16, 4, None) == _lib.EUNSUPPORTED


def test_state_dict_keys_match_reference_layout():
    cfg = TransformerConfig(2, 8, 32, 4, 64, 2, True)
    keys = set(UserOptimizedTransformer(cfg).state_dict())
    want = set()
    for i in range(2):
        p = f"layers.{i}."
        for n in ("norm1", "norm2"):
            want |= {p + n + ".weight", p + n + ".bias"}
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            want |= {p + f"attention.{n}.weight", p + f"attention.{n}.bias"}
        for n in ("ffn_in", "ffn_out"):
            want |= {p + n + ".weight", p + n + ".bias"}
    want |= {"final_norm.weight", "final_norm.bias"}
    assert keys == want
    sd = UserOptimizedTransformer(cfg).state_dict()
    assert sd["layers.0.ffn_in.weight"].shape == (64, 32)
    assert sd["layers.0.ffn_out.weight"].shape == (32, 64)


def test_config_validation():
    with pytest.raises(ValueError):
        TransformerConfig(1, 8, 30, 4, 64, 1, True).validate()
    with pytest.raises(ValueError):
        TransformerConfig(0, 8, 32, 4, 64, 1, True).validate()


def test_no_cpu_path():
    cfg = TransformerConfig(1, 4, 32, 4, 64, 1, True)
    m = UserOptimizedTransformer(cfg).eval()
    with pytest.raises(RuntimeError, match="ROCm"):
        m(torch.randn(1, 4, 32))
    with pytest.raises(RuntimeError, match="ROCm"):
        plans_mod.default_plan(1, 4, 32, 4, 64, 1, True, torch.float32, torch.device("cpu"))


def test_plan_json_round_trip_and_table(tmp_path, monkeypatch):
    p = Plan(compute_dtype=torch.float16, gemm_qkv=2, attn_plan=1, cuda_graph=False, label="x")
    assert Plan.from_json(json.loads(json.dumps(p.to_json()))) == p
    key = plans_mod.shape_key(4, 2048, 1024, 16, 4096, 4, True, torch.bfloat16, "gfx950")
    assert key == "b4_s2048_d1024_h16_f4096_l4_causal_bfloat16@gfx950"
    f = tmp_path / "plans.json"
    monkeypatch.setattr(plans_mod, "TUNED", plans_mod.PlanTable(f))
    plans_mod.save_plans({key: p})
    plans_mod.save_plans({"other@gfx950": Plan(label="y")})
    table = plans_mod.TUNED.plans()
    assert table[key] == p and table["other@gfx950"].label == "y"
    # an unreadable table is ignored, never fatal
    f.write_text("{not json")
    monkeypatch.setattr(plans_mod, "TUNED", plans_mod.PlanTable(f))
    assert plans_mod.TUNED.plans() == {}
    # tables written before the FFN knob named the two-launch FFN "hip"
    assert Plan.from_json({"ffn": "hip", "compute_dtype": "float16"}).ffn == "gemm"
    # the committed table parses, and every entry validates
    for plan in plans_mod.PlanTable(plans_mod.TUNED_PATH).plans().values():
        plan.validate()


def test_plan_validation_rejects_fallback_backends():
    with pytest.raises(ValueError, match="only 'hip'"):
        Plan(attn="sdpa").validate()
    with pytest.raises(ValueError, match="residual_dtype"):
        Plan(residual_dtype=torch.int8).validate()
    with pytest.raises(ValueError, match="ffn="):
        Plan(ffn="torch").validate()
    Plan().validate()
    Plan(ffn="fused").validate()
    # 2-byte residual streams (the reference's knob) run the deferred scheme:
    # the GEMM epilogues add into an fp32 residual only
    for rdt in (torch.float16, torch.bfloat16):
        p = Plan(residual_dtype=rdt)
        p.validate()
        assert p.residual_epilogue and not p.epilogue_residual
        assert Plan.from_json(p.to_json()) == p
    assert Plan().epilogue_residual and not Plan(residual_epilogue=False).epilogue_residual


def test_override_and_env_knobs(monkeypatch):
    forced = Plan(label="forced")
    plans_mod.set_override(forced)
    try:
        assert plans_mod.select_plan(1, 1, 8, 1, 8, 1, True, torch.float32,
                                     torch.device("cpu")) is forced
    finally:
        plans_mod.set_override(None)
    monkeypatch.setattr(plans_mod, "device_arch", lambda d: "gfx950")
    monkeypatch.setattr(plans_mod, "TUNED", plans_mod.PlanTable(Path("/nonexistent/plans.json")))
    dev = torch.device("cuda", 0)
    base = plans_mod.select_plan(4, 2048, 1024, 16, 4096, 4, True, torch.bfloat16, dev)
    assert not base.cuda_graph and base.compute_dtype == torch.bfloat16 and base.residual_epilogue
    assert base.ffn == "gemm"  # d = 1024: the two-launch FFN
    small = plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev)
    assert small.cuda_graph and small.residual_epilogue  # launch-bound: replayed as a hipGraph
    assert small.ffn == "gemm"  # C2: two launches measured faster than the single-launch FFN
    tiny = plans_mod.select_plan(2, 64, 128, 4, 512, 2, True, torch.float32, dev)
    assert tiny.ffn == "fused" and tiny.compute_dtype == torch.float32  # C1
    big = plans_mod.select_plan(64, 4096, 1024, 16, 4096, 4, True, torch.bfloat16, dev)
    assert not big.cuda_graph  # x above 64 MiB: no whole-forward graph
    # fp32 compute at C2's d = 512 has no single-launch FFN kernel: two launches
    monkeypatch.setenv("TJ_COMPUTE_DTYPE", "float32")
    p32 = plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev)
    assert p32.compute_dtype == torch.float32 and p32.ffn == "gemm"
    monkeypatch.delenv("TJ_COMPUTE_DTYPE")
    monkeypatch.setenv("TJ_NO_GRAPH", "1")
    monkeypatch.setenv("TJ_DEFERRED_RESIDUAL", "1")
    p = plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev)
    assert not p.cuda_graph and not p.residual_epilogue
    assert p.pack_prefix and p.attn_plan == -1
    monkeypatch.setenv("TJ_NO_PACK", "1")
    monkeypatch.setenv("TJ_ATTN_PLAN", "1")
    monkeypatch.setenv("TJ_FFN", "gemm")
    p = plans_mod.select_plan(4, 2048, 1024, 16, 4096, 4, True, torch.bfloat16, dev)
    assert not p.pack_prefix and p.attn_plan == 1
    assert plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev).ffn == "gemm"
    monkeypatch.setenv("TJ_FFN", "fused")
    assert plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev).ffn == "fused"
    monkeypatch.setenv("TJ_ATTN_BLOCK", "1")
    assert plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev).attn_block
    monkeypatch.setenv("TJ_DEFERRED_RESIDUAL", "0")
    assert plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev).residual_epilogue
    monkeypatch.setenv("TJ_DEFERRED_RESIDUAL", "1")
    monkeypatch.setenv("TJ_LN_GEMM", "1")
    assert plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev).ln_gemm
    monkeypatch.delenv("TJ_LN_GEMM")
    # TJ_RESIDUAL_DTYPE, plans.py:183-185 of the reference
    assert plans_mod.select_plan(1, 128, 512, 8, 2048, 4, True, torch.float16, dev).residual_dtype == torch.float32
    monkeypatch.setenv("TJ_RESIDUAL_DTYPE", "float16")
    p = plans_mod.select_plan(4, 2048, 1024, 16, 4096, 4, True, torch.bfloat16, dev)
    assert p.residual_dtype == torch.float16 and not p.epilogue_residual
    assert plans_mod.Plan.from_json(p.to_json()) == p


def test_sweep_runs_cases_in_subprocesses_and_tabulates(tmp_path, monkeypatch):
    """The sweep runs each workload through bench.py in its own process and
    tabulates the JSON line; a crash or OOM in one case is recorded, not
    raised (stand-in bench scripts, no GPU)."""
    from tjkernels import sweep
    ok = tmp_path / "ok.py"
    ok.write_text("import json, os, sys\n"
                  "w = sys.argv[sys.argv.index('--workload') + 1]\n"
                  "v = 2.0 if os.environ.get('TJ_NO_GRAPH') == '1' else 1.0\n"
                  "print('noise')\n"
                  "print(json.dumps({'metric': 'm', 'value': v, 'p90_ms': v, 'tflops': 10.0, "
                  "'pct_peak': 0.4, 'tflops_padded_equiv': 12.0, 'roofline': {'kernel': 'gemm_qkv', "
                  "'achieved': 9.0, 'frac': 0.5}, 'accuracy': {'passed': True, 'max_abs': 1e-3}, "
                  "'cpu_baseline': None, 'config': {'workload': w}}))\n")
    oom = tmp_path / "oom.py"
    oom.write_text("import sys\nprint('HIP out of memory', file=sys.stderr)\nsys.exit(1)\n")
    monkeypatch.setattr(sweep, "BENCH", ok)
    r = sweep.run_case("C2", 3, 1, False, {}, 60)
    assert r["status"] == "PASS" and r["result"]["value"] == 1.0 and "--no-cpu-baseline" in r["cmd"]
    monkeypatch.setattr(sweep, "BENCH", oom)
    bad = sweep.run_case("C5", 3, 1, False, {}, 60)
    assert bad["status"] == "OOM" and "result" not in bad
    table = sweep.sweep_table([r, bad])
    assert "| C2 | PASS | 1.0000" in table and "| C5 | OOM |" in table
    monkeypatch.setattr(sweep, "BENCH", ok)
    rc = sweep.main(["--workloads", "C2", "--ablation", "C2,C3", "--steps", "2", "--warmup", "0",
                     "--out", str(tmp_path / "out"), "--tag", "t"])
    assert rc == 0
    md = list((tmp_path / "out").glob("t-*.md"))[0].read_text()
    assert "| without hipGraph capture | 2.0000 (2.00x) | 2.0000 (2.00x) |" in md


def test_mask_classification():
    cfg = TransformerConfig(2, 6, 32, 4, 64, 1, True)
    eng = Engine(UserOptimizedTransformer(cfg))
    assert eng._mask_mode(None) == MASK_NONE
    assert eng._mask_mode(torch.ones(2, 6, dtype=torch.bool)) == MASK_NONE
    prefix = torch.arange(6)[None, :] < torch.tensor([[3], [6]])
    assert eng._mask_mode(prefix) == MASK_PREFIX
    general = prefix.clone()
    general[0, 1] = False
    assert eng._mask_mode(general) == MASK_GENERAL
    assert eng._mask_info(prefix) == (MASK_PREFIX, (3, 6))
    # packing is exact without causal attention too (padded keys are excluded
    # by restricting each packed sequence to its own rows)
    cfg_nc = TransformerConfig(2, 6, 32, 4, 64, 1, False)
    eng_nc = Engine(UserOptimizedTransformer(cfg_nc))
    assert eng_nc._mask_info(prefix) == (MASK_PREFIX, (3, 6))
    assert eng_nc._mask_mode(general) == MASK_GENERAL


def test_packing_row_maps():
    """gather / scatter / cu_seqlens of the packed layout, against a
    brute-force enumeration of the valid (b, s) positions."""
    from tjkernels.engine import build_packing
    lengths, seq = (3, 0, 5, 1), 5
    pk = build_packing(lengths, seq, torch.device("cpu"))
    valid = [(b, s) for b in range(len(lengths)) for s in range(seq) if s < lengths[b]]
    assert pk.tokens == len(valid) == 9
    assert pk.gather.tolist() == [b * seq + s for b, s in valid]
    assert pk.cu_seqlens.tolist() == [0, 3, 3, 8, 9]
    expect = [-1] * (len(lengths) * seq)
    for r, (b, s) in enumerate(valid):
        expect[b * seq + s] = r
    assert pk.scatter.tolist() == expect
    # scatter inverts gather on the valid rows
    assert all(pk.scatter[g].item() == r for r, g in enumerate(pk.gather.tolist()))
    empty = build_packing((0, 0), 4, torch.device("cpu"))
    assert empty.tokens == 0 and empty.gather.numel() == 0 and (empty.scatter == -1).all()



def test_static_attention_workspace_rejects_too_many_slots():
    """tjk_flash_fwd_sched_static refuses a work list whose split slots
    exceed its static array before it makes any HIP call, so no device
    pointer is needed (NULL everywhere, no stream)."""
    lib = _lib.load()
    cap = lib.tjk_flash_sched_static_bytes()
    per_slot = lib.tjk_flash_partial_bytes(128, 1)
    too_many = cap // per_slot + 1
    assert lib.tjk_flash_partial_bytes(128, too_many) > cap
    rc = lib.tjk_flash_fwd_sched_static(None, 384, 128, 128, None, 128, 1, 128, 1, 128, 0.1, 1, None, None, 1, 1,
                                        too_many, _lib.BF16, None)
    assert rc == _lib.EUNSUPPORTED and b"static" in lib.tjk_last_error_string()

def test_graph_capture_failure_degrades_to_eager(capsys):
    cache = GraphCache()
    # capture cannot happen on the CPU; the cache records None and warns once
    g = cache.get(("k",), lambda: None, torch.device("cpu"))
    assert g is None and len(cache) == 1
    assert cache.get(("k",), lambda: None, torch.device("cpu")) is None


def test_engine_cached_on_module_without_touching_state_dict():
    cfg = TransformerConfig(1, 4, 32, 4, 64, 1, True)
    m = UserOptimizedTransformer(cfg)
    before = set(m.state_dict())
    e = tjkernels.get_engine(m)
    assert tjkernels.get_engine(m) is e
    assert set(m.state_dict()) == before
    tjkernels.reset_engines(m)
    assert tjkernels.get_engine(m) is not e


def test_tj_disable_calls_parent_forward(monkeypatch):
    """TJ_DISABLE=1 defers to the parent class (the harness's baseline)."""
    class Parent(torch.nn.Module):
        def __init__(self, cfg):
            super().__init__()
            self.config = cfg
            self.w = torch.nn.Parameter(torch.zeros(1))

        def forward(self, x, mask=None):
            return x + 1

    class Hook(Parent):
        def forward(self, x, mask=None):
            return tjkernels.forward(self, x, mask)

    monkeypatch.setenv("TJ_DISABLE", "1")
    h = Hook(TransformerConfig(1, 2, 4, 1, 4, 1, True))
    assert torch.equal(h(torch.zeros(1, 2, 4)), torch.ones(1, 2, 4))


def test_valid_token_flops():
    """The executed-work FLOP count reduces to the padded-S formula at full
    lengths and counts each sequence's own pairs otherwise (hand count)."""
    from tjkernels.workloads import WORKLOADS, flops_per_forward, flops_valid_tokens
    for name in ("C2", "C4", "C5"):
        w = WORKLOADS[name]
        assert flops_valid_tokens(w, [w.seq] * w.batch) == flops_per_forward(w)
    w = WORKLOADS["C4"]
    d, f, L = w.d_model, w.ffn_dim, w.layers
    lens = [3, 1]
    gemm = (6 + 2) * 4 * d * d + 4 * 4 * d * f          # 4 valid rows
    attn = 4 * d * (6 + 1)                              # 3*4/2 + 1*2/2 causal pairs
    assert flops_valid_tokens(w, lens) == L * (gemm + attn)


def test_attention_schedule_covers_every_tile_once():
    """Every (sequence, head, query block, key tile) pair appears in exactly
    one work item, split items pair up (first half before second, adjacent
    key ranges), items are issued longest first, and no unsplit item exceeds
    the split target."""
    from tjkernels.schedule import BMQ, BNK, build_items
    for causal in (True, False):
        lengths, heads, slots = [1380, 1710, 0, 1054, 1, 129], 3, 100
        work, n_slots = build_items(lengths, heads, causal, slots, split_factor=1.0)
        seen = {}
        for cost, bh, qb, lo, hi, slot in work:
            assert hi - lo == cost and cost > 0
            for t in range(lo, hi):
                key = (bh, qb, t)
                assert key not in seen
                seen[key] = slot
        expect = set()
        for b, n in enumerate(lengths):
            for qb in range((n + BMQ - 1) // BMQ):
                kend = min((qb + 1) * BMQ, n) if causal else n
                for t in range((kend + BNK - 1) // BNK):
                    for h in range(heads):
                        expect.add((b * heads + h, qb, t))
        assert set(seen) == expect
        costs = [w[0] for w in work]
        assert costs == sorted(costs, reverse=True)
        total = sum(costs)
        target = max(total / slots, 6)
        assert all(w[0] <= target for w in work if w[5] == -1), "an item above the target was not split"
        assert n_slots > 0 or not causal
        for s_ in range(n_slots):
            first = [i for i, w in enumerate(work) if w[5] == s_]
            second = [i for i, w in enumerate(work) if w[5] == -2 - s_]
            assert len(first) == 1 and len(second) == 1
            a, b = work[first[0]], work[second[0]]
            assert first[0] < second[0], "a second half is issued before its first half"
            assert (a[1], a[2]) == (b[1], b[2]) and a[3] == 0 and a[4] == b[3]


def test_mask_memo_follows_in_place_updates(monkeypatch):
    """The classification is remembered per tensor and recomputed after an
    in-place update (the version counter moved), so a reused mask buffer
    never packs with stale lengths; an unchanged mask is classified once."""
    from tjkernels import engine as engine_mod
    cfg = TransformerConfig(2, 6, 32, 4, 64, 1, True)
    eng = Engine(UserOptimizedTransformer(cfg))
    calls = []
    real = engine_mod.classify_mask
    monkeypatch.setattr(engine_mod, "classify_mask", lambda m: calls.append(1) or real(m))
    mask = torch.arange(6)[None, :] < torch.tensor([[3], [6]])
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), mask)
    assert (info.mode, info.lengths) == (MASK_PREFIX, (3, 6))
    eng._decode_mask(torch.zeros(2, 6, 32), mask)
    assert len(calls) == 1  # memoised
    mask[0, 3] = True  # a longer prefix, written in place
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), mask)
    assert (info.mode, info.lengths) == (MASK_PREFIX, (4, 6)) and len(calls) == 2
    with torch.inference_mode():
        mask[1, 0] = False  # in-place update under inference mode: still versioned
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), mask)
    assert info.mode == MASK_GENERAL
    mask.fill_(True)
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), mask)
    assert info.mode == MASK_NONE
    # integer prefix lengths take the same memo
    lengths = torch.tensor([2, 6])
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), lengths)
    assert (info.mode, info.lengths) == (MASK_PREFIX, (2, 6))
    lengths[0] = 5
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), lengths)
    assert (info.mode, info.lengths) == (MASK_PREFIX, (5, 6))
    lengths[0] = 9  # clamped to S
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), lengths)
    assert info.mode == MASK_NONE
    # a mask created under inference mode has no version counter: it is
    # classified on every call, so an in-place update is still seen
    with torch.inference_mode():
        imask = torch.arange(6)[None, :] < torch.tensor([[3], [6]])
    assert imask.is_inference()
    calls.clear()
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), imask)
    assert (info.mode, info.lengths) == (MASK_PREFIX, (3, 6))
    with torch.inference_mode():
        imask[0, 3] = True
    _, info = eng._decode_mask(torch.zeros(2, 6, 32), imask)
    assert (info.mode, info.lengths) == (MASK_PREFIX, (4, 6)) and len(calls) == 2


def test_work_list_validation_rejects_broken_lists():
    """validate_work accepts the lists build_items makes and rejects each
    kind of corruption the kernel would otherwise run: an item outside the
    launch, a gap or an overlap in a query block's key tiles, a second half
    issued before its first half, a slot out of range or reused."""
    from tjkernels.schedule import build_items, validate_work
    lengths, heads = [300, 70, 0, 260], 2
    work, n_slots = build_items(lengths, heads, True, slots=32, min_split=2, split_factor=1.0)
    assert n_slots > 0
    good = [(bh, qb, lo, hi, slot) for _, bh, qb, lo, hi, slot in work]
    validate_work(good, lengths, heads, True, n_slots)
    first = next(i for i, w in enumerate(good) if w[4] >= 0)
    second = next(i for i, w in enumerate(good) if w[4] == -2 - good[first][4])
    whole = next(i for i, w in enumerate(good) if w[4] == -1)

    def broken(edit):
        w = [list(x) for x in good]
        edit(w)
        return [tuple(x) for x in w]

    cases = {
        "outside": broken(lambda w: w.__setitem__(whole, [len(lengths) * heads] + w[whole][1:])),
        "gap": broken(lambda w: w[whole].__setitem__(3, w[whole][3] - 1) if w[whole][3] > 1 else
                      w[whole].__setitem__(2, 1)),
        "overlap": broken(lambda w: w[second].__setitem__(2, w[second][2] - 1)),
        "order": broken(lambda w: w.insert(first, w.pop(second))),
        "slot range": broken(lambda w: w[first].__setitem__(4, n_slots)),
        "slot reuse": broken(lambda w: w.append(list(w[whole][:4]) + [w[first][4]])),
        "missing": good[:whole] + good[whole + 1:],
    }
    for name, bad in cases.items():
        with pytest.raises(ValueError):
            validate_work(bad, lengths, heads, True, n_slots)


def test_attention_lists_balance_items_and_head_split_halves():
    """pack_lists deals every item of build_items' list exactly once into
    n_lists lists laid out item-major (item j of list w at j * n_lists + w,
    HOLE padding), first halves of split items at list heads, largest cost
    first into the least-loaded list: no list ends more than one item's cost
    above the lightest (the LPT bound), and at the C4 lengths the heaviest
    list is the longest single item.  validate_work accepts the layout and
    rejects a first half moved off a list head."""
    from tjkernels.schedule import HOLE, ITEM_OVERHEAD, build_items, pack_lists, validate_work
    for lengths, heads, slots, n_lists, split in (([1380, 1710, 1054, 1286], 16, 512, 512, 2.0),
                                                  ([300, 70, 0, 260, 129, 1], 3, 32, 16, 1.0)):
        work, n_slots = build_items(lengths, heads, True, slots, min_split=2, split_factor=split)
        assert (n_slots > 0) == (n_lists == 16)
        laid = pack_lists(work, n_lists)
        assert len(laid) % n_lists == 0
        items = [w for w in laid if w != HOLE]
        assert sorted(items) == sorted(w[1:] for w in work)
        validate_work(laid, lengths, heads, True, n_slots, n_lists)
        heads_ = [laid[i] for i in range(n_lists)]
        assert {w[1:] for w in work if w[5] >= 0} <= set(heads_)
        load = [0] * n_lists
        last = [0] * n_lists
        for j, w in enumerate(laid):
            if w != HOLE:
                load[j % n_lists] += w[3] - w[2] + ITEM_OVERHEAD
                last[j % n_lists] = w[3] - w[2] + ITEM_OVERHEAD
        assert all(load[i] - last[i] <= min(load) for i in range(n_lists)), "an item went to a heavier list"
        if n_slots == 0:
            assert max(load) == max(w[0] for w in work) + ITEM_OVERHEAD
        if n_slots:
            first = next(j for j in range(n_lists) if laid[j][4] >= 0)
            moved = list(laid)
            moved[first], moved[first + n_lists] = moved[first + n_lists], moved[first]
            with pytest.raises(ValueError):
                validate_work(moved, lengths, heads, True, n_slots, n_lists)
    work, n_slots = build_items([300, 260], 2, True, 8, min_split=2, split_factor=0.5)
    assert n_slots == 8
    with pytest.raises(ValueError):  # more split items than lists
        pack_lists(work, 7)


def test_gemm_tile_classes_follow_the_library_table():
    """Each timed candidate set holds plans of one K order only (the same
    k_groups in the library's own table), and the class is a function of the
    shape alone -- so the timed choice cannot change results."""
    from tjkernels import ops, tiles
    info = {pid: kg for pid, _, _, _, kg in ops.gemm_plans(torch.bfloat16)}
    for cls, cands in tiles.CLASS_TILES_16.items():
        assert {info[c] for c in cands} == {cls}
    for (m, n, k) in [(128, 1536, 512), (128, 512, 2048), (2442, 768, 3072), (5430, 4096, 1024),
                      (5430, 1024, 4096), (8192, 3072, 1024)]:
        cls = tiles.k_class(m, n, k, torch.bfloat16)
        assert cls == tiles.k_class(m, n, k, torch.bfloat16)
        assert set(tiles.candidates(m, n, k, torch.bfloat16)) == set(tiles.CLASS_TILES_16[cls])
    assert tiles.k_class(128, 512, 2048, torch.bfloat16) == 4   # C2 FFN2: launch-bound, long K
    assert tiles.k_class(128, 1536, 512, torch.bfloat16) == 2   # C2 QKV
    assert tiles.k_class(2442, 768, 3072, torch.bfloat16) == 2  # C3 FFN2
    assert tiles.k_class(5430, 4096, 1024, torch.bfloat16) == 1  # C4 FFN1
    assert tiles.candidates(96, 512, 128, torch.float32) == tiles.CANDIDATES_32


def test_rocprof_summary_groups_forwards_by_rows_and_kernels(tmp_path):
    """The profile summarizer labels each launch of a forward by position
    and keeps forwards of the same rows through different kernels (the
    bench's timed forward and its masked comparison run) in separate
    groups, with per-label averages over each group's forwards only."""
    from tjkernels import rocprof_summary as rs
    names = {
        "ln_first": "_ZN3tjk20add_layernorm_kernelIDF16bDF16bDF16bLi4ELb1EE",
        "gemm_qkv": "_ZN3tjk15gemm_dtl_kernelIDF16bLi192ELi384EE",
        "gemm_out_residual": "_ZN3tjk15gemm_dtl_kernelIDF16bLi96ELi128EE",
        "add_layernorm": "_ZN3tjk20add_layernorm_kernelIffDF16bLi4ELb1EE",
        "gemm_ffn1_gelu": "_ZN3tjk15gemm_dtl_kernelIDF16bLi192ELi128EE",
        "gemm_ffn2_residual": "_ZN3tjk15gemm_dtl_kernelIDF16bLi192ELi128EE",
        "ln_final": "_ZN3tjk20add_layernorm_kernelIffDF16bLi4ELb1EE",
    }
    rows, t = [], 0
    for attn, dur in (("_ZN3tjk17flash_pipe_kernelIDF16bLi64E", 10), ("_ZN3tjk16flash_fwd_kernelIDF16bLi64E", 30),
                      ("_ZN3tjk17flash_pipe_kernelIDF16bLi64E", 12)):
        for lab in rs._labels(1):
            name = attn if lab == "flash_attention" else names[lab]
            d = dur if lab == "flash_attention" else 5
            rows.append({"Kernel_Name": name, "Start_Timestamp": str(t), "End_Timestamp": str(t + d * 1000),
                         "Grid_Size_X": "4096", "Workgroup_Size_X": "256"})
            t += d * 1000 + 100
    trace = tmp_path / "k_kernel_trace.csv"
    with open(trace, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = rs.summarize(str(trace), layers=1)
    blocks = [b for b in out.split("\n\n") if b.startswith("forward group")]
    assert len(blocks) == 2
    pipe = next(b for b in blocks if "flash_pipe" in b)
    masked = next(b for b in blocks if "flash_fwd" in b)
    assert "2 forwards" in pipe and "1 forwards" in masked
    attn_line = next(line for line in pipe.splitlines() if line.startswith("flash_attention"))
    assert float(attn_line.split()[2]) == 11.0  # (10 + 12) / 2, the masked run's 30 kept out


def test_tile_choices_describe_both_gemm_kinds(monkeypatch):
    """bench.py reports the measured tiles of the plain and the LayerNorm
    GEMMs together, in shape order."""
    from tjkernels import tiles
    monkeypatch.setattr(tiles, "_choice", tiles.OrderedDict())
    tiles._choice[(128, 1536, 512, torch.float16, 0)] = 22
    tiles._choice[("ln", 128, 2048, 512, torch.float16, 1)] = 1
    tiles._choice[(64, 512, 512, torch.float16, 2)] = 24
    assert list(tiles.describe().items()) == [("64x512x512/epi2", 24), ("128x1536x512/epi0", 22),
                                              ("ln:128x2048x512/epi1", 1)]


def test_rocprof_summary_labels_deferred_projections():
    """Out-proj / FFN2 launches without the residual epilogue (EPI 0) are
    labelled by what they are."""
    from tjkernels import rocprof_summary as rs
    epi2 = "_ZN3tjk15gemm_dtl_kernelIDF16bLi192ELi128ELi2ELi2ELi128ELi4ELi2ELi1EEEvPKT_lS3_lS3_Pvliii"
    epi0 = "_ZN3tjk15gemm_dtl_kernelIDF16bLi96ELi128ELi1ELi4ELi128ELi2ELi0ELi1EEEvPKT_lS3_lS3_Pvliii"
    assert rs._gemm_epilogue(epi2) == 2 and rs._gemm_epilogue(epi0) == 0
    assert rs._relabel("gemm_ffn2_residual", epi2) == "gemm_ffn2_residual"
    assert rs._relabel("gemm_out_residual", epi0) == "gemm_out"
    assert rs._relabel("gemm_qkv", epi0) == "gemm_qkv"
    # the wave-specialized kernel <T, BM, BN, WM, WN, STAGES, L, EPI> counts as a GEMM launch too
    ws2 = "_ZN3tjk14gemm_ws_kernelIDF16bLi192ELi128ELi2ELi4ELi4ELi4ELi2EEEvPKT_lS3_lS3_Pvliii"
    assert rs._gemm_epilogue(ws2) == 2 and rs._kind_ok("gemm_out_residual", ws2)
    assert rs._relabel("gemm_out_residual", ws2) == "gemm_out_residual" and rs._tjk(ws2)
    # the first layer's out-proj adding the input rows (EPI 4) is a residual GEMM as well
    ws4 = "_ZN3tjk14gemm_ws_kernelIDF16bLi192ELi128ELi2ELi4ELi4ELi4ELi4EEEvPKT_lS3_lS3_PvliiiNS_6ResSrcE"
    assert rs._gemm_epilogue(ws4) == 4 and rs._relabel("gemm_out_residual", ws4) == "gemm_out_residual"


def test_plan_tile_rows_round_trip_and_validation():
    """Plan.tile_rows (the row bucket the autotuner measured the gemm_*
    tiles at) survives plans.json and must be a row count >= 0."""
    from dataclasses import replace
    from tjkernels.plans import Plan
    p = replace(Plan(), gemm_qkv=14, gemm_out=30, gemm_ffn1=31, gemm_ffn2=29, tile_rows=5440, label="autotuned")
    q = Plan.from_json(json.loads(json.dumps(p.to_json())))
    assert q == p and q.tile_rows == 5440
    assert Plan.from_json({"label": "older table"}).tile_rows == 0  # entries written before the field
    with pytest.raises(ValueError, match="tile_rows"):
        replace(Plan(), tile_rows=-64).validate()
