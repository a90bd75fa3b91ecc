"""Per-kernel parity of the HIP C-ABI against the CPU oracle (fp64).

Each kernel is called through ``tjkernels.ops`` (ctypes -> libtjk.so) on
seeded inputs and compared with the oracle's fp64 result.  Tolerances are
stated per test: fp32 accumulation of exactly-representable products, then
one rounding to the output dtype.
"""

import math

import pytest
import torch

from oracle import model as oracle
from tjkernels import ops

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
# one rounding of an O(1) value in the output dtype, plus fp32 accumulation noise
OUT_RTOL = {torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _close(got, ref, rtol, atol):
    got = got.double().cpu()
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = ~(err <= bound)
    assert not bad.any(), (f"{int(bad.sum())}/{bad.numel()} elements off; "
                           f"max err {float(err.max()):.3e}")


# ------------------------------------------------------------------ LayerNorm

@pytest.mark.parametrize("n", [96, 128, 512, 768, 1024, 1536, 2048, 8192])
@pytest.mark.parametrize("res_dt,delta_dt,out_dt", [
    ("f32", None, "bf16"), ("bf16", None, "bf16"), ("f32", "bf16", "bf16"),
    ("f32", "f16", "f16"), ("f16", None, "f16"), ("f32", "f32", "f32"), ("f32", None, "f32"),
])
def test_add_layernorm(device, n, res_dt, delta_dt, out_dt):
    rows = 37
    g = _gen(n)
    res = (torch.randn(rows, n, generator=g) * 3 + 0.5).to(DT[res_dt])
    delta = None if delta_dt is None else torch.randn(rows, n, generator=g).to(DT[delta_dt])
    gamma = torch.randn(n, generator=g)
    beta = torch.randn(n, generator=g)
    mask = torch.rand(rows, generator=g) > 0.3
    x = res.double() + (0 if delta is None else delta.double())
    ref = oracle.layer_norm(x, gamma.double(), beta.double(), 1e-5)
    ref = ref.masked_fill(~mask[:, None], 0.0)

    res_d = res.to(device)
    out = torch.empty(rows, n, dtype=DT[out_dt], device=device)
    res_out = torch.empty(rows, n, dtype=torch.float32, device=device)
    ops.add_layernorm(res_d, None if delta is None else delta.to(device), gamma.to(device),
                      beta.to(device), 1e-5, out, res_out=res_out, row_mask=mask.to(device))
    torch.cuda.synchronize()
    # residual: one fp32 add, bit-exact
    want = res.float() + (0 if delta is None else delta.float())
    assert torch.equal(res_out.cpu(), want)
    _close(out, ref, OUT_RTOL[DT[out_dt]], 1e-5 if out_dt == "f32" else 4e-3)
    # padded rows are exact zeros
    assert (out.cpu()[~mask] == 0).all()


def test_add_layernorm_in_place_and_closed_forms(device):
    n, rows = 1024, 8
    gamma = torch.ones(n, device=device)
    beta = torch.full((n,), 0.25, device=device)
    # constant rows normalise to beta
    res = torch.full((rows, n), 3.0, device=device)
    out = torch.empty(rows, n, device=device)
    ops.add_layernorm(res, None, gamma, beta, 1e-5, out)
    assert torch.allclose(out, torch.full_like(out, 0.25), atol=1e-6)
    # in place: res_out aliases res
    g = _gen(5)
    r0 = torch.randn(rows, n, generator=g)
    d0 = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    res = r0.to(device)
    ops.add_layernorm(res, d0.to(device), gamma, torch.zeros(n, device=device), 1e-5, out, res_out=res)
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), r0 + d0.float())
    o = out.double().cpu()
    assert torch.allclose(o.mean(-1), torch.zeros(rows, dtype=torch.double), atol=1e-5)
    assert torch.allclose((o * o).mean(-1), torch.ones(rows, dtype=torch.double), atol=1e-4)


# ----------------------------------------------------------------------- GEMM

def _gemm_case(device, m, n, k, dt, epi, plan, seed=0):
    g = _gen(seed + m + 7 * n + 13 * k)
    a = torch.randn(m, k, generator=g).to(dt)
    w = (torch.randn(n, k, generator=g) / math.sqrt(k)).to(dt)
    bias = torch.randn(n, generator=g).to(dt)
    ref = a.double() @ w.double().t() + bias.double()
    if epi == ops.EPI_BIAS_GELU:
        ref = 0.5 * ref * (1 + torch.erf(ref / math.sqrt(2)))
    if epi == ops.EPI_BIAS_RESIDUAL:
        r0 = torch.randn(m, n, generator=g)
        out = r0.to(device)
        ref = ref + r0.double()
    else:
        out = torch.full((m, n), float("nan"), dtype=dt, device=device)
    ops.gemm(a.to(device), w.to(device), bias.to(device), out, epi, plan)
    torch.cuda.synchronize()
    rtol = 2e-5 if (dt == torch.float32 or epi == ops.EPI_BIAS_RESIDUAL) else OUT_RTOL[dt]
    _close(out, ref, rtol, 1e-4 if dt != torch.float32 else 1e-5)


# Plans of the staged kernel take any K % 8 == 0; direct-to-LDS plans need
# K % 64 == 0 (bf16/fp16) and reject other K with TJK_EUNSUPPORTED.
# Plans 18-20 use 4-, 8- and 6-slot rings with the spread DMA schedule;
# 16, 17 and 21-27 split K between 2 or 4 wave groups of one workgroup.
STAGED16, DTL16, DTL16_K32 = range(0, 6), list(range(6, 33)), ()
STAGED32, DTL32 = range(0, 2), range(2, 5)


@pytest.mark.parametrize("plan", list(STAGED16) + list(DTL16))
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_gemm_plans(device, plan, dt):
    # ragged M and N (not tile multiples)
    _gemm_case(device, 513, 1028, 1088, dt, ops.EPI_BIAS, plan)
    _gemm_case(device, 64, 32, 64, dt, ops.EPI_BIAS, plan)
    if plan in STAGED16 or plan in DTL16_K32:  # K = 96 is a multiple of 32, not of 64
        _gemm_case(device, 300, 200, 96, dt, ops.EPI_BIAS, plan)
    else:
        with pytest.raises(ops.TjkError, match="needs k"):
            _gemm_case(device, 300, 200, 96, dt, ops.EPI_BIAS, plan)
    if plan in DTL16_K32:
        with pytest.raises(ops.TjkError, match="needs k"):
            _gemm_case(device, 64, 64, 40, dt, ops.EPI_BIAS, plan)


@pytest.mark.parametrize("plan", [15, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31, 32])
@pytest.mark.parametrize("epi", [ops.EPI_BIAS_GELU, ops.EPI_BIAS_RESIDUAL])
def test_gemm_deep_ring_and_prefetch_plans(device, plan, epi):
    # Deep rings (18-20): K from one tile (fewer tiles than ring slots) to a
    # long pipeline.  Plans 15 and 18 read the residual before the main loop,
    # the small K-split tiles (22-27) the residual and the bias.  K-split
    # plans (21-27): fewer K tiles than groups, and counts that do not divide
    # evenly between the groups.  Wave-specialized plans (28-32): K tiles
    # fewer than, equal to and more than the ring's slots, so the loader
    # waves' tail (no further tile to issue) runs at every ring depth.
    for m, n, k in ((200, 256, 64), (300, 384, 192), (5430, 1024, 4096), (1000, 516, 1024), (128, 512, 2048)):
        _gemm_case(device, m, n, k, torch.bfloat16, epi, plan)


@pytest.mark.parametrize("epi", [ops.EPI_BIAS, ops.EPI_BIAS_GELU, ops.EPI_BIAS_RESIDUAL])
def test_gemm_k_order_classes_are_bitwise_identical(device, epi):
    """Tiles of one K-summation class (tjkernels.tiles) produce the same bits,
    so the run-time tile timing cannot change results; the two classes
    differ only in the last bits."""
    from tjkernels import tiles
    g = _gen(11)
    for m, n, k in ((5430, 1024, 4096), (128, 512, 2048), (700, 256, 1024)):
        a = torch.randn(m, k, generator=g).bfloat16().to(device)
        w = (torch.randn(n, k, generator=g) / math.sqrt(k)).bfloat16().to(device)
        b = torch.randn(n, generator=g).bfloat16().to(device)
        r0 = torch.randn(m, n, generator=g).to(device)
        for cls, plans in tiles.CLASS_TILES_16.items():
            outs = []
            for plan in plans:
                if epi == ops.EPI_BIAS_RESIDUAL:
                    out = r0.clone()
                else:
                    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
                ops.gemm(a, w, b, out, epi, plan)
                outs.append(out)
            torch.cuda.synchronize()
            for plan, out in zip(plans[1:], outs[1:]):
                assert torch.equal(out, outs[0]), f"class {cls}: plan {plan} differs from plan {plans[0]}"


@pytest.mark.parametrize("epi", [ops.EPI_BIAS, ops.EPI_BIAS_GELU, ops.EPI_BIAS_RESIDUAL])
@pytest.mark.parametrize("plan", [9, 14, 16, 21, 29])
def test_gemm_write_through_launch_equals_plain(device, epi, plan):
    """A launch whose output reaches 4 MiB stores it written through the L2
    (cache policy sc1), a smaller one with plain stores.  Rows do not depend
    on the launch's other rows, so with the tile plan fixed the first rows of
    a 2112-row launch (4.1 MiB of bf16, 8.3 MiB of fp32) are bitwise those of
    a 1000-row one (2.0 / 3.9 MiB); the large launch also against fp64."""
    n, k, big, small = 1024, 512, 2112, 1000
    g = _gen(23 + plan)
    a = torch.randn(big, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) / math.sqrt(k)).bfloat16()
    b = torch.randn(n, generator=g).bfloat16()
    r0 = torch.randn(big, n, generator=g)
    outs = []
    for m in (big, small):
        if epi == ops.EPI_BIAS_RESIDUAL:
            out = r0[:m].to(device)
        else:
            out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
        ops.gemm(a[:m].to(device), w.to(device), b.to(device), out, epi, plan)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0][:small], outs[1])
    ref = a.double() @ w.double().t() + b.double()
    if epi == ops.EPI_BIAS_GELU:
        ref = 0.5 * ref * (1 + torch.erf(ref / math.sqrt(2)))
    if epi == ops.EPI_BIAS_RESIDUAL:
        ref = ref + r0.double()
    rtol = 2e-5 if epi == ops.EPI_BIAS_RESIDUAL else OUT_RTOL[torch.bfloat16]
    _close(outs[0], ref, rtol, 1e-4)


@pytest.mark.parametrize("dt,plan", [(torch.bfloat16, p) for p in list(STAGED16) + list(DTL16)]
                         + [(torch.float16, p) for p in (0, 8, 14, 23, 30, 31)]
                         + [(torch.float32, p) for p in list(STAGED32) + list(DTL32)])
def test_gemm_residual_from_equals_residual_over_gathered_rows(device, dt, plan):
    """tjk_gemm_bias_residual_from (residual read from x through a row map,
    the out-projection of the first layer) equals, bit for bit, the residual
    epilogue over an fp32 copy of the gathered rows -- the residual the first
    LayerNorm would write -- with and without a row map, with and without
    the residual prefetch (small and large tiles), on ragged shapes; and the
    sum against fp64."""
    for m, n, k, x_rows in ((513, 1028, 1088, 700), (1000, 516, 1024, 1000), (200, 256, 64, 333)):
        g = _gen(31 + plan + m)
        a = torch.randn(m, k, generator=g).to(dt)
        w = (torch.randn(n, k, generator=g) / math.sqrt(k)).to(dt)
        b = torch.randn(n, generator=g).to(dt)
        x = torch.randn(x_rows, n, generator=g).to(dt)
        maps = [torch.randperm(x_rows, generator=g)[:m].int() if x_rows >= m
                else torch.randint(0, x_rows, (m,), generator=g).int()]
        if x_rows >= m:
            maps.append(None)
        for rows in maps:
            gathered = (x if rows is None else x[rows.long()])[:m].float()
            want = gathered.to(device)
            got = torch.full((m, n), float("nan"), device=device)
            ad, wd, bd = a.to(device), w.to(device), b.to(device)
            ops.gemm(ad, wd, bd, want, ops.EPI_BIAS_RESIDUAL, plan)
            ops.gemm_residual_from(ad, wd, bd, got, x.to(device), None if rows is None else rows.to(device),
                                   plan=plan)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"plan {plan} {m}x{n}x{k} map={rows is not None}"
            ref = a.double() @ w.double().t() + b.double() + gathered.double()
            _close(got, ref, 2e-5, 1e-4 if dt != torch.float32 else 1e-5)


def test_gemm_residual_from_rows_outside_x_add_zeros_and_are_counted(device):
    """Row-map entries outside [0, x_rows) (negative, or at / past x_rows)
    add zeros, read nothing outside x and are counted once each in
    index_errors; the other rows are unaffected."""
    m, n, k, x_rows = 300, 512, 256, 260
    g = _gen(5)
    a = torch.randn(m, k, generator=g).bfloat16().to(device)
    w = (torch.randn(n, k, generator=g) / math.sqrt(k)).bfloat16().to(device)
    b = torch.randn(n, generator=g).bfloat16().to(device)
    x = torch.randn(x_rows, n, generator=g).bfloat16()
    rows = torch.randint(0, x_rows, (m,), generator=g).int()
    bad = torch.tensor([0, 7, 64, 65, 299])
    rows[bad] = torch.tensor([-1, x_rows, x_rows + 5, -7, 1 << 30], dtype=torch.int32)
    for plan in (0, 9, 30):
        errors = torch.zeros(1, dtype=torch.int32, device=device)
        got = torch.full((m, n), float("nan"), device=device)
        ops.gemm_residual_from(a, w, b, got, x.to(device), rows.to(device), index_errors=errors, plan=plan)
        want = x[rows.long().clamp(0, x_rows - 1)].float()
        want[bad] = 0
        want = want.to(device)
        ops.gemm(a, w, b, want, ops.EPI_BIAS_RESIDUAL, plan)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"plan {plan}"
        assert int(errors.item()) == len(bad), f"plan {plan}: {int(errors.item())} errors counted"
        # an x with no rows: every row adds zeros and is counted
        errors.zero_()
        xd = x.to(device)
        got = torch.full((m, n), float("nan"), device=device)
        ops.gemm_residual_from(a, w, b, got, xd[:0], rows.to(device), index_errors=errors, plan=plan)
        want = torch.zeros(m, n, device=device)
        ops.gemm(a, w, b, want, ops.EPI_BIAS_RESIDUAL, plan)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"plan {plan}, empty x"
        assert int(errors.item()) == m, f"plan {plan}, empty x: {int(errors.item())} errors counted"


@pytest.mark.parametrize("plan", list(STAGED32) + list(DTL32))
def test_gemm_fp32_plans(device, plan):
    _gemm_case(device, 257, 516, 256, torch.float32, ops.EPI_BIAS, plan)
    if plan in STAGED32:
        _gemm_case(device, 300, 200, 96, torch.float32, ops.EPI_BIAS, plan)


@pytest.mark.parametrize("epi", [ops.EPI_BIAS_GELU, ops.EPI_BIAS_RESIDUAL])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_gemm_epilogues(device, epi, dt):
    _gemm_case(device, 256, 384, 512, dt, epi, -1)
    _gemm_case(device, 200, 388, 96, dt, epi, -1)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_gemm_gelu_accuracy_sweep(device, dt):
    """The GELU epilogue over v in [-12, 12] (plus 0 and tiny values), each
    value passed through the GEMM exactly (A = e_0, W[n, 0] = v_n), against
    0.5 v (1 + erf(v / sqrt 2)) in fp64 (math.erf): within 8e-7 absolute plus
    two fp32 ulps for fp32, one output rounding for bf16."""
    vals = torch.cat([torch.linspace(-12, 12, 4001), torch.tensor([0.0, 1e-6, -1e-6, 1e-30, -3.5, 3.5])])
    n = (vals.numel() + 3) // 4 * 4
    v = torch.zeros(n)
    v[:vals.numel()] = vals
    v = v.to(dt)  # the values the GEMM sees
    a = torch.zeros(64, 64, dtype=dt)
    a[:, 0] = 1
    w = torch.zeros(n, 64, dtype=dt)
    w[:, 0] = v
    out = torch.empty(64, n, dtype=dt, device=device)
    ops.gemm(a.to(device), w.to(device), None, out, ops.EPI_BIAS_GELU)
    torch.cuda.synchronize()
    x = v.double()
    ref = torch.tensor([0.5 * t * (1 + math.erf(t / math.sqrt(2))) for t in x.tolist()], dtype=torch.float64)
    got = out[0].cpu().double()
    if dt == torch.float32:
        bound = 8e-7 + 2.4e-7 * ref.abs()
    else:
        bound = 8e-7 + 2 ** -8 * ref.abs()
    err = (got - ref).abs()
    assert bool((err <= bound).all()), f"max err {float(err.max()):.3e} at v={float(x[err.argmax()]):.4f}"
    assert torch.equal(out[1:].cpu(), out[:1].cpu().expand(63, n))


def test_gemm_headline_shapes(device):
    # the four C4 projections at full size, against fp64 on the CPU
    for (m, n, k) in [(8192, 3072, 1024), (8192, 1024, 1024), (8192, 4096, 1024), (8192, 1024, 4096)]:
        _gemm_case(device, m, n, k, torch.bfloat16, ops.EPI_BIAS, -1)


def test_gemm_zero_weight_gives_bias(device):
    a = torch.randn(64, 128, device=device, dtype=torch.bfloat16)
    w = torch.zeros(256, 128, device=device, dtype=torch.bfloat16)
    b = torch.randn(256, device=device, dtype=torch.bfloat16)
    out = torch.empty(64, 256, device=device, dtype=torch.bfloat16)
    ops.gemm(a, w, b, out)
    assert torch.equal(out, b.expand(64, 256))


@pytest.mark.parametrize("out_dt", ["bf16", "f32"])
def test_add_layernorm_gather_scatter(device, out_dt):
    """row_index: output row r is LN(res[row_index[r]]), zeros where the index
    is negative -- the packing (gather) and unpacking (scatter) of prefix
    masked tokens."""
    n, rows = 768, 40
    g = _gen(5)
    x = (torch.randn(rows, n, generator=g) * 2).to(torch.bfloat16)
    gamma, beta = torch.randn(n, generator=g), torch.randn(n, generator=g)
    ref_all = oracle.layer_norm(x.double(), gamma.double(), beta.double(), 1e-5)
    gather = torch.tensor([3, 4, 5, 17, 0, 39, 38, 20, 21], dtype=torch.int32)
    out = torch.full((gather.numel(), n), float("nan"), dtype=DT[out_dt], device=device)
    res_out = torch.full((gather.numel(), n), float("nan"), dtype=torch.float32, device=device)
    ops.add_layernorm(x.to(device), None, gamma.to(device), beta.to(device), 1e-5, out,
                      res_out=res_out, row_index=gather.to(device))
    torch.cuda.synchronize()
    assert torch.equal(res_out.cpu(), x.float()[gather.long()])
    _close(out, ref_all[gather.long()], OUT_RTOL[DT[out_dt]], 1e-5 if out_dt == "f32" else 4e-3)
    # scatter: 12 output rows from 5 packed rows, holes are exact zeros
    packed = res_out[:5].contiguous()
    scatter = torch.tensor([-1, 0, 1, -1, -1, 2, 3, 4, -1, -1, -1, -1], dtype=torch.int32)
    out2 = torch.full((scatter.numel(), n), float("nan"), dtype=DT[out_dt], device=device)
    ops.add_layernorm(packed, None, gamma.to(device), beta.to(device), 1e-5, out2,
                      row_index=scatter.to(device))
    torch.cuda.synchronize()
    got = out2.cpu()
    hole = scatter < 0
    assert (got[hole] == 0).all()
    src = gather[:5].long()[scatter[~hole].long()]
    _close(got[~hole], ref_all[src], OUT_RTOL[DT[out_dt]], 1e-5 if out_dt == "f32" else 4e-3)
    # an in-place residual update cannot be a gather
    with pytest.raises(ops.TjkError):
        r = torch.zeros(8, n, device=device)
        ops.add_layernorm(r, None, gamma.to(device), beta.to(device), 1e-5,
                          torch.empty(8, n, device=device), res_out=r,
                          row_index=torch.arange(8, dtype=torch.int32, device=device))



@pytest.mark.parametrize("case", ["delta", "gather", "scatter", "split", "two_byte"])
def test_add_layernorm_write_through_launch_equals_plain(device, case):
    """A LayerNorm launch whose normalised output reaches 4 MiB is the
    write-through instantiation (stores with cache policy sc1, gamma / beta
    loaded before the row); a smaller one the plain instantiation.  Each
    output row depends on its own input row only, so the first rows of a
    2176-row launch (4.25 MiB of bf16 at n = 1024; fp32 output: 8.5 MiB) are
    bitwise those of a 600-row one; the large launch also against fp64.
    Covers the row kernel (delta, row mask, fp32 and 2-byte residual
    output, gather and scatter with holes) and the split-delta kernel."""
    n, big, small = 1024, 2176, 600
    g = _gen(31)
    gamma, beta = torch.randn(n, generator=g).to(device), torch.randn(n, generator=g).to(device)
    res = (torch.randn(big, n, generator=g) * 2).to(device)
    delta = torch.randn(big, n, generator=g).bfloat16().to(device)
    parts = torch.randn(8, big, n, generator=g).to(device)
    mask = (torch.rand(big, generator=g) > 0.2).to(device)
    index = torch.randperm(big, generator=g).to(torch.int32)
    index[::7] = -1
    index = index.to(device)
    out_dt = torch.float32 if case == "gather" else torch.bfloat16

    def run(m):
        out = torch.full((m, n), float("nan"), dtype=out_dt, device=device)
        ro = None
        if case == "delta":
            ro = torch.empty(m, n, device=device)
            ops.add_layernorm(res[:m], delta[:m], gamma, beta, 1e-5, out, res_out=ro, row_mask=mask[:m])
        elif case == "gather":
            ro = torch.empty(m, n, device=device)
            ops.add_layernorm(res.bfloat16(), None, gamma, beta, 1e-5, out, res_out=ro,
                              row_index=index[:m].clamp(min=0))
        elif case == "scatter":
            ops.add_layernorm(res, None, gamma, beta, 1e-5, out, row_index=index[:m])
        elif case == "split":
            ro = res[:m].clone()
            ops.add_layernorm(ro, parts[:, :m], gamma, beta, 1e-5, out, res_out=ro)
        else:  # two_byte: bf16 residual stream in and out
            ro = torch.empty(m, n, dtype=torch.bfloat16, device=device)
            ops.add_layernorm(res[:m].bfloat16(), delta[:m], gamma, beta, 1e-5, out, res_out=ro)
        return out, ro

    (ob, rb), (os_, rs) = run(big), run(small)
    torch.cuda.synchronize()
    assert torch.equal(ob[:small], os_)
    if rb is not None:
        assert torch.equal(rb[:small], rs)
    # the large launch against fp64
    x = res.double().cpu()
    rows = torch.arange(big)
    if case == "delta" or case == "two_byte":
        x = (res.bfloat16() if case == "two_byte" else res).double().cpu() + delta.double().cpu()
    elif case == "gather":
        rows = index.cpu().clamp(min=0).long()
        x = res.bfloat16().double().cpu()
    elif case == "scatter":
        rows = index.cpu().long()
    elif case == "split":
        x = x + parts.double().cpu().sum(0)
    ref = oracle.layer_norm(x[rows.clamp(min=0)], gamma.double().cpu(), beta.double().cpu(), 1e-5)
    if case == "delta":
        ref = ref.masked_fill(~mask.cpu()[:, None], 0.0)
    if case == "scatter":
        ref = ref.masked_fill((rows < 0)[:, None], 0.0)
        assert (ob.cpu()[rows < 0] == 0).all()
    _close(ob, ref, OUT_RTOL[out_dt], 1e-5 if out_dt == torch.float32 else 4e-3)


@pytest.mark.parametrize("split_delta", [False, True])
def test_add_layernorm_index_past_source_rows(device, split_delta):
    """A row_index entry at or past the rows the call declares for res /
    delta is not followed: that output row is written as zeros and counted
    in the error word, once per row.  The indices used still point inside
    the allocation (res is a prefix view of a larger tensor), so a broken
    bound cannot read outside it."""
    n, full, declared = 256, 24, 10
    g = _gen(17)
    base = torch.randn(full, n, generator=g).to(device)
    res = base[:declared]
    gamma, beta = torch.randn(n, generator=g).to(device), torch.randn(n, generator=g).to(device)
    delta = None
    if split_delta:
        delta = torch.randn(3, full, n, generator=g).to(device)[:, :declared]
    index = torch.tensor([0, 9, 10, 23, -1, 5, 12, 9], dtype=torch.int32, device=device)
    errors = torch.zeros(1, dtype=torch.int32, device=device)
    out = torch.full((index.numel(), n), float("nan"), dtype=torch.float32, device=device)
    for _ in range(2):
        ops.add_layernorm(res, delta, gamma, beta, 1e-5, out, row_index=index, index_errors=errors)
    torch.cuda.synchronize()
    assert errors.item() == 2 * 3  # entries 10, 23 and 12, on each of the two calls
    got, idx = out.cpu(), index.cpu()
    bad = idx >= declared
    assert (got[bad] == 0).all() and (got[idx < 0] == 0).all()
    x = res.double().cpu()
    if split_delta:
        x = x + delta.double().cpu().sum(0)
    ref = oracle.layer_norm(x, gamma.double().cpu(), beta.double().cpu(), 1e-5)
    ok = (idx >= 0) & ~bad
    _close(got[ok], ref[idx[ok].long()], OUT_RTOL[torch.float32], 1e-5)


# ------------------------------------------------------------------ attention

def _attn_ref(qkv, causal, key_mask=None):
    """fp64 brute force on [B,S,3,H,hd] (bench/test_flash.py:36-48 pattern)."""
    b, s, _, h, hd = qkv.shape
    q, k, v = (qkv[:, :, i].transpose(1, 2).double() for i in range(3))
    scores = (q @ k.transpose(-2, -1)) * hd ** -0.5
    if causal:
        scores = scores.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    if key_mask is not None:
        scores = scores.masked_fill(~key_mask[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores, -1).nan_to_num(0.0)
    return (probs @ v).transpose(1, 2).reshape(b * s, h * hd)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hd", [8, 32, 64, 128])
@pytest.mark.parametrize("seq", [1, 37, 200])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_shapes(device, dt, hd, seq, causal):
    b, h = 2, 3
    g = _gen(hd * 1000 + seq)
    qkv = torch.randn(b, seq, 3, h, hd, generator=g).to(dt)
    ref = _attn_ref(qkv, causal)
    for plan in (0, 1, 2, 3) + ((4,) if seq <= 128 else ()):
        out = torch.full((b * seq, h * hd), float("nan"), dtype=dt, device=device)
        ops.flash_attention(qkv.to(device), out, causal=causal, plan=plan)
        torch.cuda.synchronize()
        _close(out, ref, 1e-5 if dt == torch.float32 else 1e-2,
               1e-5 if dt == torch.float32 else 1e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_flash_key_mask_and_lengths(device, dt):
    b, s, h, hd = 3, 150, 2, 64
    g = _gen(77)
    qkv = torch.randn(b, s, 3, h, hd, generator=g).to(dt)
    key_mask = torch.rand(b, s, generator=g) > 0.4
    key_mask[:, 0] = True
    for causal in (True, False):
        ref = _attn_ref(qkv, causal, key_mask)
        for plan in (0, 1, 3):
            out = torch.empty(b * s, h * hd, dtype=dt, device=device)
            ops.flash_attention(qkv.to(device), out, causal=causal, key_mask=key_mask.to(device), plan=plan)
            torch.cuda.synchronize()
            _close(out, ref, 1e-5 if dt == torch.float32 else 1e-2, 1e-5 if dt == torch.float32 else 1e-2)
    lengths = torch.tensor([150, 1, 77], dtype=torch.int32)
    pm = torch.arange(s)[None, :] < lengths[:, None].long()
    ref = _attn_ref(qkv, False, pm)
    for plan in (0, 1, 3):
        out = torch.empty(b * s, h * hd, dtype=dt, device=device)
        ops.flash_attention(qkv.to(device), out, causal=False, lengths=lengths.to(device), plan=plan)
        torch.cuda.synchronize()
        _close(out, ref, 1e-5 if dt == torch.float32 else 1e-2, 1e-5 if dt == torch.float32 else 1e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hd", [8, 32, 64, 128])
def test_flash_short_sequences(device, dt, hd):
    """Plan 4 (a whole sequence of <= 128 tokens per one-wave workgroup of
    32 queries) against fp64: lengths around the 32-key blocks, causal and
    not, a per-key mask, prefix lengths, packed sequences (no row outside a
    sequence written), agreement with plan 1, and sequences over 128 tokens
    refused."""
    g = _gen(400 + hd)
    tol = 1e-5 if dt == torch.float32 else 1e-2
    h = 3
    for seq in (1, 31, 32, 33, 96, 128):
        qkv = torch.randn(2, seq, 3, h, hd, generator=g).to(dt)
        for causal in (True, False):
            ref = _attn_ref(qkv, causal)
            out = torch.full((2 * seq, h * hd), float("nan"), dtype=dt, device=device)
            ops.flash_attention(qkv.to(device), out, causal=causal, plan=4)
            out1 = torch.empty_like(out)
            ops.flash_attention(qkv.to(device), out1, causal=causal, plan=1)
            torch.cuda.synchronize()
            _close(out, ref, tol, tol)
            assert (out.float() - out1.float()).abs().max().item() <= 2 * tol + 1e-6, (seq, causal)
    # per-key mask and prefix lengths
    seq = 128
    qkv = torch.randn(3, seq, 3, h, hd, generator=g).to(dt)
    key_mask = torch.rand(3, seq, generator=g) > 0.4
    key_mask[:, 0] = True
    for causal in (True, False):
        out = torch.empty(3 * seq, h * hd, dtype=dt, device=device)
        ops.flash_attention(qkv.to(device), out, causal=causal, key_mask=key_mask.to(device), plan=4)
        torch.cuda.synchronize()
        _close(out, _attn_ref(qkv, causal, key_mask), tol, tol)
    lengths = torch.tensor([128, 1, 77], dtype=torch.int32)
    pm = torch.arange(seq)[None, :] < lengths[:, None].long()
    out = torch.empty(3 * seq, h * hd, dtype=dt, device=device)
    ops.flash_attention(qkv.to(device), out, causal=False, lengths=lengths.to(device), plan=4)
    torch.cuda.synchronize()
    _close(out, _attn_ref(qkv, False, pm), tol, tol)
    # packed sequences, including an empty one
    lens = [128, 0, 1, 77, 33]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    t = cu[-1]
    packed = torch.randn(t, 3, h, hd, generator=g).to(dt)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=device)
    for causal in (True, False):
        out = torch.full((t + 5, h * hd), 7.0, dtype=dt, device=device)
        ops.flash_attention(packed.to(device), out, causal=causal, plan=4, cu_seqlens=cu_d, max_seqlen=128)
        torch.cuda.synchronize()
        got = out.cpu()
        for b, n in enumerate(lens):
            if n:
                _close(got[cu[b]:cu[b + 1]], _attn_ref(packed[cu[b]:cu[b + 1]].unsqueeze(0), causal), tol, tol)
        assert (got[t:] == 7.0).all(), "rows past the packed tokens were written"
    # the automatic plan takes plan 4 up to 128 tokens and refuses it above
    qkv = torch.randn(1, 129, 3, h, hd, generator=g).to(dt)
    with pytest.raises(ops.TjkError):
        ops.flash_attention(qkv.to(device), torch.empty(129, h * hd, dtype=dt, device=device), plan=4)


def test_flash_closed_forms(device):
    b, s, h, hd = 2, 96, 4, 64
    qkv = torch.randn(b, s, 3, h, hd, device=device, dtype=torch.bfloat16)
    out = torch.empty(b * s, h * hd, device=device, dtype=torch.bfloat16)
    ops.flash_attention(qkv, out, causal=True)
    # causal row 0 sees only key 0: output = V_0 exactly
    v0 = qkv[:, 0, 2].reshape(b, h * hd)
    assert torch.equal(out.view(b, s, h * hd)[:, 0], v0)
    # perturbing the last key changes no earlier row
    qkv2 = qkv.clone()
    qkv2[:, -1, 1:] += 1.0
    out2 = torch.empty_like(out)
    ops.flash_attention(qkv2, out2, causal=True)
    assert torch.equal(out.view(b, s, -1)[:, :-1], out2.view(b, s, -1)[:, :-1])


@pytest.mark.parametrize("pattern", ["rising", "falling", "huge"])
def test_flash_offset_changes_across_tiles(device, pattern):
    """Scores that climb across key tiles (the running offset must be raised
    mid-sequence, repeatedly), that peak in the first tile and fall, or that
    reach |S * scale| ~ 1e3 (exp2 far outside fp32 without an offset): every
    plan against fp64, causal and not."""
    b, s, h, hd = 2, 700, 2, 64
    g = _gen({"rising": 11, "falling": 12, "huge": 13}[pattern])
    qkv = torch.randn(b, s, 3, h, hd, generator=g) * 0.5
    direction = torch.randn(h, hd, generator=g)
    direction = direction / direction.norm(dim=-1, keepdim=True)
    pos = torch.arange(s, dtype=torch.float32)[None, :, None, None]
    if pattern == "rising":    # score grows ~ +0.25 per key: +175 over the sequence
        qkv[:, :, 0] += 4.0 * direction
        qkv[:, :, 1] += (pos / 16.0) * direction
    elif pattern == "falling":  # largest scores in the first tile
        qkv[:, :, 0] += 4.0 * direction
        qkv[:, :, 1] += ((s - pos) / 16.0) * direction
    else:                      # scores of order 1e3 with both signs
        qkv[:, :, 0] *= 40.0
    qkv = qkv.to(torch.bfloat16)
    for causal in (True, False):
        ref = _attn_ref(qkv, causal)
        for plan in (0, 1, 3):
            out = torch.full((b * s, h * hd), float("nan"), dtype=torch.bfloat16, device=device)
            ops.flash_attention(qkv.to(device), out, causal=causal, plan=plan)
            torch.cuda.synchronize()
            assert torch.isfinite(out.float()).all(), (pattern, causal, plan)
            _close(out, ref, 1e-2, 2e-2)


def test_flash_packed_layout_headline(device):
    # C4 attention shape read in place from the packed QKV GEMM output
    b, s, h, hd = 4, 2048, 16, 64
    qkv = torch.randn(b * s, 3 * h * hd, device=device, dtype=torch.bfloat16)
    q5 = qkv.view(b, s, 3, h, hd)
    out = torch.empty(b * s, h * hd, device=device, dtype=torch.bfloat16)
    ops.flash_attention(q5, out, causal=True)
    torch.cuda.synchronize()
    sel = [0, 1, 63, 64, 127, 128, 777, 2047]
    ref = _attn_ref(q5[:1].cpu(), True).view(s, h * hd)
    got = out.view(b, s, h * hd)[0].cpu()
    _close(got[sel], ref[sel], 1e-2, 1e-2)
    # every plan agrees on every row
    for plan in (0, 1, 2, 3):
        out1 = torch.empty_like(out)
        ops.flash_attention(q5, out1, causal=True, plan=plan)
        torch.cuda.synchronize()
        assert (out.float() - out1.float()).abs().max().item() < 2e-2


def _attn_rows_ref(q, k, v, rows, causal):
    """fp64 attention of selected query rows of one (sequence, head): q, k, v
    [S, hd] on the CPU; memory O(S) per row, so it scales to S = 100000."""
    hd = q.shape[-1]
    out = []
    for i in rows:
        n = i + 1 if causal else k.shape[0]
        sc = (k[:n].double() @ q[i].double()) * hd ** -0.5
        p = torch.softmax(sc, 0)
        out.append(p @ v[:n].double())
    return torch.stack(out)


@pytest.mark.parametrize("causal", [True, False])
def test_flash_long_sequence_streams(device, causal):
    """Long-sequence streaming (the reference matrix's case 14 length,
    bench/shapes.py:67-69): S = 100000, padded [B,S,3,H,hd] and packed
    (varlen) layouts, against fp64 on sampled query rows, each computed in
    O(S) memory on the CPU.  The kernel holds O(tile) state per query block,
    so nothing of size S x S exists anywhere."""
    s, h, hd = 100000, 2, 64
    g = _gen(14 + int(causal))
    qkv = torch.randn(1, s, 3, h, hd, generator=g).to(torch.bfloat16)
    rows = [0, 1, 63, 64, 4095, 33333, 65536, 99998, 99999]
    out = torch.empty(s, h * hd, dtype=torch.bfloat16, device=device)
    ops.flash_attention(qkv.to(device), out, causal=causal)
    torch.cuda.synchronize()
    got = out.cpu().view(s, h, hd)
    for hh in range(h):
        q, k, v = (qkv[0, :, i, hh] for i in range(3))
        ref = _attn_rows_ref(q, k, v, rows, causal)
        _close(got[rows, hh], ref, 1e-2, 1e-2)
    # packed: the long sequence after a short one (rows offset by 37)
    short = torch.randn(37, 3, h, hd, generator=g).to(torch.bfloat16)
    packed = torch.cat([short, qkv[0]], 0)
    cu = torch.tensor([0, 37, 37 + s], dtype=torch.int32, device=device)
    out2 = torch.empty(37 + s, h * hd, dtype=torch.bfloat16, device=device)
    ops.flash_attention(packed.to(device), out2, causal=causal, cu_seqlens=cu, max_seqlen=s)
    torch.cuda.synchronize()
    assert (out2[37:].float() - out.float()).abs().max().item() < 2e-2
    if causal:  # the same kernel and key order per query: equal rows
        assert torch.equal(out2[37:37 + 4096], out[:4096])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_packed_sequences(device, dt, hd, causal):
    """cu_seqlens: B sequences of different lengths back to back; each must
    equal the fp64 brute force over its own rows, and no other row of the
    output may be touched."""
    lengths = [130, 0, 1, 257, 64]
    h, max_len = 2, 300
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    t = cu[-1]
    g = _gen(hd + (0 if causal else 1))
    qkv = torch.randn(t, 3, h, hd, generator=g).to(dt)
    tol = 1e-5 if dt == torch.float32 else 1e-2
    cu_d = torch.tensor(cu, dtype=torch.int32, device=device)
    for plan in (0, 1, 2, 3):
        out = torch.full((t + 7, h * hd), 7.0, dtype=dt, device=device)
        ops.flash_attention(qkv.to(device), out, causal=causal, plan=plan,
                            cu_seqlens=cu_d, max_seqlen=max_len)
        torch.cuda.synchronize()
        got = out.cpu()
        for b, n in enumerate(lengths):
            if n == 0:
                continue
            ref = _attn_ref(qkv[cu[b]:cu[b + 1]].unsqueeze(0), causal)
            _close(got[cu[b]:cu[b + 1]], ref, tol, tol)
        assert (got[t:] == 7.0).all(), "rows past the packed tokens were written"


def test_flash_packed_length_above_seq_is_clamped(device):
    """A packed sequence whose cu_seqlens length exceeds the launch's seq is
    taken as seq rows long: its first seq rows get the attention of those
    rows, the rows past them are neither read nor written.  The buffer holds
    every row cu_seqlens names, so a broken clamp stays inside it."""
    heads, hd, seq = 2, 64, 40
    cu = [0, 70, 80]  # lengths 70 (> seq) and 10
    g = _gen(23)
    qkv = torch.randn(cu[-1], 3, heads, hd, generator=g).to(torch.bfloat16)
    want0 = _attn_ref(qkv[0:seq][None], True)
    want1 = _attn_ref(qkv[70:80][None], True)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=device)
    for plan in range(5):  # every kernel: pipelined (0), grid (1-3), short (4)
        out = torch.full((cu[-1], heads * hd), 7.0, dtype=torch.bfloat16, device=device)
        ops.flash_attention(qkv.to(device), out, causal=True, cu_seqlens=cu_d, max_seqlen=seq, plan=plan)
        torch.cuda.synchronize()
        got = out.cpu().float()
        assert (got[seq:70] == 7.0).all(), plan
        assert (got[0:seq] - want0).abs().max() < 2e-2, plan
        assert (got[70:80] - want1).abs().max() < 2e-2, plan


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_scheduled(device, dt, hd, causal):
    """The scheduled kernel (work list; key-split items whose second half
    merges the first's partial) against the fp64 brute force per sequence,
    with many slots so that most items are split, and against the plain
    packed kernel.  The flags end cleared and no wait timed out."""
    from tjkernels.schedule import build_schedule
    lengths = [300, 0, 1, 129, 64, 200]
    h = 3
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    t = cu[-1]
    g = _gen(hd * 3 + int(causal))
    qkv = torch.randn(t, 3, h, hd, generator=g).to(dt)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=device)
    # split target = max(total tiles / slots, min_split): (many slots, 2)
    # splits every item of more than 2 key tiles, (1 slot, 6) splits none
    for slots, min_split in ((100000, 2), (1, 6)):
        sched = build_schedule(lengths, h, hd, causal, dt, device, slots=slots, min_split=min_split,
                               split_factor=1.0)
        assert (sched.n_slots > 0) == (min_split == 2)
        out = torch.full((t + 5, h * hd), 7.0, dtype=dt, device=device)
        ops.flash_attention_sched(qkv.to(device), out, cu_d, max(lengths), sched, causal=causal)
        torch.cuda.synchronize()
        got = out.cpu()
        for b, n in enumerate(lengths):
            if n:
                ref = _attn_ref(qkv[cu[b]:cu[b + 1]].unsqueeze(0), causal)
                _close(got[cu[b]:cu[b + 1]], ref, 1e-2, 1e-2)
        assert (got[t:] == 7.0).all(), "rows past the packed tokens were written"
        plain = torch.empty(t, h * hd, dtype=dt, device=device)
        ops.flash_attention(qkv.to(device), plain, causal=causal, plan=0, cu_seqlens=cu_d,
                            max_seqlen=max(lengths))
        torch.cuda.synchronize()
        if min_split == 6:  # no split: same kernel, same tiles, bitwise equal
            assert torch.equal(got[:t], plain.cpu())
        else:
            assert (got[:t].float() - plain.cpu().float()).abs().max().item() < 2e-2
            # the partial slots are followed by the error word and the flags
            hdp = 32 if hd <= 32 else 64 if hd <= 64 else 128
            tail = sched.partials.view(torch.int32)[sched.n_slots * 128 * (hdp + 2):].cpu()
            assert int(tail.abs().sum()) == 0, "a flag was left set or a wait timed out"
            again = torch.full((t + 5, h * hd), 7.0, dtype=dt, device=device)
            ops.flash_attention_sched(qkv.to(device), again, cu_d, max(lengths), sched, causal=causal)
            torch.cuda.synchronize()
            assert torch.equal(again.cpu(), got), "split merge is not deterministic"


@pytest.mark.parametrize("hd", [64, 128])
def test_flash_output_staging_matches_direct_stores(device, hd):
    """The direct-to-LDS kernels stage each wave's output block through LDS
    and store whole-row pieces when the output rows are 16-byte aligned
    (written through the L2 for launches of 4 MiB or more); an output view
    whose rows are only 8-byte aligned takes the direct per-lane stores.
    Both give the same bits, on the grid path (a ragged last query block:
    waves with fewer than 32 rows) and on the scheduled path, and neither
    writes outside its rows and columns."""
    from tjkernels.schedule import build_schedule
    h, dt = 4, torch.bfloat16
    g = _gen(hd + 5)
    # the second case writes 2 x 2048 x 4 x 128 x 2 bytes = 4 MiB at hd 128 (written through)
    for seqs in ((300, 77), (2048, 2048)):
        t = sum(seqs)
        qkv = torch.randn(t, 3, h, hd, generator=g).to(dt).to(device)
        cu = torch.tensor([0, seqs[0], t], dtype=torch.int32, device=device)
        sched = build_schedule(list(seqs), h, hd, True, dt, device)
        outs = {}
        for col0 in (0, 4):  # rows 16-byte aligned (staged), 8-byte aligned (direct)
            for name in ("sched", "grid"):
                buf = torch.full((t + 3, h * hd + 8), float("nan"), dtype=dt, device=device)
                view = buf[:t, col0:col0 + h * hd]
                assert (view.data_ptr() % 16 == 0) == (col0 == 0) and view.stride(0) % 8 == 0
                if name == "sched":
                    ops.flash_attention_sched(qkv, view, cu, max(seqs), sched)
                else:
                    ops.flash_attention(qkv, view, causal=True, plan=0, cu_seqlens=cu, max_seqlen=max(seqs))
                torch.cuda.synchronize()
                assert torch.isfinite(view.float()).all(), f"{name}: a row or column was not written"
                rest = buf.clone()
                rest[:t, col0:col0 + h * hd] = 0
                assert torch.isnan(rest.float()[rest != 0]).all(), f"{name}: wrote outside its output"
                outs[(name, col0)] = view.clone()
        for name in ("sched", "grid"):
            assert torch.equal(outs[(name, 0)], outs[(name, 4)]), f"{name}: staged and direct stores differ"


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hd", [64, 128])
def test_flash_scheduled_lists(device, causal, hd):
    """More items than workgroups: 16 lists (build_schedule's slots), each
    workgroup running its items back to back, with split items' first halves
    at list heads (causal: 6 splits).  Against fp64, bitwise repeatable, no
    wait timed out and every flag cleared; without splits, bitwise equal to
    one workgroup per item (the same items, the same arithmetic)."""
    from tjkernels import schedule as sched_mod
    lengths, h, dt = [1000] + [64] * 8, 2, torch.bfloat16
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    t = cu[-1]
    qkv = torch.randn(t, 3, h, hd, generator=_gen(hd + int(causal))).to(dt)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=device)
    sched = sched_mod.build_schedule(lengths, h, hd, causal, dt, device, slots=16, min_split=2,
                                     split_factor=1.0, lists=True)
    assert sched.n_lists == 16 and sched.work.shape[0] > 16
    assert (sched.n_slots == 6) == causal and (sched.n_slots == 0) == (not causal)
    outs = []
    for _ in range(2):
        out = torch.full((t, h * hd), 7.0, dtype=dt, device=device)
        ops.flash_attention_sched(qkv.to(device), out, cu_d, max(lengths), sched, causal=causal)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert sched_mod.error_count(sched) == 0
    hdp = 64 if hd <= 64 else 128
    assert int(sched.partials.view(torch.int32)[sched.n_slots * 128 * (hdp + 2):].abs().sum()) == 0
    got = outs[0].cpu()
    for b, n in enumerate(lengths):
        ref = _attn_ref(qkv[cu[b]:cu[b + 1]].unsqueeze(0), causal)
        _close(got[cu[b]:cu[b + 1]], ref, 1e-2, 1e-2)
    if not causal:
        one = sched_mod.build_schedule(lengths, h, hd, causal, dt, device, slots=100000, min_split=1 << 14)
        assert one.n_lists == 0
        per_item = torch.full((t, h * hd), 7.0, dtype=dt, device=device)
        ops.flash_attention_sched(qkv.to(device), per_item, cu_d, max(lengths), one, causal=causal)
        torch.cuda.synchronize()
        assert torch.equal(per_item, outs[0])


def test_flash_scheduled_reports_items_it_cannot_run(device):
    """Failure handling, forced from the host with lists validate_work would
    reject (written straight to the device): an item for a (b, h) outside
    the launch is dropped, an item with a slot outside [0, n_slots) writes
    NaN rows, and a second half whose first half never runs waits out its
    bounded poll, writes NaN rows and claims the flag -- each counted once
    in the error word, every kernel exiting normally."""
    from tjkernels import schedule as sched_mod
    lengths, h, hd, dt = [128, 128], 2, 64, torch.bfloat16
    t = sum(lengths)
    qkv = torch.randn(t, 3, h, hd, generator=_gen(1)).to(dt).to(device)
    cu = torch.tensor([0, 128, 256], dtype=torch.int32, device=device)
    sched = sched_mod.build_schedule(lengths, h, hd, True, dt, device)
    assert sched.n_slots == 0 and sched_mod.error_count(sched) == 0
    work = sched.work.clone()
    work[0, 0] = 99               # (b, h) outside the launch: dropped
    work[1, 3] = 5                # slot 5 with no slots: NaN rows
    bad = sched_mod.AttentionSchedule(work=work, n_slots=0, partials=sched.partials, max_item=sched.max_item,
                                      total=sched.total, error_index=sched.error_index)
    out = torch.zeros(t, h * hd, dtype=dt, device=device)
    ops.flash_attention_sched(qkv, out, cu, 128, bad, causal=True)
    torch.cuda.synchronize()
    assert sched_mod.error_count(bad) == 2
    bh1 = int(work[1, 0])
    b1, h1 = bh1 // h, bh1 % h
    rows = out[128 * b1:128 * (b1 + 1), h1 * hd:(h1 + 1) * hd]
    assert torch.isnan(rows.float()).all()
    # a lone second half (slot -2 of one slot): its wait times out
    lone = sched_mod.build_schedule(lengths, h, hd, True, dt, device, slots=100000, min_split=1,
                                    split_factor=1.0)
    assert lone.n_slots > 0
    w = lone.work.cpu()
    second = int((w[:, 3] == -2).nonzero()[0])
    only = w[second:second + 1].to(device)
    solo = sched_mod.AttentionSchedule(work=only, n_slots=lone.n_slots, partials=lone.partials, max_item=1,
                                       total=1, error_index=lone.error_index)
    out.zero_()
    ops.flash_attention_sched(qkv, out, cu, 128, solo, causal=True)
    torch.cuda.synchronize()
    assert sched_mod.error_count(solo) == 1
    flag = lone.partials.view(torch.int32)[lone.error_index + 1].item()
    assert flag == -1, "the timed-out second half claims the flag"
    bh2 = int(w[second, 0])
    b2, h2 = bh2 // h, bh2 % h
    assert torch.isnan(out[128 * b2:128 * (b2 + 1), h2 * hd:(h2 + 1) * hd].float()).all()
    # the late first half finds the claim and resets the flag for the next launch
    first = int((w[:, 3] == 0).nonzero()[0])
    late = sched_mod.AttentionSchedule(work=w[first:first + 1].to(device), n_slots=lone.n_slots,
                                       partials=lone.partials, max_item=1, total=1, error_index=lone.error_index)
    ops.flash_attention_sched(qkv, out, cu, 128, late, causal=True)
    torch.cuda.synchronize()
    assert lone.partials.view(torch.int32)[lone.error_index + 1].item() == 0


# ------------------------------------------------------------ fused FFN

def _ffn_reference(a_t, w1, b1, w2, b2, dtype):
    """fp64 FFN with the kernel's roundings: A and the GELU intermediate in
    the compute dtype (as the reference rounds its hidden activation)."""
    hdn = a_t.double() @ w1.double().t() + b1.double()
    hdn = (0.5 * hdn * (1 + torch.erf(hdn / math.sqrt(2)))).to(dtype).double()
    return hdn @ w2.double().t() + b2.double()


FFN_TOL = {torch.float32: (2e-5, 2e-5), torch.float16: (2e-3, 2e-3), torch.bfloat16: (1e-2, 1e-2)}


@pytest.mark.parametrize("dt,d,f", [(torch.float16, 512, 2048), (torch.bfloat16, 512, 2048),
                                     (torch.bfloat16, 256, 1024), (torch.float16, 128, 256),
                                     (torch.float32, 128, 512), (torch.float32, 256, 384)])
@pytest.mark.parametrize("rows", [1, 31, 96, 200])
@pytest.mark.parametrize("slice_cols", [64, 128])
def test_ffn_fused_against_fp64(device, dt, d, f, rows, slice_cols):
    """P = gelu_erf(A W1^T + b1) W2^T + b2 from h (no LayerNorm) and from
    the fp32 residual (LayerNorm in the kernel), split over f / 128 slices
    and summed, against fp64; rows past the input are never written."""
    g = _gen(d * 3 + f + rows)
    splits = f // slice_cols
    res = torch.randn(rows, d, generator=g) * 2 + 0.3
    gamma, beta = torch.randn(d, generator=g), torch.randn(d, generator=g) * 0.1
    w1 = (torch.randn(f, d, generator=g) / math.sqrt(d)).to(dt)
    b1 = (torch.randn(f, generator=g) * 0.1).to(dt)
    w2 = (torch.randn(d, f, generator=g) / math.sqrt(f)).to(dt)
    b2 = (torch.randn(d, generator=g) * 0.1).to(dt)
    dev = [t.to(device) for t in (res, gamma, beta, w1, b1, w2, b2)]
    res_d, gamma_d, beta_d, w1_d, b1_d, w2_d, b2_d = dev
    h = torch.empty(rows, d, dtype=dt, device=device)
    ops.add_layernorm(res_d, None, gamma_d, beta_d, 1e-5, h)
    rtol, atol = FFN_TOL[dt]
    outs = []
    for use_ln in (False, True):
        parts = torch.full((splits, rows + 3, d), float("nan"), device=device)
        ops.ffn(res_d if use_ln else h, w1_d, b1_d, w2_d, b2_d, parts[:, :rows], splits=splits,
                ln=(gamma_d, beta_d, 1e-5) if use_ln else None)
        torch.cuda.synchronize()
        assert torch.isnan(parts[:, rows:]).all(), "rows past the input were written"
        outs.append(parts[:, :rows].cpu())
    # the in-kernel LayerNorm equals the add+LayerNorm kernel bit for bit
    assert torch.equal(outs[0], outs[1])
    ref = _ffn_reference(h.cpu(), w1, b1, w2, b2, dt)
    _close(outs[0].double().sum(0), ref, rtol, atol)
    # a single split adds straight into the residual
    c = slice_cols
    if ops.ffn_supported(d, c, 1, dt):
        r0 = torch.randn(rows, d, generator=g)
        acc = r0.to(device)
        ops.ffn(h, w1_d[:c], b1_d[:c], w2_d[:, :c].contiguous(), b2_d, acc, splits=1, accumulate=True)
        torch.cuda.synchronize()
        ref1 = _ffn_reference(h.cpu(), w1[:c], b1[:c], w2[:, :c], b2, dt) + r0.double()
        _close(acc, ref1, rtol, atol)


def test_ffn_fused_closed_forms(device):
    """W1 = 0: the intermediate is gelu(b1), so P = gelu(b1) W2^T + b2 for
    every row; W2 = 0: P = b2 (split 0) and 0 (other splits)."""
    d, f, rows, dt = 512, 2048, 40, torch.float16
    g = _gen(3)
    h = torch.randn(rows, d, generator=g).to(dt).to(device)
    b1 = torch.randn(f, generator=g).to(dt)
    w2 = (torch.randn(d, f, generator=g) / 45).to(dt)
    b2 = torch.randn(d, generator=g).to(dt)
    parts = torch.empty(16, rows, d, device=device)
    ops.ffn(h, torch.zeros(f, d, dtype=dt, device=device), b1.to(device), w2.to(device), b2.to(device), parts,
            splits=16)
    hdn = (0.5 * b1.double() * (1 + torch.erf(b1.double() / math.sqrt(2)))).to(dt).double()
    want = (hdn @ w2.double().t() + b2.double()).expand(rows, d)
    _close(parts.sum(0), want, 2e-3, 2e-3)
    ops.ffn(h, torch.randn(f, d, dtype=dt, device=device), b1.to(device), torch.zeros(d, f, dtype=dt, device=device),
            b2.to(device), parts, splits=16)
    torch.cuda.synchronize()
    assert torch.equal(parts[0].cpu(), b2.float().expand(rows, d))
    assert (parts[1:] == 0).all()


def test_ffn_rejects_unsupported_shapes(device):
    h = torch.zeros(8, 1024, dtype=torch.bfloat16, device=device)
    w1 = torch.zeros(4096, 1024, dtype=torch.bfloat16, device=device)
    w2 = torch.zeros(1024, 4096, dtype=torch.bfloat16, device=device)
    with pytest.raises(ops.TjkError, match="unsupported"):
        ops.ffn(h, w1, None, w2, None, torch.zeros(32, 8, 1024, device=device), splits=32)


@pytest.mark.parametrize("n,splits", [(128, 4), (512, 16), (512, 3), (1024, 8), (512, 32), (96, 2)])
def test_add_layernorm_split_delta(device, n, splits):
    """A [splits, rows, n] fp32 delta is summed in the documented fixed
    order -- four consecutive groups of ceil(splits / 4) slices, each in
    slice order, then the group sums in group order -- and added to the
    residual: res_out equals that fp32 sum exactly, and the normalised
    output matches fp64; scatter rows read the delta rows of their source."""
    rows = 45
    g = _gen(n + splits)
    res = torch.randn(rows, n, generator=g)
    parts = torch.randn(splits, rows + 5, n, generator=g)[:, :rows]
    gamma, beta = torch.randn(n, generator=g), torch.randn(n, generator=g)
    q = (splits + 3) // 4
    acc = None
    for grp in range(4):
        sl = list(range(grp * q, min(grp * q + q, splits)))
        if not sl:
            continue
        part = parts[sl[0]].clone()
        for s_ in sl[1:]:
            part = part + parts[s_]
        acc = part if acc is None else acc + part
    want_res = res + acc
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=device)
    res_d = res.to(device)
    ops.add_layernorm(res_d, parts.to(device), gamma.to(device), beta.to(device), 1e-5, out, res_out=res_d)
    torch.cuda.synchronize()
    assert torch.equal(res_d.cpu(), want_res)
    ref = oracle.layer_norm(want_res.double(), gamma.double(), beta.double(), 1e-5)
    _close(out, ref, OUT_RTOL[torch.bfloat16], 4e-3)
    # scatter: output row r reads source row idx[r] (and its delta rows)
    idx = torch.tensor([3, -1, 0, 44, -1, 7], dtype=torch.int32)
    out2 = torch.empty(idx.numel(), n, dtype=torch.float32, device=device)
    ops.add_layernorm(res.to(device), parts.to(device), gamma.to(device), beta.to(device), 1e-5, out2,
                      row_index=idx.to(device))
    torch.cuda.synchronize()
    for r, src in enumerate(idx.tolist()):
        if src < 0:
            assert (out2[r] == 0).all()
        else:
            _close(out2[r:r + 1], ref[src:src + 1], 2e-5, 1e-5)


@pytest.mark.parametrize("n", [128, 1024, 1536, 2048])
@pytest.mark.parametrize("res_dt,delta_dt,ro_dt", [
    ("bf16", None, "f16"), ("f16", "f16", "f16"), ("f16", "bf16", "f16"), ("bf16", "bf16", "bf16"),
    ("f16", "f32", "f16"), ("f32", "bf16", "bf16"),
])
def test_add_layernorm_two_byte_residual(device, n, res_dt, delta_dt, ro_dt):
    """A 2-byte residual stream (the reference's residual_dtype knob): the
    stored residual is the fp32 sum res + delta rounded once to its dtype,
    bit for bit, and the output is the LayerNorm of the unrounded sum (as
    the reference's kernel normalises its fp32 x, layernorm.py:50-60)."""
    rows = 37
    g = _gen(n + 3)
    res = (torch.randn(rows, n, generator=g) * 3 + 0.5).to(DT[res_dt])
    delta = None if delta_dt is None else torch.randn(rows, n, generator=g).to(DT[delta_dt])
    gamma, beta = torch.randn(n, generator=g), torch.randn(n, generator=g)
    x32 = res.float() + (0 if delta is None else delta.float())
    ref = oracle.layer_norm(res.double() + (0 if delta is None else delta.double()), gamma.double(),
                            beta.double(), 1e-5)
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=device)
    res_out = torch.full((rows, n), float("nan"), dtype=DT[ro_dt], device=device)
    ops.add_layernorm(res.to(device), None if delta is None else delta.to(device), gamma.to(device),
                      beta.to(device), 1e-5, out, res_out=res_out)
    torch.cuda.synchronize()
    assert torch.equal(res_out.cpu(), x32.to(DT[ro_dt]))
    _close(out, ref, OUT_RTOL[torch.bfloat16], 4e-3)
    # in place (res_out aliases res) when they share the dtype
    if ro_dt == res_dt:
        res_d = res.to(device)
        ops.add_layernorm(res_d, None if delta is None else delta.to(device), gamma.to(device),
                          beta.to(device), 1e-5, out, res_out=res_d)
        torch.cuda.synchronize()
        assert torch.equal(res_d.cpu(), x32.to(DT[ro_dt]))


def test_add_layernorm_two_byte_residual_split_delta(device):
    """Split fp32 partials added to an fp16 residual in place: the fixed
    summation order, then one rounding of the stored residual."""
    n, rows, splits = 512, 33, 8
    g = _gen(99)
    res = torch.randn(rows, n, generator=g).to(torch.float16)
    parts = torch.randn(splits, rows, n, generator=g)
    gamma, beta = torch.randn(n, generator=g), torch.randn(n, generator=g)
    acc = None
    q = (splits + 3) // 4
    for grp in range(4):
        part = parts[grp * q].clone()
        for s_ in range(grp * q + 1, grp * q + q):
            part = part + parts[s_]
        acc = part if acc is None else acc + part
    x32 = res.float() + acc
    res_d = res.to(device)
    out = torch.empty(rows, n, dtype=torch.float16, device=device)
    ops.add_layernorm(res_d, parts.to(device), gamma.to(device), beta.to(device), 1e-5, out, res_out=res_d)
    torch.cuda.synchronize()
    assert torch.equal(res_d.cpu(), x32.to(torch.float16))
    ref = oracle.layer_norm(x32.double(), gamma.double(), beta.double(), 1e-5)
    _close(out, ref, OUT_RTOL[torch.float16], 1e-3)


def test_add_layernorm_rejects_cross_dtype_alias(device):
    """Writing the residual in place in another dtype (or with a row index)
    would overwrite bytes of rows other waves still read: rejected before
    any launch."""
    n, rows = 256, 4
    buf = torch.zeros(rows, n, dtype=torch.float32, device=device)
    gamma, beta = torch.ones(n, device=device), torch.zeros(n, device=device)
    out = torch.empty(rows, n, dtype=torch.float16, device=device)
    as16 = buf.view(torch.float16)[:, :n]
    with pytest.raises(ops.TjkError, match="alias"):
        ops.add_layernorm(buf, None, gamma, beta, 1e-5, out, res_out=as16)


# ------------------------------------------------- LayerNorm-prologue GEMM

@pytest.mark.parametrize("k", [256, 512, 768, 1024])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_gemm_ln_equals_layernorm_then_gemm(device, k, dt):
    """tjk_gemm_ln (LayerNorm inside the GEMM) equals tjk_add_layernorm
    followed by a class-1 GEMM plan bit for bit, for every column-tile plan
    and both epilogues, on ragged rows and columns; and matches fp64."""
    g = _gen(k + (dt == torch.float16))
    for m, n in ((128, 1536), (45, 100), (300, 2048)):
        res = torch.randn(m, k, generator=g) * 2 + 0.3
        gamma, beta = torch.randn(k, generator=g), torch.randn(k, generator=g) * 0.1
        w = (torch.randn(n, k, generator=g) / math.sqrt(k)).to(dt)
        bias = torch.randn(n, generator=g).to(dt)
        rd, gd, bd, wd, biasd = (t.to(device) for t in (res, gamma, beta, w, bias))
        h = torch.empty(m, k, dtype=dt, device=device)
        ops.add_layernorm(rd, None, gd, bd, 1e-5, h)
        hx = oracle.layer_norm(res.double(), gamma.double(), beta.double(), 1e-5)
        for epi in (ops.EPI_BIAS, ops.EPI_BIAS_GELU):
            want = torch.empty(m, n, dtype=dt, device=device)
            ops.gemm(h, wd, biasd, want, epi, 9)  # class 1: one K chain
            for plan in range(ops.gemm_ln_plan_count()):
                got = torch.full((m, n), float("nan"), dtype=dt, device=device)
                ops.gemm_ln(rd, gd, bd, 1e-5, wd, biasd, got, epi, plan)
                torch.cuda.synchronize()
                assert torch.equal(got.cpu(), want.cpu()), (m, n, epi, plan)
            ref = hx.to(dt).double() @ w.double().t() + bias.double()
            if epi == ops.EPI_BIAS_GELU:
                ref = 0.5 * ref * (1 + torch.erf(ref / math.sqrt(2)))
            _close(got, ref, OUT_RTOL[dt], 2e-3)


def test_gemm_ln_rejects_unsupported(device):
    """Shapes and epilogues the LayerNorm GEMM does not take are refused
    before any launch."""
    res = torch.zeros(32, 640, device=device)
    gamma, beta = torch.ones(640, device=device), torch.zeros(640, device=device)
    w = torch.zeros(64, 640, dtype=torch.bfloat16, device=device)
    out = torch.empty(32, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ops.TjkError, match="not supported"):  # k = 640
        ops.gemm_ln(res, gamma, beta, 1e-5, w, None, out)
    assert not ops.gemm_ln_supported(640, torch.bfloat16) and ops.gemm_ln_supported(512, torch.float16)
    assert not ops.gemm_ln_supported(512, torch.float32)
    res, gamma, beta = res[:, :512], gamma[:512], beta[:512]
    w = torch.zeros(64, 512, dtype=torch.bfloat16, device=device)
    with pytest.raises(ops.TjkError, match="epilogue"):
        ops.gemm_ln(res.contiguous(), gamma.contiguous(), beta.contiguous(), 1e-5, w, None, out,
                    ops.EPI_BIAS_RESIDUAL)


# ------------------------------------------------------------ attention block

def _block_case(g, lengths, d, dt):
    rows = sum(lengths)
    x = torch.randn(rows, d, generator=g).to(dt)
    wqkv = (torch.randn(3 * d, d, generator=g) / math.sqrt(d)).to(dt)
    bqkv = (torch.randn(3 * d, generator=g) * 0.1).to(dt)
    wout = (torch.randn(d, d, generator=g) / math.sqrt(d)).to(dt)
    bout = (torch.randn(d, generator=g) * 0.1).to(dt)
    return x, wqkv, bqkv, wout, bout


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,lengths,causal,packed", [
    (512, [128], True, False),              # C2's shape
    (256, [100, 100], True, False),         # uniform batch, partial last query block
    (384, [1, 37, 128, 64, 0, 96], True, True),  # packed ragged lengths, one empty
    (128, [77, 128, 5], False, True),       # non-causal packed
    (512, [96, 96, 96], False, False),
    (256, [1], True, False),
])
def test_attn_block_against_unfused_and_fp64(device, dt, d, lengths, causal, packed):
    """tjk_attn_block == the unfused launches: its context equals the QKV
    GEMM (plan 9, which sums K in the same order) followed by attention plan
    4, bit for bit; the per-head partials sum to ctx W_out^T + b_out (fp64 of
    the kernel's own context, fp32 accumulation tolerance); the context
    matches fp64 attention of that Q/K/V; rows past the input are never
    written."""
    heads = d // 64
    g = _gen(d + 7 * len(lengths) + int(causal))
    x, wqkv, bqkv, wout, bout = _block_case(g, lengths, d, dt)
    rows = x.shape[0]
    xd, wqkv_d, bqkv_d, wout_d, bout_d = (t.to(device) for t in (x, wqkv, bqkv, wout, bout))
    parts = torch.full((heads, rows + 3, d), float("nan"), device=device)
    ctx = torch.full((rows + 3, d), float("nan"), dtype=dt, device=device)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32)
    kw = dict(cu_seqlens=cu.to(device), max_seqlen=max(lengths)) if packed else \
        dict(batch=len(lengths), seq=lengths[0])
    ops.attn_block(xd, wqkv_d, bqkv_d, wout_d, bout_d, parts[:, :rows], heads, causal=causal,
                   ctx_out=ctx[:rows], **kw)
    # the unfused launches on the same inputs
    qkv = torch.empty(rows, 3 * d, dtype=dt, device=device)
    ops.gemm(xd, wqkv_d, bqkv_d, qkv, ops.EPI_BIAS, plan=9)
    ref_ctx = torch.empty(rows, d, dtype=dt, device=device)
    if packed:
        ops.flash_attention(qkv.view(rows, 3, heads, 64), ref_ctx, causal=causal, plan=4,
                            cu_seqlens=cu.to(device), max_seqlen=max(lengths))
    else:
        ops.flash_attention(qkv.view(len(lengths), lengths[0], 3, heads, 64), ref_ctx, causal=causal, plan=4)
    torch.cuda.synchronize()
    got_ctx = ctx[:rows].cpu()
    assert torch.isnan(ctx[rows:].float()).all() and torch.isnan(parts[:, rows:]).all(), \
        "rows past the input were written"
    assert torch.equal(got_ctx, ref_ctx.cpu()), "context differs from QKV GEMM + attention plan 4"
    # out-projection partials: their sum is ctx W_out^T + b_out
    want = got_ctx.double() @ wout.double().t() + bout.double()
    _close(parts[:, :rows].double().sum(0), want, 1e-5, 1e-5)
    # the context against fp64 attention of the GEMM's Q / K / V
    qkv_c = qkv.cpu()
    start = 0
    for n in lengths:
        if n:
            seq_qkv = qkv_c[start:start + n].view(1, n, 3, heads, 64)
            _close(got_ctx[start:start + n], _attn_ref(seq_qkv, causal), 1e-2, 1e-2)
        start += n


def test_attn_block_closed_forms(device):
    """W_qkv = 0: Q = bq, K = bk, V = bv for every row, so every query's
    context is bv (softmax weights sum to 1), and the partials sum to
    bv_heads W_out^T + b_out on every row; W_out = 0: only head 0 carries
    b_out."""
    d, heads, n, dt = 256, 4, 70, torch.bfloat16
    g = _gen(11)
    x = torch.randn(n, d, generator=g).to(dt)
    bqkv = torch.randn(3 * d, generator=g).to(dt)
    wout = (torch.randn(d, d, generator=g) / 16).to(dt)
    bout = torch.randn(d, generator=g).to(dt)
    parts = torch.empty(heads, n, d, device=device)
    ctx = torch.empty(n, d, dtype=dt, device=device)
    ops.attn_block(x.to(device), torch.zeros(3 * d, d, dtype=dt, device=device), bqkv.to(device),
                   wout.to(device), bout.to(device), parts, heads, causal=True, batch=1, seq=n, ctx_out=ctx)
    torch.cuda.synchronize()
    bv = bqkv[2 * d:].float()
    _close(ctx, bv.double().expand(n, d), 8e-3, 1e-3)
    want = (bv.to(dt).double() @ wout.double().t() + bout.double()).expand(n, d)
    _close(parts.sum(0), want, 1e-2, 1e-2)
    ops.attn_block(x.to(device), torch.randn(3 * d, d, dtype=dt, device=device) / 16, bqkv.to(device),
                   torch.zeros(d, d, dtype=dt, device=device), bout.to(device), parts, heads, causal=True,
                   batch=1, seq=n)
    torch.cuda.synchronize()
    assert torch.equal(parts[0].cpu(), bout.float().expand(n, d))
    assert (parts[1:] == 0).all()


def test_attn_block_rejects_unsupported_shapes(device):
    d = 512
    x = torch.zeros(200, d, dtype=torch.bfloat16, device=device)
    w = torch.zeros(3 * d, d, dtype=torch.bfloat16, device=device)
    wo = torch.zeros(d, d, dtype=torch.bfloat16, device=device)
    parts = torch.zeros(8, 200, d, device=device)
    with pytest.raises(ops.TjkError, match="unsupported|at most 128"):
        ops.attn_block(x, w, None, wo, None, parts, 8, batch=1, seq=200)   # sequence longer than 128
    with pytest.raises(ops.TjkError, match="unsupported|head_dim"):
        ops.attn_block(x[:, :d], w, None, wo, None, torch.zeros(16, 200, d, device=device), 16,
                       batch=2, seq=100)   # head_dim 32
    assert not ops.attn_block_supported(1024, 16, 64, 128, torch.bfloat16)
    assert not ops.attn_block_supported(512, 8, 64, 128, torch.float32)
    assert ops.attn_block_supported(512, 8, 64, 128, torch.float16)
