"""Pins the CPU oracle (oracle/model.py) before it is trusted as the checker.

The reference ships no golden vectors for this path, so each piece is pinned
by an independent library routine, a closed form, or an invariant, chosen so
that a plausible mistake (unbiased variance, missing scale, tanh GELU, a
transposed weight, a dropped causal mask, q/k swapped) fails one of them.
``test_planted_mistakes_are_caught`` plants such mistakes in the oracle and
checks that the pins notice.
"""

import math
from pathlib import Path

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import model as oracle
from tjkernels.modules import TransformerConfig, TransformerLayout
from tjkernels.workloads import WORKLOADS, flops_per_forward, make_inputs, make_state_dict


def _random_sd(cfg, seed=0, dtype=torch.float64):
    torch.manual_seed(seed)
    m = TransformerLayout(cfg)
    sd = {k: v.detach().to(dtype) for k, v in m.state_dict().items()}
    g = torch.Generator()
    g.manual_seed(seed + 1)
    for k in sd:  # non-trivial LN affine and biases
        if "norm" in k or k.endswith("bias"):
            sd[k] = sd[k] + 0.1 * torch.randn(sd[k].shape, generator=g, dtype=dtype)
    return sd


def _torch_encoder(cfg, sd):
    """nn.TransformerEncoder (pre-LN, exact GELU, no dropout) carrying sd."""
    layer = nn.TransformerEncoderLayer(cfg.d_model, cfg.num_heads, cfg.ffn_dim, dropout=0.0,
                                       activation="gelu", batch_first=True, norm_first=True)
    enc = nn.TransformerEncoder(layer, cfg.num_layers, norm=nn.LayerNorm(cfg.d_model),
                                enable_nested_tensor=False).double().eval()
    with torch.no_grad():
        for i, lyr in enumerate(enc.layers):
            p = f"layers.{i}."
            a = p + "attention."
            lyr.self_attn.in_proj_weight.copy_(torch.cat([sd[a + n + ".weight"] for n in ("q_proj", "k_proj", "v_proj")]))
            lyr.self_attn.in_proj_bias.copy_(torch.cat([sd[a + n + ".bias"] for n in ("q_proj", "k_proj", "v_proj")]))
            lyr.self_attn.out_proj.weight.copy_(sd[a + "out_proj.weight"])
            lyr.self_attn.out_proj.bias.copy_(sd[a + "out_proj.bias"])
            lyr.linear1.weight.copy_(sd[p + "ffn_in.weight"])
            lyr.linear1.bias.copy_(sd[p + "ffn_in.bias"])
            lyr.linear2.weight.copy_(sd[p + "ffn_out.weight"])
            lyr.linear2.bias.copy_(sd[p + "ffn_out.bias"])
            for n in ("norm1", "norm2"):
                getattr(lyr, n).weight.copy_(sd[p + n + ".weight"])
                getattr(lyr, n).bias.copy_(sd[p + n + ".bias"])
        enc.norm.weight.copy_(sd["final_norm.weight"])
        enc.norm.bias.copy_(sd["final_norm.bias"])
    return enc


def _library_forward(cfg, sd, x, mask):
    enc = _torch_encoder(cfg, sd)
    s = x.shape[1]
    attn_mask = nn.Transformer.generate_square_subsequent_mask(s, dtype=torch.float64) if cfg.causal else None
    kpm = None if mask is None else torch.zeros(mask.shape, dtype=torch.float64).masked_fill(~mask, float("-inf"))
    with torch.no_grad():
        return enc(x, mask=attn_mask, src_key_padding_mask=kpm, is_causal=cfg.causal and kpm is None)


CFGS = [
    TransformerConfig(2, 24, 32, 4, 48, 2, True),
    TransformerConfig(3, 17, 48, 3, 64, 3, True),
    TransformerConfig(2, 20, 32, 2, 40, 2, False),
]


@pytest.mark.parametrize("cfg", CFGS, ids=["causal", "ragged", "non-causal"])
@pytest.mark.parametrize("padded", [False, True])
def test_model_matches_torch_transformer_encoder(cfg, padded):
    """Whole forward vs nn.TransformerEncoder (library routine for the same
    pre-LN block), on valid rows; padded rows must be exactly zero."""
    sd = _random_sd(cfg)
    g = torch.Generator()
    g.manual_seed(7)
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g, dtype=torch.float64)
    mask = None
    if padded:
        lengths = torch.randint(1, cfg.seq_len + 1, (cfg.batch_size,), generator=g)
        lengths[0] = cfg.seq_len
        mask = torch.arange(cfg.seq_len)[None, :] < lengths[:, None]
        x = x.masked_fill(~mask[..., None], 0.0)
    got = oracle.forward(sd, x, mask, cfg.num_heads, cfg.causal, torch.float64)
    want = _library_forward(cfg, sd, x, mask)
    valid = torch.ones(x.shape[:2], dtype=torch.bool) if mask is None else mask
    assert torch.allclose(got[valid], want[valid], rtol=1e-10, atol=1e-10)
    assert (got[~valid] == 0).all()


def test_layer_norm_matches_library():
    g = torch.Generator()
    g.manual_seed(0)
    x = torch.randn(7, 96, generator=g, dtype=torch.float64) * 5 + 2
    w = torch.randn(96, generator=g, dtype=torch.float64)
    b = torch.randn(96, generator=g, dtype=torch.float64)
    assert torch.allclose(oracle.layer_norm(x, w, b), F.layer_norm(x, (96,), w, b, 1e-5), atol=1e-12)
    # closed forms: constant row -> beta; gamma=1, beta=0 -> zero mean, unit biased variance
    c = torch.full((3, 96), 4.0, dtype=torch.float64)
    assert torch.allclose(oracle.layer_norm(c, w, b), b.expand(3, 96))
    y = oracle.layer_norm(x, torch.ones(96, dtype=torch.float64), torch.zeros(96, dtype=torch.float64), 0.0)
    assert torch.allclose(y.mean(-1), torch.zeros(7, dtype=torch.float64), atol=1e-12)
    assert torch.allclose((y * y).mean(-1), torch.ones(7, dtype=torch.float64), atol=1e-12)


def test_gelu_is_exact_erf():
    xs = [-6.0, -3.1, -1.0, -0.25, 0.0, 1e-3, 0.5, 1.0, 2.2, 7.5]
    got = oracle.gelu_erf(torch.tensor(xs, dtype=torch.float64))
    want = [0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in xs]
    assert torch.allclose(got, torch.tensor(want, dtype=torch.float64), rtol=1e-14, atol=1e-300)
    # and it is not the tanh approximation
    assert not torch.allclose(got, F.gelu(torch.tensor(xs, dtype=torch.float64), approximate="tanh"),
                              rtol=1e-6, atol=0)


def test_attention_closed_forms():
    cfg = TransformerConfig(2, 1, 32, 4, 64, 1, True)
    sd = _random_sd(cfg)
    pre = "layers.0.attention."
    h = torch.randn(2, 1, 32, dtype=torch.float64)
    # S = 1: softmax over one key is 1, so the context is V itself
    out = oracle.attention(h, sd, pre, 4, None, True)
    v = h @ sd[pre + "v_proj.weight"].t() + sd[pre + "v_proj.bias"]
    want = v @ sd[pre + "out_proj.weight"].t() + sd[pre + "out_proj.bias"]
    assert torch.allclose(out, want, atol=1e-12)


def test_attention_matches_sdpa_with_masks():
    cfg = TransformerConfig(2, 19, 32, 4, 64, 1, False)
    sd = _random_sd(cfg)
    pre = "layers.0.attention."
    g = torch.Generator()
    g.manual_seed(3)
    h = torch.randn(2, 19, 32, generator=g, dtype=torch.float64)
    mask = torch.rand(2, 19, generator=g) > 0.3
    mask[:, 0] = True
    for causal in (False, True):
        got = oracle.attention(h, sd, pre, 4, mask, causal)

        def proj(n, t):
            return t @ sd[pre + n + ".weight"].t() + sd[pre + n + ".bias"]
        q, k, v = (proj(n, h).view(2, 19, 4, 8).transpose(1, 2) for n in ("q_proj", "k_proj", "v_proj"))
        allowed = mask[:, None, None, :].expand(2, 4, 19, 19)
        if causal:
            allowed = allowed & torch.ones(19, 19, dtype=torch.bool).tril()
        ctx = F.scaled_dot_product_attention(q, k, v, attn_mask=allowed)
        want = proj("out_proj", ctx.transpose(1, 2).reshape(2, 19, 32))
        want = want.masked_fill(~mask[..., None], 0.0)
        valid = mask & allowed.any(-1)[:, 0]
        assert torch.allclose(got[valid], want[valid], atol=1e-12)


def test_causality_and_prefix_independence():
    cfg = TransformerConfig(2, 16, 32, 4, 48, 2, True)
    sd = _random_sd(cfg)
    g = torch.Generator()
    g.manual_seed(11)
    x = torch.randn(2, 16, 32, generator=g, dtype=torch.float64)
    base = oracle.forward(sd, x, None, 4, True, torch.float64)
    x2 = x.clone()
    x2[:, 9:] += torch.randn(2, 7, 32, generator=g, dtype=torch.float64)
    pert = oracle.forward(sd, x2, None, 4, True, torch.float64)
    assert torch.allclose(base[:, :9], pert[:, :9], atol=1e-12)
    assert not torch.allclose(base[:, 9:], pert[:, 9:])
    # causal + prefix mask: valid rows do not depend on padded positions
    lengths = torch.tensor([10, 16])
    mask = torch.arange(16)[None, :] < lengths[:, None]
    a = oracle.forward(sd, x.masked_fill(~mask[..., None], 0), mask, 4, True, torch.float64)
    b = oracle.forward(sd, x, mask, 4, True, torch.float64)
    assert torch.allclose(a, b, atol=1e-12)
    assert (a[~mask] == 0).all()


def test_planted_mistakes_are_caught(monkeypatch):
    """Each planted oracle bug makes the library comparison fail."""
    cfg = CFGS[0]
    sd = _random_sd(cfg)
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, dtype=torch.float64)
    want = _library_forward(cfg, sd, x, None)

    def unbiased_ln(x, w, b, eps=1e-5):
        return (x - x.mean(-1, keepdim=True)) / torch.sqrt(x.var(-1, keepdim=True, unbiased=True) + eps) * w + b

    def tanh_gelu(x):
        return F.gelu(x, approximate="tanh")

    real_attention = oracle.attention

    def no_causal(x, p, prefix, heads, mask, causal):
        return real_attention(x, p, prefix, heads, mask, False)

    for name, fake in (("layer_norm", unbiased_ln), ("gelu_erf", tanh_gelu), ("attention", no_causal)):
        with monkeypatch.context() as m:
            m.setattr(oracle, name, fake)
            got = oracle.forward(sd, x, None, cfg.num_heads, True, torch.float64)
        assert not torch.allclose(got, want, rtol=1e-6, atol=1e-6), f"planted {name} bug not caught"
    # a transposed weight is caught too
    sd_t = dict(sd)
    w = sd_t["layers.0.attention.q_proj.weight"]
    sd_t["layers.0.attention.q_proj.weight"] = w.t().contiguous()
    got = oracle.forward(sd_t, x, None, cfg.num_heads, True, torch.float64)
    assert not torch.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_compare_outputs_or_rule():
    ref = torch.tensor([1.0, 100.0, 0.0, 1.0])
    # |d| <= atol passes; |d| <= rtol*|ref| passes; otherwise fails; NaN fails
    r = oracle.compare_outputs(ref, torch.tensor([1.002, 101.9, 0.0019, 1.0]), rtol=0.02, atol=0.002)
    assert r["passed"]
    r = oracle.compare_outputs(ref, torch.tensor([1.03, 100.0, 0.0, 1.0]), rtol=0.02, atol=0.002)
    assert not r["passed"] and r["failed"] == 1
    r = oracle.compare_outputs(ref, torch.tensor([1.0, 100.0, float("nan"), 1.0]), rtol=0.02, atol=0.002)
    assert r["failed"] == 1
    assert abs(oracle.budget_usage(ref.double(), torch.tensor([1.01, 100.0, 0.0, 1.0], dtype=torch.float64), 0.02, 0.002) - 0.5) < 1e-9


def test_golden_fixture_is_reproduced():
    """The committed C1 vectors: same seeded inputs/weights, same oracle output."""
    fx = torch.load(Path(__file__).parent / "golden" / "c1_fixture.pt", weights_only=True)
    w = WORKLOADS["C1"]
    sd = make_state_dict(w, seed=int(fx["param_seed"]))
    chk = torch.tensor([[float(v.double().sum()), float((v.double() ** 2).sum())]
                        for _, v in sorted(sd.items())], dtype=torch.float64)
    assert torch.allclose(chk, fx["weight_checksum"], rtol=1e-12, atol=1e-9)
    x, mask, lengths = make_inputs(w, seed=int(fx["input_seed"]))
    assert torch.equal(x, fx["x"]) and torch.equal(mask, fx["mask"])
    assert torch.equal(lengths, fx["lengths"])
    out = oracle.forward(sd, x, mask, w.heads, w.causal, torch.float64)
    assert torch.allclose(out, fx["out_fp64"], rtol=1e-10, atol=1e-10)
    out32 = oracle.forward(sd, x, mask, w.heads, w.causal, torch.float32)
    assert torch.allclose(out32.double(), fx["out_fp64"], atol=1e-4)


def test_workload_generators_and_flops():
    # FLOP model: the BASELINE table values
    want = {"C1": 0.105, "C2": 3.289, "C3": 244.84, "C4": 962.14, "C5": 5772.6}
    for name, gflop in want.items():
        got = flops_per_forward(WORKLOADS[name]) / 1e9
        assert abs(got - gflop) / gflop < 5e-3, (name, got)
    w = WORKLOADS["C3"]
    x, mask, lengths = make_inputs(w, seed=1)
    assert lengths.min() >= 1 and lengths.max() <= w.seq
    assert torch.equal(mask, torch.arange(w.seq)[None, :] < lengths[:, None].long())
    assert (x[~mask] == 0).all()
    x2, _, _ = make_inputs(w, seed=1)
    assert torch.equal(x, x2)
    # rounded to the model dtype
    assert torch.equal(x, x.to(w.dtype).float())
    sd = make_state_dict(WORKLOADS["C2"], seed=0)
    assert abs(float(sd["layers.0.ffn_in.weight"].std()) - 0.02) < 1e-3
    assert (sd["layers.0.norm1.weight"] == 1).all() and (sd["layers.0.ffn_in.bias"] == 0).all()
