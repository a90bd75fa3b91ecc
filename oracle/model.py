"""CPU oracle for the fused Transformer forward.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may import this module, and only as the
checker (or as the CPU baseline being timed).  The product path
(``tjkernels``) never imports it and has no CPU fallback.

This is a from-scratch restatement, in plain PyTorch on the CPU, of the
reference's ``BaselineTransformer.forward`` (torch_transformer_benchmark.py:
66-179).  It runs in float32 or float64 on the rounded model-dtype weights
and inputs upcast to that dtype, so only compute error is measured
(the pattern of bench/test_bf16_limit.py:73-77,88).  Step by step:

* attention (:98-129): q/k/v projections, ``scores = (q @ k^T) * hd^-1/2``
  (:104), causal ``triu(1) -> -inf`` (:106-110), invalid keys ``-inf``
  (:112-115), softmax (:118), ``probs @ v`` (:119), heads merged (:120-124),
  out-proj (:125), invalid rows zeroed (:127-128);
* block (:147-151): ``x + attn(LN1 x)``, then
  ``x + W2 gelu_erf(W1 LN2 x + b1) + b2``, invalid rows zeroed;
* model (:174-178): the blocks, final LayerNorm, invalid rows zeroed.

LayerNorm is biased-variance with the module's eps (nn.LayerNorm default
1e-5, :135,137,167).  GELU is the exact erf form (:148, approximate="none").

Pinned by ``tests/test_oracle.py``: against ``torch.nn.TransformerEncoder``
(a library routine that reduces to the same pre-LN block), against
``F.layer_norm`` / ``F.scaled_dot_product_attention``, against ``math.erf``,
against closed forms (S=1 gives out = V, constant row LN gives beta), and
against invariants (causality, batch-split, prefix independence).
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import torch

__all__ = [
    "layer_norm", "gelu_erf", "attention", "block", "forward",
    "compare_outputs", "budget_usage",
]


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
               eps: float = 1e-5) -> torch.Tensor:
    """Biased-variance LayerNorm over the last dim (nn.LayerNorm semantics)."""
    mean = x.mean(dim=-1, keepdim=True)
    centered = x - mean
    var = (centered * centered).mean(dim=-1, keepdim=True)
    return centered / torch.sqrt(var + eps) * weight + bias


def gelu_erf(x: torch.Tensor) -> torch.Tensor:
    """0.5 x (1 + erf(x / sqrt(2))) -- F.gelu(approximate="none")."""
    return 0.5 * x * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))


def attention(x: torch.Tensor, p: Dict[str, torch.Tensor], prefix: str,
              heads: int, mask: Optional[torch.Tensor], causal: bool) -> torch.Tensor:
    """torch_transformer_benchmark.py:92-129 on a [B,S,d] input."""
    b, s, d = x.shape
    hd = d // heads

    def proj(name, t):
        return t @ p[f"{prefix}{name}.weight"].t() + p[f"{prefix}{name}.bias"]

    def split(t):
        return t.view(b, s, heads, hd).transpose(1, 2)

    q = split(proj("q_proj", x))
    k = split(proj("k_proj", x))
    v = split(proj("v_proj", x))
    scores = (q @ k.transpose(-2, -1)) * (hd ** -0.5)
    if causal:
        tri = torch.ones((s, s), dtype=torch.bool).triu(diagonal=1)
        scores = scores.masked_fill(tri, float("-inf"))
    if mask is not None:
        scores = scores.masked_fill(~mask[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    ctx = (probs @ v).transpose(1, 2).reshape(b, s, d)
    out = proj("out_proj", ctx)
    if mask is not None:
        out = out.masked_fill(~mask[..., None], 0.0)
    return out


def block(x: torch.Tensor, p: Dict[str, torch.Tensor], i: int, heads: int,
          mask: Optional[torch.Tensor], causal: bool, eps: float = 1e-5) -> torch.Tensor:
    """torch_transformer_benchmark.py:141-152."""
    pre = f"layers.{i}."
    h = layer_norm(x, p[pre + "norm1.weight"], p[pre + "norm1.bias"], eps)
    x = x + attention(h, p, pre + "attention.", heads, mask, causal)
    h2 = layer_norm(x, p[pre + "norm2.weight"], p[pre + "norm2.bias"], eps)
    hidden = gelu_erf(h2 @ p[pre + "ffn_in.weight"].t() + p[pre + "ffn_in.bias"])
    x = x + (hidden @ p[pre + "ffn_out.weight"].t() + p[pre + "ffn_out.bias"])
    if mask is not None:
        x = x.masked_fill(~mask[..., None], 0.0)
    return x


@torch.no_grad()
def forward(state_dict: Dict[str, torch.Tensor], x: torch.Tensor,
            mask: Optional[torch.Tensor], heads: int, causal: bool = True,
            dtype: torch.dtype = torch.float32, eps: float = 1e-5) -> torch.Tensor:
    """Whole-model forward (torch_transformer_benchmark.py:169-179) on the CPU.

    ``state_dict`` and ``x`` are upcast to ``dtype``; the result is in
    ``dtype``.  Work is done one sequence at a time (rows of different
    sequences never interact), which bounds the [H,S,S] score tensor.
    """
    p = {k: v.detach().to("cpu", dtype) for k, v in state_dict.items()}
    layers = 1 + max(int(k.split(".")[1]) for k in p if k.startswith("layers."))
    x = x.detach().to("cpu", dtype)
    m = None if mask is None else mask.detach().to("cpu", torch.bool)
    outs = []
    for bi in range(x.shape[0]):
        xb = x[bi:bi + 1]
        mb = None if m is None else m[bi:bi + 1]
        for i in range(layers):
            xb = block(xb, p, i, heads, mb, causal, eps)
        xb = layer_norm(xb, p["final_norm.weight"], p["final_norm.bias"], eps)
        if mb is not None:
            xb = xb.masked_fill(~mb[..., None], 0.0)
        outs.append(xb)
    return torch.cat(outs, dim=0)


def compare_outputs(reference: torch.Tensor, optimized: torch.Tensor,
                    rtol: float, atol: float) -> Dict[str, float]:
    """Per-element OR rule of torch_transformer_benchmark.py:293-360:
    an element passes if it is finite and ``|d| <= atol`` or ``|d| <= rtol*|ref|``."""
    ref = reference.detach().double().cpu()
    opt = optimized.detach().double().cpu()
    if ref.shape != opt.shape:
        raise AssertionError(f"shape mismatch {tuple(ref.shape)} vs {tuple(opt.shape)}")
    err = (opt - ref).abs()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    ok = finite & ((err <= atol) | (err <= rtol * ref.abs()))
    return {
        "passed": bool(ok.all()),
        "failed": int((~ok).sum()),
        "total": ref.numel(),
        "max_abs": float(err.max()) if err.numel() else 0.0,
        "mean_abs": float(err.mean()) if err.numel() else 0.0,
    }


def budget_usage(reference: torch.Tensor, optimized: torch.Tensor,
                 rtol: float, atol: float) -> float:
    """Worst per-element use of ``max(atol, rtol*|ref|)`` (bench/autotune.py:61-68)."""
    ref = reference.detach().double().cpu()
    err = (optimized.detach().double().cpu() - ref).abs()
    return float((err / (ref.abs() * rtol).clamp_min(atol)).max())
