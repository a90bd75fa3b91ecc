"""Named workloads and seeded synthetic inputs.

The five configurations C1..C5 are the shapes this build is measured and
parity-tested on.  Input generation restates the reference harness's
``generate_random_case`` (torch_transformer_benchmark.py:238-276): draw
``x ~ N(0,1)`` of shape [B,S,d], draw per-sequence prefix lengths with
``randint(low=min_len, high=S+1)``, build ``mask = arange(S) < len`` and zero
the padded rows of ``x`` (:275).  Everything is drawn on a CPU
``torch.Generator`` in fp32 and then rounded to the model dtype, so the same
seed gives the same tensors on every machine.

Weights follow the configs' recipe instead of ``nn.Linear``'s default init:
``N(0, std)`` for every projection, zero biases, LayerNorm gamma=1 and
beta=0.  The parameter names and shapes are exactly the reference module's
``state_dict`` keys (torch_transformer_benchmark.py:79-82,135-139,167).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from .modules import TransformerConfig


@dataclass(frozen=True)
class Workload:
    name: str
    layers: int
    d_model: int
    heads: int
    ffn_dim: int
    batch: int
    seq: int
    dtype: torch.dtype
    min_len: Optional[int]          # None -> every sequence is full length
    weight_std: float
    causal: bool = True
    note: str = ""

    @property
    def config(self) -> TransformerConfig:
        return TransformerConfig(
            batch_size=self.batch, seq_len=self.seq, d_model=self.d_model,
            num_heads=self.heads, ffn_dim=self.ffn_dim,
            num_layers=self.layers, causal=self.causal,
        )

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def describe(self) -> str:
        lens = "full" if self.min_len is None else f"U[{self.min_len},{self.seq}]"
        return (f"{self.name}: L{self.layers} d{self.d_model} H{self.heads} "
                f"f{self.ffn_dim} B{self.batch} S{self.seq} "
                f"{str(self.dtype).replace('torch.', '')} lengths {lens}")


WORKLOADS: Dict[str, Workload] = {
    "C1": Workload("C1", 2, 128, 4, 512, 2, 64, torch.float32, 32, 0.02,
                   note="tiny fp32, CPU reference path + GPU fp32 plan"),
    "C2": Workload("C2", 4, 512, 8, 2048, 1, 128, torch.float16, None, 0.02,
                   note="launch-bound, hipGraph capture"),
    "C3": Workload("C3", 4, 768, 12, 3072, 8, 512, torch.float16, 1, 0.02,
                   note="ragged padding"),
    "C4": Workload("C4", 4, 1024, 16, 4096, 4, 2048, torch.bfloat16, 1024, 0.02,
                   note="headline MFMA-utilisation config"),
    "C5": Workload("C5", 6, 2048, 16, 8192, 2, 4096, torch.bfloat16, None, 0.01,
                   note="large contraction, hd=128"),
    # The reference matrix's case 14 (bench/shapes.py:67-69), which it never
    # ran (README.md:167-180: 13 GB of input, an S x S score tensor in its
    # reference).  Here attention streams K/V tiles in O(S) memory and the
    # whole forward fits in ~65 GB of the 288 GB HBM.
    "C14": Workload("C14", 2, 1024, 16, 1024, 32, 100000, torch.bfloat16, None, 0.02,
                    note="reference case 14: S=100000 streaming"),
}


def flops_per_forward(w: Workload) -> float:
    """Algorithmic FLOPs of one forward over the full padded S.

    F = L * [6 T d^2 (QKV) + 2 T d^2 (out) + 4 T d f (FFN) + 2 B d S (S+1)]
    where the last term counts causal QK^T and PV over S(S+1)/2 pairs per
    head.  Non-causal attention counts all S^2 pairs (4 B d S^2).
    """
    t, d, f = w.tokens, w.d_model, w.ffn_dim
    attn = 2.0 * w.batch * d * w.seq * (w.seq + 1) if w.causal else 4.0 * w.batch * d * w.seq ** 2
    return w.layers * (6.0 * t * d * d + 2.0 * t * d * d + 4.0 * t * d * f + attn)


def flops_valid_tokens(w: Workload, lengths) -> float:
    """FLOPs of the work a packed forward executes: the GEMMs over the
    sum(lengths) valid rows and attention over each sequence's own valid
    (query, key) pairs (causal: len(len+1)/2 per head)."""
    t, d, f = sum(lengths), w.d_model, w.ffn_dim
    pairs = sum(n * (n + 1) // 2 if w.causal else n * n for n in lengths)
    return w.layers * (6.0 * t * d * d + 2.0 * t * d * d + 4.0 * t * d * f + 4.0 * d * pairs)


def make_state_dict(w: Workload, seed: int = 0) -> Dict[str, torch.Tensor]:
    """fp32 CPU state_dict with the reference module's keys, rounded to the
    model dtype and returned in fp32 (so the oracle sees the rounded values)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    d, f, std = w.d_model, w.ffn_dim, w.weight_std
    sd: Dict[str, torch.Tensor] = {}

    def normal(*shape):
        t = torch.randn(*shape, generator=g, dtype=torch.float32) * std
        return t.to(w.dtype).float()

    for i in range(w.layers):
        p = f"layers.{i}."
        sd[p + "norm1.weight"] = torch.ones(d)
        sd[p + "norm1.bias"] = torch.zeros(d)
        for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
            sd[p + f"attention.{name}.weight"] = normal(d, d)
            sd[p + f"attention.{name}.bias"] = torch.zeros(d)
        sd[p + "norm2.weight"] = torch.ones(d)
        sd[p + "norm2.bias"] = torch.zeros(d)
        sd[p + "ffn_in.weight"] = normal(f, d)
        sd[p + "ffn_in.bias"] = torch.zeros(f)
        sd[p + "ffn_out.weight"] = normal(d, f)
        sd[p + "ffn_out.bias"] = torch.zeros(d)
    sd["final_norm.weight"] = torch.ones(d)
    sd["final_norm.bias"] = torch.zeros(d)
    return sd


def make_inputs(
    w: Workload, seed: int = 1, min_len: Optional[int] = -1,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(x [B,S,d] fp32 rounded to the model dtype, mask [B,S] bool, lengths [B] int32).

    Follows torch_transformer_benchmark.py:246-276: x first, then lengths from
    the same generator, padded x rows zeroed.  ``min_len=-1`` uses the
    workload's own setting; ``None`` forces full-length sequences.
    """
    if min_len == -1:
        min_len = w.min_len
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    x = torch.randn(w.batch, w.seq, w.d_model, generator=g, dtype=torch.float32)
    if min_len is None:
        lengths = torch.full((w.batch,), w.seq, dtype=torch.int64)
    else:
        lengths = torch.randint(low=max(1, min_len), high=w.seq + 1,
                                size=(w.batch,), generator=g)
    mask = torch.arange(w.seq)[None, :] < lengths[:, None]
    x = x.masked_fill(~mask[..., None], 0.0)
    x = x.to(w.dtype).float()
    return x, mask, lengths.to(torch.int32)
