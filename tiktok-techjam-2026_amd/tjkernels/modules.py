"""Module skeleton for the drop-in hook.

``TransformerConfig`` mirrors the harness's frozen dataclass
(torch_transformer_benchmark.py:36-63).  ``TransformerLayout`` builds the same
parameter tree as ``BaselineTransformer`` (torch_transformer_benchmark.py:
66-179): ``layers.{i}.norm1``, ``layers.{i}.attention.{q,k,v,out}_proj``,
``layers.{i}.norm2``, ``layers.{i}.ffn_in``, ``layers.{i}.ffn_out`` and
``final_norm``, so a strict ``load_state_dict`` from the baseline
(torch_transformer_benchmark.py:207-217) works unchanged.  It carries no
forward of its own: the only forward in this package is the HIP engine.

``UserOptimizedTransformer`` is the hook (torch_transformer_benchmark.py:
182-204): its forward is one call to ``tjkernels.forward``.  Inside the
reference harness the same one-line body is placed in the harness's own
``UserOptimizedTransformer(BaselineTransformer)``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn


@dataclass(frozen=True)
class TransformerConfig:
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for field in ("batch_size", "seq_len", "d_model", "num_heads",
                      "ffn_dim", "num_layers"):
            if getattr(self, field) <= 0:
                raise ValueError(f"{field} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by "
                f"num_heads ({self.num_heads})"
            )


class _Attention(nn.Module):
    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)


class _Block(nn.Module):
    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = _Attention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)


class TransformerLayout(nn.Module):
    """Parameters of the pre-LN causal encoder, with no forward."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__()
        config.validate()
        self.config = config
        self.layers = nn.ModuleList(
            [_Block(config.d_model, config.num_heads, config.ffn_dim)
             for _ in range(config.num_layers)]
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x, valid_token_mask=None):  # pragma: no cover - guard
        raise NotImplementedError(
            "TransformerLayout only holds parameters; use UserOptimizedTransformer "
            "(or tjkernels.forward) to run the HIP forward"
        )


class UserOptimizedTransformer(TransformerLayout):
    """The drop-in hook: same constructor, parameters and forward signature
    as the reference's ``UserOptimizedTransformer``."""

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
    ) -> torch.Tensor:
        from .engine import forward as _forward
        return _forward(self, x, valid_token_mask)
