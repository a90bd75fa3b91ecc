"""Shape -> execution-plan dispatch.

Mirrors the reference's dispatcher (tjkernels/plans.py:29-198): a frozen
``Plan`` of knobs, a shape key, a heuristic ``default_plan``, a JSON table of
tuned plans (``plans.json``, written by ``tjkernels.autotune``) that
overrides the heuristic per shape, environment overrides for ablation, and a
programmatic ``set_override``.

Differences, all MI355X-specific:
* every kernel knob names a HIP implementation; there is no torch/SDPA
  backend to select (the product path has no non-HIP fallback);
* the plan carries tile-plan ids for each GEMM and for attention
  (-1 = the library's own heuristic), and ``residual_epilogue`` (add the
  out-proj and FFN outputs into the fp32 residual inside the GEMM epilogue
  instead of deferring them to the next LayerNorm);
* an fp32 model runs the IEEE fp32 plan by default, since only fp32 compute
  holds the 1e-4 per-element budget of fp32 plans;
* tuned entries are keyed by shape *and* GPU architecture (``@gfx950``);
* ``pack_prefix``: prefix-masked batches run only their valid tokens (off:
  every padded row is computed and zeroed at the end, the reference's way).

Environment knobs (applied to the heuristic plan, so ablations set
``TJ_IGNORE_PLANS=1`` as the reference's ablation does): ``TJ_NO_GRAPH``,
``TJ_COMPUTE_DTYPE``, ``TJ_DEFERRED_RESIDUAL``, ``TJ_NO_PACK``,
``TJ_ATTN_PLAN``; ``TJ_GEMM_TUNE=0`` (tjkernels.tiles) skips the measured
tile choice.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass, fields, replace
from pathlib import Path
from typing import Dict, Optional

import torch

_PLAN_FILE = Path(__file__).with_name("plans.json")

_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
_DTYPE_NAMES = {v: k for k, v in _DTYPES.items()}


@dataclass(frozen=True)
class Plan:
    """Execution knobs for one (shape, dtype, architecture)."""

    compute_dtype: torch.dtype = torch.bfloat16
    residual_dtype: torch.dtype = torch.float32
    attn: str = "hip"
    ffn: str = "hip"
    norm: str = "hip"
    packed_qkv: bool = True
    cuda_graph: bool = True          # whole-forward hipGraph capture
    residual_epilogue: bool = True   # GEMM epilogues update the fp32 residual
    gemm_qkv: int = -1               # tile plan ids, -1 = library heuristic
    gemm_out: int = -1
    gemm_ffn1: int = -1
    gemm_ffn2: int = -1
    attn_plan: int = -1
    pack_prefix: bool = True         # run only the valid tokens of prefix masks
    label: str = "default"

    def to_json(self) -> Dict[str, object]:
        blob = {f.name: getattr(self, f.name) for f in fields(self)}
        blob["compute_dtype"] = _DTYPE_NAMES[self.compute_dtype]
        blob["residual_dtype"] = _DTYPE_NAMES[self.residual_dtype]
        return blob

    @staticmethod
    def from_json(blob: Dict[str, object]) -> "Plan":
        blob = dict(blob)
        blob["compute_dtype"] = _DTYPES[str(blob.get("compute_dtype", "bfloat16"))]
        blob["residual_dtype"] = _DTYPES[str(blob.get("residual_dtype", "float32"))]
        names = {f.name for f in fields(Plan)}
        return Plan(**{k: v for k, v in blob.items() if k in names})

    def validate(self) -> None:
        if self.residual_dtype != torch.float32:
            raise ValueError("only a float32 residual stream is implemented")
        for knob in ("attn", "ffn", "norm"):
            if getattr(self, knob) != "hip":
                raise ValueError(f"{knob}={getattr(self, knob)!r}: only 'hip' kernels exist "
                                 "(no torch/SDPA fallback in this build)")
        if not self.packed_qkv:
            raise ValueError("only the packed QKV layout is implemented")


def device_arch(device: torch.device) -> str:
    if device.type != "cuda":
        return device.type
    name = torch.cuda.get_device_properties(device).gcnArchName
    return name.split(":")[0]


def shape_key(batch: int, seq: int, d_model: int, heads: int, ffn_dim: int,
              layers: int, causal: bool, dtype: torch.dtype, arch: str = "gfx950") -> str:
    return (f"b{batch}_s{seq}_d{d_model}_h{heads}_f{ffn_dim}_l{layers}"
            f"_{'causal' if causal else 'full'}_{_DTYPE_NAMES[dtype]}@{arch}")


def default_plan(batch: int, seq: int, d_model: int, heads: int, ffn_dim: int,
                 layers: int, causal: bool, dtype: torch.dtype, device: torch.device) -> Plan:
    """Heuristic plan used before (or without) autotuning."""
    if device.type != "cuda":
        raise RuntimeError("tjkernels runs on ROCm GPUs only; got device "
                           f"{device} (there is no CPU path)")
    # hipGraph replay pays only where launches dominate.  Measured on MI355X
    # (same box, alternating runs): C2 (128 x 512 activations) 0.186 ms with
    # the graph vs 0.222 ms eager, but C3 / C4 (3.1M / 8.4M activation
    # elements) 2-3% faster with eager stream launches, the kernels being
    # long enough to keep the queue ahead.  So the graph is used up to 2^20
    # activation elements, and never above the reference's 64 MiB of x
    # (tjkernels/plans.py:109-110).
    elems = batch * seq * d_model
    x_bytes = elems * dtype.itemsize
    return Plan(compute_dtype=dtype, residual_dtype=torch.float32,
                cuda_graph=elems <= (1 << 20) and x_bytes <= 64 * 1024 * 1024, label="heuristic")


_cache: Optional[Dict[str, Plan]] = None
_override: Optional[Plan] = None


def set_override(plan: Optional[Plan]) -> None:
    """Force a specific plan regardless of shape (used by the autotuner and tests)."""
    global _override
    _override = plan


def _load_tuned() -> Dict[str, Plan]:
    global _cache
    if _cache is None:
        _cache = {}
        if _PLAN_FILE.exists() and os.environ.get("TJ_IGNORE_PLANS") != "1":
            try:
                raw = json.loads(_PLAN_FILE.read_text())
                _cache = {k: Plan.from_json(v) for k, v in raw.items()}
            except Exception as exc:  # an unreadable table never breaks a run
                print(f"[tjkernels] ignoring unreadable plans.json: {exc}")
                _cache = {}
    return _cache


def select_plan(batch: int, seq: int, d_model: int, heads: int, ffn_dim: int,
                layers: int, causal: bool, dtype: torch.dtype, device: torch.device) -> Plan:
    if _override is not None:
        return _override
    arch = device_arch(device)
    key = shape_key(batch, seq, d_model, heads, ffn_dim, layers, causal, dtype, arch)
    tuned = _load_tuned().get(key)
    if tuned is not None:
        return tuned

    plan = default_plan(batch, seq, d_model, heads, ffn_dim, layers, causal, dtype, device)
    if os.environ.get("TJ_NO_GRAPH") == "1":
        plan = replace(plan, cuda_graph=False)
    forced = os.environ.get("TJ_COMPUTE_DTYPE")
    if forced in _DTYPES:
        plan = replace(plan, compute_dtype=_DTYPES[forced])
    if os.environ.get("TJ_DEFERRED_RESIDUAL") == "1":
        plan = replace(plan, residual_epilogue=False)
    if os.environ.get("TJ_NO_PACK") == "1":
        plan = replace(plan, pack_prefix=False)
    attn_plan = os.environ.get("TJ_ATTN_PLAN")
    if attn_plan is not None and attn_plan.lstrip("-").isdigit():
        plan = replace(plan, attn_plan=int(attn_plan))
    return plan


def save_plans(plans: Dict[str, Plan], path: Optional[Path] = None) -> None:
    """Merge ``plans`` into plans.json (existing keys for other shapes kept)."""
    global _cache
    path = path or _PLAN_FILE
    existing: Dict[str, object] = {}
    if path.exists():
        try:
            existing = json.loads(path.read_text())
        except Exception:
            existing = {}
    existing.update({k: v.to_json() for k, v in plans.items()})
    path.write_text(json.dumps(existing, indent=2, sort_keys=True) + "\n")
    _cache = None
