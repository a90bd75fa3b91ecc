"""Shape -> execution-plan dispatch (the reference's tjkernels/plans.py:29-198).

A ``Plan`` is a frozen bundle of knobs for one (shape, dtype, architecture).
``select_plan`` resolves it in this order:

1. a plan forced with ``set_override`` (the autotuner and tests use it);
2. the tuned entry for the shape key in ``plans.json`` (written by
   ``tjkernels.autotune``; skipped with ``TJ_IGNORE_PLANS=1``);
3. ``default_plan``'s heuristic, adjusted by the ``TJ_*`` environment knobs
   below (so ablations run with ``TJ_IGNORE_PLANS=1``, as the reference's
   ablation does).

Knobs, all naming HIP kernels of this build (there is no torch/SDPA backend
to select, and the product path has no non-HIP fallback):

* ``compute_dtype`` / ``residual_dtype``: GEMM / attention operand dtype and
  the residual stream's dtype.  An fp32 model runs the IEEE fp32 plan, since
  only fp32 compute holds the 1e-4 budget of fp32 plans.  A 2-byte residual
  stream (fp16 / bf16, the reference's knob, tjkernels/plans.py:33-36) runs
  the deferred scheme whatever ``residual_epilogue`` says: the projections
  write the compute dtype and each LayerNorm adds, normalises the fp32 sum and
  stores the residual rounded (tjkernels/kernels/layernorm.py:50-60);
* ``ffn``: ``"gemm"`` (two GEMM launches, GELU in the first one's epilogue,
  the [T, f] intermediate in HBM) or ``"fused"`` (one launch per layer with
  the intermediate in LDS and LayerNorm 2 inside, split over ``ffn_splits``
  f-slices whose partials the next LayerNorm sums; 0 = f / 128);
* ``attn_block``: for sequences of at most 128 tokens, the QKV GEMM,
  attention and out-projection of each layer as one launch
  (``tjk_attn_block``) whose per-head partials LayerNorm 2 sums; forwards
  it does not take (longer sequences, general masks) use the three
  launches;
* ``ln_gemm``: compute LayerNorm 1 (layers after the first) and LayerNorm 2
  inside the QKV and FFN1 GEMMs (``tjk_gemm_ln``) instead of as launches of
  their own, where nothing is pending for them (residual epilogues, the
  two-launch FFN, no attention block) and the forward has at most
  ``LN_GEMM_MAX_ROWS`` rows, since every column tile recomputes its rows'
  LayerNorm;
* ``cuda_graph``: replay the layer body as one hipGraph;
* ``whole_graph`` (with ``cuda_graph``): capture the first and final
  LayerNorm too, reading x from a static input buffer and writing a static
  output that is cloned -- the reference's copy-in / clone-out
  (graphs.py:57-64): one graph launch and two copies per forward instead of
  two eager LayerNorm launches around the replayed body;
* ``residual_epilogue``: add the out-proj (and two-launch FFN) outputs into
  the fp32 residual in the GEMM epilogue instead of deferring them to the
  next LayerNorm (the reference's scheme, engine.py:232-264); fp32 residual
  only;
* ``gemm_*`` / ``attn_plan``: force a tile or attention plan (-1: chosen
  at run time; attention 0-4 are the library's plans of tjk_flash_fwd,
  ``ATTN_SCHEDULED`` (5) the work-list kernel for packed sequences);
* ``tile_rows``: the packed row count (a multiple of ``tiles.M_BUCKET``)
  the ``gemm_*`` tiles were measured at by the autotuner, inside whole
  forwards; a forward whose row count rounds up to another value times its
  own tiles as if they were -1.  0 applies them at every row count;
* ``pack_prefix``: run only the valid tokens of prefix masks.

Environment: ``TJ_NO_GRAPH``, ``TJ_WHOLE_GRAPH`` (0 / 1), ``TJ_ATTN_BLOCK`` (0 / 1), ``TJ_LN_GEMM`` (0 / 1),
``TJ_COMPUTE_DTYPE``,
``TJ_RESIDUAL_DTYPE``, ``TJ_DEFERRED_RESIDUAL`` (0 / 1), ``TJ_NO_PACK``, ``TJ_ATTN_PLAN``, ``TJ_FFN`` (gemm | fused), ``TJ_FFN_SPLITS``;
``TJ_GEMM_TUNE=0`` (tjkernels.tiles) skips the measured tile choice.
Tuned keys carry the GPU architecture (``...@gfx950``).
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass, fields, replace
from pathlib import Path
from typing import Dict, Optional

import torch

DTYPE_BY_NAME = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
NAME_BY_DTYPE = {dt: name for name, dt in DTYPE_BY_NAME.items()}
FFN_KINDS = ("gemm", "fused")
# attn_plan id beyond the library's tjk_flash_fwd plans (0-4): the scheduled
# work-list kernel for packed sequences (tjk_flash_fwd_sched)
ATTN_SCHEDULED = 5

# The single-launch FFN is the default up to this many (tokens x ffn_dim)
# elements of intermediate, where the two-launch path is launch-bound.
# Measured on MI355X: C1 (2^16 elements, fp32) 0.075 ms fused against
# 0.097 ms with two launches; C2 (2^18) 0.147 against 0.140 ms, since the
# 32-row K-split GEMM tiles made the two launches cheaper.
FUSED_FFN_MAX_ELEMS = 1 << 17

# The LayerNorm GEMM (Plan.ln_gemm) recomputes each row's LayerNorm once per
# 32-column tile, so the engine applies it up to this many rows only (C2:
# 128); at C4's 5430 rows it measured 2.31 against 0.89 ms per forward.
LN_GEMM_MAX_ROWS = 512


@dataclass(frozen=True)
class Plan:
    """Execution knobs for one (shape, dtype, architecture)."""

    compute_dtype: torch.dtype = torch.bfloat16
    residual_dtype: torch.dtype = torch.float32
    attn: str = "hip"
    ffn: str = "gemm"
    norm: str = "hip"
    ffn_splits: int = 0
    packed_qkv: bool = True
    cuda_graph: bool = True
    whole_graph: bool = False
    attn_block: bool = False
    ln_gemm: bool = False
    residual_epilogue: bool = True
    gemm_qkv: int = -1
    gemm_out: int = -1
    gemm_ffn1: int = -1
    gemm_ffn2: int = -1
    tile_rows: int = 0
    attn_plan: int = -1
    pack_prefix: bool = True
    label: str = "default"

    def to_json(self) -> Dict[str, object]:
        blob: Dict[str, object] = {}
        for f in fields(self):
            value = getattr(self, f.name)
            blob[f.name] = NAME_BY_DTYPE[value] if isinstance(value, torch.dtype) else value
        return blob

    @classmethod
    def from_json(cls, blob: Dict[str, object]) -> "Plan":
        known = {f.name: f for f in fields(cls)}
        kwargs = {}
        for name, value in blob.items():
            if name not in known:
                continue  # keys of other versions are ignored
            if name in ("compute_dtype", "residual_dtype"):
                value = DTYPE_BY_NAME[str(value)]
            if name == "ffn" and value == "hip":
                value = "gemm"  # the two-launch FFN's name in earlier tables
            kwargs[name] = value
        return cls(**kwargs)

    @property
    def epilogue_residual(self) -> bool:
        """Whether the GEMM epilogues add into the residual (fp32 only)."""
        return self.residual_epilogue and self.residual_dtype == torch.float32

    def validate(self) -> None:
        if self.residual_dtype not in NAME_BY_DTYPE:
            raise ValueError(f"residual_dtype={self.residual_dtype}: one of {sorted(DTYPE_BY_NAME)}")
        if self.attn != "hip" or self.norm != "hip":
            raise ValueError(f"attn={self.attn!r} norm={self.norm!r}: only 'hip' kernels exist "
                             "(no torch/SDPA fallback in this build)")
        if self.ffn not in FFN_KINDS:
            raise ValueError(f"ffn={self.ffn!r}: one of {FFN_KINDS}")
        if not self.packed_qkv:
            raise ValueError("only the packed QKV layout is implemented")
        if self.tile_rows < 0:
            raise ValueError(f"tile_rows={self.tile_rows}: a row count >= 0")


def device_arch(device: torch.device) -> str:
    if device.type != "cuda":
        return device.type
    return torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]


def shape_key(batch: int, seq: int, d_model: int, heads: int, ffn_dim: int,
              layers: int, causal: bool, dtype: torch.dtype, arch: str = "gfx950") -> str:
    mode = "causal" if causal else "full"
    return f"b{batch}_s{seq}_d{d_model}_h{heads}_f{ffn_dim}_l{layers}_{mode}_{NAME_BY_DTYPE[dtype]}@{arch}"


def fused_ffn_ok(d_model: int, ffn_dim: int, compute_dtype: torch.dtype, splits: int = 0) -> bool:
    """Whether the single-launch FFN kernel takes the shape (tjk_ffn_supported):
    ``splits`` slices, or with 0 both slice widths the engine may pick."""
    from . import ops
    if splits > 0:
        return ops.ffn_supported(d_model, ffn_dim, splits, compute_dtype)
    return all(ops.ffn_supported(d_model, ffn_dim, max(ffn_dim // w, 1), compute_dtype) for w in (64, 128))


def attn_block_ok(seq: int, d_model: int, heads: int, compute_dtype: torch.dtype) -> bool:
    """Whether the one-launch attention block takes the shape
    (tjk_attn_block_supported)."""
    from . import ops
    return d_model % heads == 0 and ops.attn_block_supported(d_model, heads, d_model // heads, seq, compute_dtype)


def default_plan(batch: int, seq: int, d_model: int, heads: int, ffn_dim: int,
                 layers: int, causal: bool, dtype: torch.dtype, device: torch.device) -> Plan:
    """Heuristic plan used before (or without) autotuning."""
    if device.type != "cuda":
        raise RuntimeError(f"tjkernels runs on ROCm GPUs only; got device {device} (there is no CPU path)")
    # hipGraph replay pays only where launches dominate: measured on MI355X,
    # C2 (128 x 512 activations) 0.186 ms replayed vs 0.222 ms eager, but
    # C3 / C4 (3.1M / 8.4M activation elements) 2-3% faster launched
    # eagerly.  So up to 2^20 activation elements, and never above the
    # reference's 64 MiB of x (tjkernels/plans.py:109-110).
    elems = batch * seq * d_model
    graph = elems <= (1 << 20) and elems * dtype.itemsize <= 64 * 1024 * 1024
    fused = batch * seq * ffn_dim <= FUSED_FFN_MAX_ELEMS and fused_ffn_ok(d_model, ffn_dim, dtype)
    # The one-launch attention block is not the default: measured on MI355X
    # at C2 it runs 15.1 us per layer, which with the LayerNorm launch that
    # sums its per-head partials equals the QKV GEMM + attention + out-proj
    # it replaces (0.1527 vs 0.1530 ms per forward); the autotuner tries it.
    # The out-proj / FFN2 outputs are added into the fp32 residual in the
    # GEMM epilogue, not deferred to the next LayerNorm in the compute dtype
    # (the reference's scheme): deferring measured ~1% faster at C4 (0.879
    # against 0.887 ms) but rounds each projection output once more, and the
    # autotuner's accuracy gate put its worst element at 78% of the budget
    # against 69% (C5: 59% against 39%).
    return Plan(compute_dtype=dtype, cuda_graph=graph, ffn="fused" if fused else "gemm", label="heuristic")


class PlanTable:
    """The tuned plans of ``plans.json``, read once, keyed by ``shape_key``."""

    def __init__(self, path: Path) -> None:
        self.path = path
        self._plans: Optional[Dict[str, Plan]] = None

    def plans(self) -> Dict[str, Plan]:
        if self._plans is None:
            self._plans = {}
            if os.environ.get("TJ_IGNORE_PLANS") != "1" and self.path.exists():
                try:
                    raw = json.loads(self.path.read_text())
                    self._plans = {key: Plan.from_json(blob) for key, blob in raw.items()}
                except (OSError, ValueError, KeyError, TypeError) as exc:
                    # a broken table costs the tuning, never the run
                    print(f"[tjkernels] plans.json not used ({exc})")
        return self._plans

    def get(self, key: str) -> Optional[Plan]:
        return self.plans().get(key)

    def merge(self, new: Dict[str, Plan], path: Optional[Path] = None) -> None:
        """Write ``new`` into the table file, keeping other shapes' entries."""
        target = path or self.path
        table: Dict[str, object] = {}
        if target.exists():
            try:
                table = json.loads(target.read_text())
            except ValueError:
                table = {}
        for key, plan in new.items():
            table[key] = plan.to_json()
        target.write_text(json.dumps(table, indent=2, sort_keys=True) + "\n")
        self._plans = None


TUNED_PATH = Path(__file__).with_name("plans.json")
TUNED = PlanTable(TUNED_PATH)
_forced: Optional[Plan] = None


def set_override(plan: Optional[Plan]) -> None:
    """Force ``plan`` for every shape (None lifts it)."""
    global _forced
    _forced = plan


def _env_adjusted(plan: Plan, d_model: int, ffn_dim: int) -> Plan:
    env = os.environ
    changes: Dict[str, object] = {}
    if env.get("TJ_NO_GRAPH") == "1":
        changes["cuda_graph"] = False
    if env.get("TJ_WHOLE_GRAPH") in ("0", "1"):
        changes["whole_graph"] = env["TJ_WHOLE_GRAPH"] == "1"
    if env.get("TJ_ATTN_BLOCK") in ("0", "1"):
        changes["attn_block"] = env["TJ_ATTN_BLOCK"] == "1"
    if env.get("TJ_LN_GEMM") in ("0", "1"):
        changes["ln_gemm"] = env["TJ_LN_GEMM"] == "1"
    if env.get("TJ_COMPUTE_DTYPE") in DTYPE_BY_NAME:
        changes["compute_dtype"] = DTYPE_BY_NAME[env["TJ_COMPUTE_DTYPE"]]
    if env.get("TJ_RESIDUAL_DTYPE") in DTYPE_BY_NAME:
        changes["residual_dtype"] = DTYPE_BY_NAME[env["TJ_RESIDUAL_DTYPE"]]
    if env.get("TJ_DEFERRED_RESIDUAL") in ("0", "1"):
        changes["residual_epilogue"] = env["TJ_DEFERRED_RESIDUAL"] == "0"
    if env.get("TJ_NO_PACK") == "1":
        changes["pack_prefix"] = False
    if env.get("TJ_FFN") in FFN_KINDS:
        changes["ffn"] = env["TJ_FFN"]
    splits = env.get("TJ_FFN_SPLITS", "")
    if splits.isdigit():
        changes["ffn_splits"] = int(splits)
    attn = env.get("TJ_ATTN_PLAN", "")
    if attn.lstrip("-").isdigit():
        changes["attn_plan"] = int(attn)
    out = replace(plan, **changes) if changes else plan
    # a compute dtype the single-launch FFN has no kernel for (fp32 at
    # d = 512) falls back to the two-launch FFN unless TJ_FFN forces it
    if (out.ffn == "fused" and "ffn" not in changes
            and not fused_ffn_ok(d_model, ffn_dim, out.compute_dtype, out.ffn_splits)):
        out = replace(out, ffn="gemm")
    return out


def select_plan(batch: int, seq: int, d_model: int, heads: int, ffn_dim: int,
                layers: int, causal: bool, dtype: torch.dtype, device: torch.device) -> Plan:
    if _forced is not None:
        return _forced
    key = shape_key(batch, seq, d_model, heads, ffn_dim, layers, causal, dtype, device_arch(device))
    tuned = TUNED.get(key)
    if tuned is not None:
        return tuned
    return _env_adjusted(default_plan(batch, seq, d_model, heads, ffn_dim, layers, causal, dtype, device),
                         d_model, ffn_dim)


def save_plans(plans: Dict[str, Plan], path: Optional[Path] = None) -> None:
    """Merge ``plans`` into plans.json (entries for other shapes are kept)."""
    TUNED.merge(plans, path)
