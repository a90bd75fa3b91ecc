"""Execution engine of the hook: the reference's tjkernels/engine.py:58-324.

An ``Engine`` lives on the module (set with ``object.__setattr__``, so the
``state_dict`` keeps the baseline's keys) and owns packed copies of the
module's parameters, never the parameters themselves.  A forward is a
pre-LN causal encoder over a residual stream ``res`` (fp32 unless
``Plan.residual_dtype`` says otherwise):

    res, h = x, LN1(x)                     layer 0: the first LayerNorm
    per layer:
        qkv  = h Wqkv^T + bqkv             one [3d, d] GEMM, rows q | k | v
        ctx  = attention(qkv viewed as [B, S, 3, H, hd])
        res += ctx Wo^T + bo               GEMM residual epilogue
              (``Plan.attn_block``, sequences of <= 128 tokens: the three
              in one launch, its per-head partials of ctx Wo^T + bo summed
              into res by LayerNorm 2)
        FFN:  "gemm"  -- h = LN2(res); mid = gelu_erf(h W1^T + b1) (GEMM
                         epilogue); res += mid W2^T + b2 (residual epilogue)
              "fused" -- one launch: LN2, both GEMMs and GELU with the
                         [T, f] intermediate in LDS; its f-slice partials
                         are summed by the next LayerNorm
        h = LN1 of the next layer (res [+ pending FFN partials])
    out = LN_final(res [+ pending]), padded rows exact zeros

``Plan.residual_epilogue=False`` writes the out-proj and FFN outputs in the
compute dtype and lets the following LayerNorm add them, the reference's
deferred-residual scheme (engine.py:232-264).  A 2-byte ``residual_dtype``
always runs that scheme (the GEMM epilogues add into fp32 only); the
LayerNorms store the updated residual rounded to it, and the fused FFN's
output goes through its partials buffer even unsplit.

Masks (reference engine.py:131-158): NONE -- no mask or every token valid;
PREFIX -- sequence b valid on its first len_b tokens; GENERAL -- anything
else.  PREFIX forwards pack the valid tokens: no valid row depends on a
padded one (under causal attention a valid query never sees a key at or past
its sequence's length, engine.py:147-150; without it the padded keys are
masked; every other op is row-wise), so the first LayerNorm gathers the
sum(len_b) valid rows into consecutive rows, every GEMM and LayerNorm runs on
those rows, attention runs on the packed sequences (cu_seqlens), and the
final LayerNorm scatters them back with the padded rows written as exact
zeros.  The reference computes the padded rows and zeroes them at the end
(engine.py:267-268); the valid rows come out the same.  GENERAL hands the
mask to attention as a per-key mask and zeroes padded rows at the end.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from dataclasses import dataclass
from typing import Dict, NamedTuple, Optional, Tuple

import torch

from . import ops, schedule as sched_mod, tiles
from .graphs import GraphCache
from .plans import ATTN_SCHEDULED, LN_GEMM_MAX_ROWS, Plan, attn_block_ok, fused_ffn_ok, select_plan

try:
    from torch.utils.weak import WeakTensorKeyDictionary
except ImportError:  # pragma: no cover - torch < 2.0
    WeakTensorKeyDictionary = None

MASK_NONE, MASK_PREFIX, MASK_GENERAL = 0, 1, 2


# --------------------------------------------------------------- weights

class Norm(NamedTuple):
    weight: torch.Tensor  # fp32 [d]
    bias: torch.Tensor    # fp32 [d]
    eps: float


class Linear(NamedTuple):
    weight: torch.Tensor  # compute dtype, nn.Linear [out, in]: the K-contiguous GEMM operand
    bias: torch.Tensor    # compute dtype [out]


class BlockWeights(NamedTuple):
    norm1: Norm
    qkv: Linear   # [3d, d]: q rows, then k, then v
    out: Linear
    norm2: Norm
    fc1: Linear   # [f, d]
    fc2: Linear   # [d, f]


class ModelWeights(NamedTuple):
    blocks: Tuple[BlockWeights, ...]
    final: Norm
    compute_dtype: torch.dtype


def _norm(ln: torch.nn.LayerNorm) -> Norm:
    return Norm(ln.weight.detach().float().contiguous(), ln.bias.detach().float().contiguous(), ln.eps)


def _linear(*layers: torch.nn.Linear, dtype: torch.dtype) -> Linear:
    weight = torch.cat([layer.weight.detach() for layer in layers], 0)
    bias = torch.cat([layer.bias.detach() for layer in layers], 0)
    return Linear(weight.to(dtype).contiguous(), bias.to(dtype).contiguous())


def pack_weights(module: torch.nn.Module, dtype: torch.dtype) -> ModelWeights:
    """Copies of the module's parameters in the layout the kernels take:
    matrices in the compute dtype (nn.Linear layout kept, q/k/v stacked into
    one [3d, d] operand), LayerNorm parameters in fp32."""
    blocks = []
    for blk in module.layers:
        at = blk.attention
        blocks.append(BlockWeights(
            norm1=_norm(blk.norm1),
            qkv=_linear(at.q_proj, at.k_proj, at.v_proj, dtype=dtype),
            out=_linear(at.out_proj, dtype=dtype),
            norm2=_norm(blk.norm2),
            fc1=_linear(blk.ffn_in, dtype=dtype),
            fc2=_linear(blk.ffn_out, dtype=dtype),
        ))
    return ModelWeights(tuple(blocks), _norm(module.final_norm), dtype)


# ------------------------------------------------------------------ masks

@dataclass(frozen=True)
class MaskInfo:
    mode: int
    lengths: Optional[Tuple[int, ...]] = None  # PREFIX only


def _version(t: torch.Tensor) -> Optional[int]:
    # inference tensors keep no version counter (torch raises on access)
    return None if t.is_inference() else t._version


class TensorMemo:
    """Host-side facts derived from a device tensor (one sync each),
    remembered per tensor object and recomputed when the tensor's version
    counter shows an in-place update since.  Tensors created under
    ``torch.inference_mode`` have no version counter, so an in-place update
    could not be seen: for them the facts are derived again on every call
    (one host sync per forward).  The reference memoises them per object
    (engine.py:139-141), where a stale entry only mislabels the mask mode;
    here a stale entry would be stale prefix lengths, i.e. wrong rows."""

    def __init__(self) -> None:
        self._memo = WeakTensorKeyDictionary() if WeakTensorKeyDictionary is not None else {}

    def get(self, t: torch.Tensor, derive):
        version = _version(t)
        if version is None:
            return derive(t)
        hit = self._memo.get(t)
        if hit is not None and hit[0] == version:
            return hit[1]
        value = derive(t)
        self._memo[t] = (version, value)
        return value


def classify_mask(mask: torch.Tensor) -> MaskInfo:
    """NONE / PREFIX (with the lengths) / GENERAL of a [B, S] bool mask."""
    seq = mask.shape[-1]
    counts = mask.sum(dim=-1)
    as_prefix = torch.arange(seq, device=mask.device)[None, :] < counts[:, None]
    if not bool(torch.equal(as_prefix, mask)):
        return MaskInfo(MASK_GENERAL)
    lengths = tuple(int(n) for n in counts.tolist())
    return MaskInfo(MASK_NONE) if min(lengths) == seq else MaskInfo(MASK_PREFIX, lengths)


def lengths_info(lengths: torch.Tensor, seq: int) -> MaskInfo:
    """MaskInfo of integer prefix lengths [B] (clamped to [0, seq])."""
    host = tuple(min(max(int(n), 0), seq) for n in lengths.tolist())
    return MaskInfo(MASK_NONE) if min(host, default=seq) == seq else MaskInfo(MASK_PREFIX, host)


# ---------------------------------------------------------------- packing

@dataclass
class Packing:
    """Row maps of one set of prefix lengths (device tensors, built once)."""

    lengths: Tuple[int, ...]
    tokens: int                  # sum(lengths): rows of the packed layout
    gather: torch.Tensor         # int32 [tokens]: [B*S] row of each packed row
    scatter: torch.Tensor        # int32 [B*S]: packed row of each output row, -1 = padding
    cu_seqlens: torch.Tensor     # int32 [B+1]
    attn: Optional[object] = None  # scheduled-attention work list (built on first use)


def build_packing(lengths: Tuple[int, ...], seq: int, device: torch.device) -> Packing:
    starts = [0]
    for n in lengths:
        starts.append(starts[-1] + n)
    if starts[-1]:
        gather = torch.cat([torch.arange(b * seq, b * seq + n, dtype=torch.int32) for b, n in enumerate(lengths)])
    else:
        gather = torch.zeros(0, dtype=torch.int32)
    scatter = torch.full((len(lengths) * seq,), -1, dtype=torch.int32)
    scatter[gather.long()] = torch.arange(starts[-1], dtype=torch.int32)
    return Packing(tuple(lengths), starts[-1], gather.to(device), scatter.to(device),
                   torch.tensor(starts, dtype=torch.int32, device=device))


# ---------------------------------------------------------------- forward

def ffn_slices(rows: int, ffn_dim: int) -> int:
    """f-slices of the single-launch FFN: 128 columns each, or 64 when 128
    would leave fewer than 32 workgroups of 32 rows (measured on MI355X: C2,
    128 rows and f = 2048, 16 slices 0.160 ms vs 32 slices 0.168 ms per
    forward; C1's fp32 FFN, 96 rows and f = 512, 9.7 us with 8 slices vs
    11.3 us with 4)."""
    blocks = -(-rows // 32)
    if ffn_dim % 128 == 0 and blocks * (ffn_dim // 128) >= 32:
        return ffn_dim // 128
    return max(ffn_dim // 64, 1)


class ModelShape(NamedTuple):
    d_model: int
    heads: int
    head_dim: int
    ffn_dim: int
    layers: int
    causal: bool


class Tiles(NamedTuple):
    qkv: int
    out: int
    fc1: int
    fc2: int
    qkv_ln: int = -1  # tjk_gemm_ln plans (LayerNorm inside the GEMM)
    fc1_ln: int = -1


@dataclass
class Workspace:
    """Activation buffers of one (B, S, plan), sized for every row."""

    res: torch.Tensor                # [T, d] residual stream (Plan.residual_dtype)
    h: torch.Tensor                  # [T, d] LayerNorm output
    qkv: torch.Tensor                # [T, 3d]
    ctx: torch.Tensor                # [T, d] attention output
    mid: Optional[torch.Tensor]      # [T, f] FFN intermediate (two-launch FFN)
    delta: Optional[torch.Tensor]    # [T, d] deferred block output (deferred plans)
    parts: Optional[torch.Tensor]    # [splits, T, d] fp32 FFN partials (fused FFN)
    attn_parts: Optional[torch.Tensor] = None  # [H, T, d] fp32 out-proj partials (attention block)


@dataclass
class Forward:
    """Static context of one forward shape: views of the processed rows,
    tile plans, the masks and packing it runs on."""

    batch: int
    seq: int
    mode: int
    rows: int
    ws: Workspace
    tiles: Tiles
    packing: Optional[Packing] = None
    key_mask: Optional[torch.Tensor] = None
    use_sched: bool = False
    use_block: bool = False
    ln_in_gemm: bool = False  # LayerNorms 1 (after layer 0) and 2 inside the QKV / FFN1 GEMMs
    # layer 0's out-proj adds x's rows itself, so the first LayerNorm writes
    # no residual (eager forwards: a graph would keep the first call's x)
    res_from_x: bool = False
    splits: int = 1
    pending: Optional[torch.Tensor] = None  # what the next LayerNorm adds to res

    def view(self, name: str) -> Optional[torch.Tensor]:
        t = getattr(self.ws, name)
        if t is None:
            return None
        return t[:, :self.rows] if name in ("parts", "attn_parts") else t[:self.rows]


class Engine:
    def __init__(self, module: torch.nn.Module) -> None:
        cfg = module.config
        first = next(module.parameters())
        self.module = module
        self.device, self.dtype = first.device, first.dtype
        self.shape = ModelShape(cfg.d_model, cfg.num_heads, cfg.d_model // cfg.num_heads, cfg.ffn_dim,
                                cfg.num_layers, cfg.causal)
        self.plan: Optional[Plan] = None
        self.weights: Optional[ModelWeights] = None
        self._plans: Dict[Tuple[int, int], Plan] = {}
        self._masks = TensorMemo()
        self._graphs = GraphCache()
        self._workspaces: Dict[Tuple, Workspace] = {}
        self._packings: "OrderedDict[Tuple[int, Tuple[int, ...]], Packing]" = OrderedDict()
        self._static_masks: Dict[Tuple[int, int], torch.Tensor] = {}
        self._forwards: "OrderedDict[Tuple, Forward]" = OrderedDict()
        self.check_waits = os.environ.get("TJ_CHECK_WAITS") == "1"

    # compatibility names used by tools and tests
    @property
    def d_model(self) -> int:
        return self.shape.d_model

    @property
    def num_heads(self) -> int:
        return self.shape.heads

    def _use_weights(self, plan: Plan) -> None:
        if self.weights is not None and self.weights.compute_dtype == plan.compute_dtype:
            return
        with torch.no_grad():
            self.weights = pack_weights(self.module, plan.compute_dtype)
        self._graphs.clear()
        self._forwards.clear()
        self._workspaces.clear()

    # -- masks and packing

    def _mask_info(self, mask: Optional[torch.Tensor]) -> Tuple[int, Optional[Tuple[int, ...]]]:
        """(mode, prefix lengths) of a [B, S] bool mask, one host sync per
        mask tensor and version."""
        if mask is None:
            return MASK_NONE, None
        info = self._masks.get(mask, classify_mask)
        return info.mode, info.lengths

    def _mask_mode(self, mask: Optional[torch.Tensor]) -> int:
        return self._mask_info(mask)[0]

    def _packing(self, lengths: Tuple[int, ...], seq: int) -> Packing:
        key = (seq, lengths)
        pk = self._packings.get(key)
        if pk is None:
            pk = build_packing(lengths, seq, self.device)
            self._packings[key] = pk
            if len(self._packings) > 64:
                self._packings.popitem(last=False)
        else:
            self._packings.move_to_end(key)
        return pk

    # -- per-shape preparation

    def _workspace(self, batch: int, seq: int, plan: Plan, splits: int, block: bool) -> Workspace:
        fused = plan.ffn == "fused"
        key = (batch, seq, plan.compute_dtype, plan.residual_dtype, plan.epilogue_residual, fused, splits, block)
        ws = self._workspaces.get(key)
        if ws is None:
            t, d, f = batch * seq, self.shape.d_model, self.shape.ffn_dim
            cdt, dev = plan.compute_dtype, self.device

            def buf(*dims, dtype=cdt):
                return torch.empty(dims, dtype=dtype, device=dev)

            # the fused FFN adds into an fp32 residual itself when unsplit
            use_parts = fused and (splits > 1 or plan.residual_dtype != torch.float32)
            ws = Workspace(res=buf(t, d, dtype=plan.residual_dtype), h=buf(t, d), qkv=buf(t, 3 * d), ctx=buf(t, d),
                           mid=None if fused else buf(t, f),
                           delta=None if plan.epilogue_residual else buf(t, d),
                           parts=buf(splits, t, d, dtype=torch.float32) if use_parts else None,
                           attn_parts=buf(self.shape.heads, t, d, dtype=torch.float32) if block else None)
            self._workspaces[key] = ws
        return ws

    def _prepare(self, batch: int, seq: int, mode: int, packing: Optional[Packing],
                 mask: Optional[torch.Tensor]) -> Forward:
        """Everything a forward needs besides x and its output.  Launches
        nothing except the one-time tile timing and schedule build of a new
        shape."""
        plan, shp = self.plan, self.shape
        fused = plan.ffn == "fused"
        rows = packing.tokens if mode == MASK_PREFIX else batch * seq
        splits = (plan.ffn_splits or ffn_slices(rows, shp.ffn_dim)) if fused else 1
        cdt, d, f = plan.compute_dtype, shp.d_model, shp.ffn_dim
        # the one-launch attention block takes no per-key mask and
        # sequences of at most 128 tokens; other forwards of the plan run the
        # QKV GEMM, attention and out-proj GEMM
        longest = max(packing.lengths) if mode == MASK_PREFIX else seq
        block = (plan.attn_block and mode != MASK_GENERAL and rows > 0
                 and attn_block_ok(longest, d, shp.heads, cdt))
        epi_res = ops.EPI_BIAS_RESIDUAL if plan.epilogue_residual else ops.EPI_BIAS
        # LayerNorm inside the QKV / FFN1 GEMMs needs nothing pending for
        # either LayerNorm: residual epilogues, the two-launch FFN and no
        # attention block
        ln_in = (plan.ln_gemm and plan.epilogue_residual and not fused and not block
                 and 0 < rows <= LN_GEMM_MAX_ROWS and ops.gemm_ln_supported(d, cdt))
        # a plan's tiles hold at the row count they were measured at (or at
        # every row count with tile_rows 0); other row counts time their own
        row_bucket = -(-rows // tiles.M_BUCKET) * tiles.M_BUCKET

        def pin(tile: int) -> int:
            return tile if plan.tile_rows in (0, row_bucket) else -1

        tp = Tiles(
            qkv=-1 if block else tiles.gemm_plan(rows, 3 * d, d, cdt, ops.EPI_BIAS, pin(plan.gemm_qkv)),
            out=-1 if block else tiles.gemm_plan(rows, d, d, cdt, epi_res, pin(plan.gemm_out)),
            fc1=-1 if fused or ln_in else tiles.gemm_plan(rows, f, d, cdt, ops.EPI_BIAS_GELU, pin(plan.gemm_ffn1)),
            fc2=-1 if fused else tiles.gemm_plan(rows, d, f, cdt, epi_res, pin(plan.gemm_ffn2)),
            qkv_ln=tiles.gemm_ln_plan(rows, 3 * d, d, cdt, ops.EPI_BIAS) if ln_in else -1,
            fc1_ln=tiles.gemm_ln_plan(rows, f, d, cdt, ops.EPI_BIAS_GELU) if ln_in else -1)
        fw = Forward(batch=batch, seq=seq, mode=mode, rows=rows,
                     ws=self._workspace(batch, seq, plan, splits, block), tiles=tp,
                     packing=packing if mode == MASK_PREFIX else None,
                     key_mask=mask if mode == MASK_GENERAL else None, use_block=block, splits=splits,
                     ln_in_gemm=ln_in,
                     res_from_x=(plan.epilogue_residual and not plan.cuda_graph and not block
                                 and cdt == self.dtype))
        if fused:
            fw.pending = fw.view("parts")
        elif not plan.epilogue_residual:
            fw.pending = fw.view("delta")
        # Packed 2-byte attention of 129 to 2047 keys follows a longest-first
        # work list (attn_plan -1, or ATTN_SCHEDULED to force it); longer
        # sequences run the plain plan-0/1 kernel, measured faster there, and
        # sequences of at most 128 keys the short-sequence plan 4; other plan
        # ids force the plain kernel.
        pk = fw.packing
        fw.use_sched = (pk is not None and cdt != torch.float32 and rows > 0 and not block
                        and (plan.attn_plan == ATTN_SCHEDULED
                             or (plan.attn_plan == -1 and 128 < max(pk.lengths) < 2048)))
        if fw.use_sched and pk.attn is None:
            pk.attn = sched_mod.build_schedule(pk.lengths, shp.heads, shp.head_dim, shp.causal, cdt, self.device)
        return fw

    # -- the launches

    def _first(self, fw: Forward, x: torch.Tensor) -> None:
        """Layer-0 LN1: reads x (gathering the valid rows of a prefix mask),
        writes h, and the residual unless layer 0's out-proj reads x."""
        n1 = self.weights.blocks[0].norm1
        gather = fw.packing.gather if fw.packing is not None else None
        ops.add_layernorm(x.reshape(fw.batch * fw.seq, self.shape.d_model), None, n1.weight, n1.bias, n1.eps,
                          fw.view("h"), res_out=None if fw.res_from_x else fw.view("res"), row_index=gather)

    def _attention(self, fw: Forward) -> None:
        shp = self.shape
        qkv, ctx, pk = fw.view("qkv"), fw.view("ctx"), fw.packing
        if fw.use_sched:
            ops.flash_attention_sched(qkv.view(fw.rows, 3, shp.heads, shp.head_dim), ctx, pk.cu_seqlens,
                                      max(pk.lengths), pk.attn, causal=shp.causal)
        elif pk is not None:
            ops.flash_attention(qkv.view(fw.rows, 3, shp.heads, shp.head_dim), ctx, causal=shp.causal,
                                plan=self.plan.attn_plan, cu_seqlens=pk.cu_seqlens, max_seqlen=max(pk.lengths))
        else:
            ops.flash_attention(qkv.view(fw.batch, fw.seq, 3, shp.heads, shp.head_dim), ctx, causal=shp.causal,
                                key_mask=fw.key_mask, plan=self.plan.attn_plan)

    def _attn_block(self, fw: Forward, blk: BlockWeights) -> None:
        """QKV GEMM, attention and out-projection in one launch; the
        out-projection's per-head partials go to attn_parts."""
        shp, pk = self.shape, fw.packing
        args = (fw.view("h"), blk.qkv.weight, blk.qkv.bias, blk.out.weight, blk.out.bias, fw.view("attn_parts"),
                shp.heads)
        if pk is not None:
            ops.attn_block(*args, causal=shp.causal, cu_seqlens=pk.cu_seqlens, max_seqlen=max(pk.lengths))
        else:
            ops.attn_block(*args, causal=shp.causal, batch=fw.batch, seq=fw.seq)

    def _ffn(self, fw: Forward, blk: BlockWeights) -> None:
        plan = self.plan
        res, h, n2 = fw.view("res"), fw.view("h"), blk.norm2
        # the attention output not yet in res: the attention block's
        # partials, or the deferred out-proj output
        attn_pending = fw.view("attn_parts") if fw.use_block else (
            None if plan.epilogue_residual else fw.view("delta"))
        if plan.ffn == "fused":
            parts = fw.view("parts")
            if attn_pending is None:
                ln, a = (n2.weight, n2.bias, n2.eps), res  # LayerNorm 2 inside the kernel
            else:
                ops.add_layernorm(res, attn_pending, n2.weight, n2.bias, n2.eps, h, res_out=res)
                ln, a = None, h
            if parts is None:
                ops.ffn(a, blk.fc1.weight, blk.fc1.bias, blk.fc2.weight, blk.fc2.bias, res, ln=ln, accumulate=True)
            else:
                ops.ffn(a, blk.fc1.weight, blk.fc1.bias, blk.fc2.weight, blk.fc2.bias, parts, splits=fw.splits,
                        ln=ln)
            return
        mid = fw.view("mid")
        if plan.epilogue_residual:
            if fw.ln_in_gemm:  # LayerNorm 2 inside the FFN1 GEMM
                ops.gemm_ln(res, n2.weight, n2.bias, n2.eps, blk.fc1.weight, blk.fc1.bias, mid,
                            ops.EPI_BIAS_GELU, fw.tiles.fc1_ln)
            else:
                ops.add_layernorm(res, attn_pending, n2.weight, n2.bias, n2.eps, h,
                                  res_out=res if attn_pending is not None else None)
                ops.gemm(h, blk.fc1.weight, blk.fc1.bias, mid, ops.EPI_BIAS_GELU, fw.tiles.fc1)
            ops.gemm(mid, blk.fc2.weight, blk.fc2.bias, res, ops.EPI_BIAS_RESIDUAL, fw.tiles.fc2)
        else:
            delta = fw.view("delta")
            ops.add_layernorm(res, attn_pending, n2.weight, n2.bias, n2.eps, h, res_out=res)
            ops.gemm(h, blk.fc1.weight, blk.fc1.bias, mid, ops.EPI_BIAS_GELU, fw.tiles.fc1)
            ops.gemm(mid, blk.fc2.weight, blk.fc2.bias, delta, ops.EPI_BIAS, fw.tiles.fc2)

    def _body(self, fw: Forward, x: Optional[torch.Tensor] = None) -> None:
        """Every layer between the first LayerNorm and the final one: the
        part the hipGraph captures (fixed buffers only).  With
        ``fw.res_from_x`` layer 0's out-proj forms the residual from the
        forward's input ``x`` (residual = x[gather] + attn_out, the sum the
        first LayerNorm's residual write and the residual epilogue form)."""
        res, h, ctx = fw.view("res"), fw.view("h"), fw.view("ctx")
        if fw.res_from_x and x is None:
            raise RuntimeError("this forward's first layer reads x: pass it to _body")
        for i, blk in enumerate(self.weights.blocks):
            # LayerNorm 1 of the layers after the first: inside the QKV GEMM,
            # or a launch of its own
            ln_qkv = i > 0 and fw.ln_in_gemm
            if i > 0 and not ln_qkv:
                n1 = blk.norm1
                ops.add_layernorm(res, fw.pending, n1.weight, n1.bias, n1.eps, h,
                                  res_out=res if fw.pending is not None else None)
            if fw.use_block:
                self._attn_block(fw, blk)
            else:
                if ln_qkv:
                    n1 = blk.norm1
                    ops.gemm_ln(res, n1.weight, n1.bias, n1.eps, blk.qkv.weight, blk.qkv.bias, fw.view("qkv"),
                                ops.EPI_BIAS, fw.tiles.qkv_ln)
                else:
                    ops.gemm(h, blk.qkv.weight, blk.qkv.bias, fw.view("qkv"), ops.EPI_BIAS, fw.tiles.qkv)
                self._attention(fw)
                if i == 0 and fw.res_from_x:
                    ops.gemm_residual_from(ctx, blk.out.weight, blk.out.bias, res,
                                           x.reshape(fw.batch * fw.seq, self.shape.d_model),
                                           rows=fw.packing.gather if fw.packing is not None else None,
                                           plan=fw.tiles.out)
                elif self.plan.epilogue_residual:
                    ops.gemm(ctx, blk.out.weight, blk.out.bias, res, ops.EPI_BIAS_RESIDUAL, fw.tiles.out)
                else:
                    ops.gemm(ctx, blk.out.weight, blk.out.bias, fw.view("delta"), ops.EPI_BIAS, fw.tiles.out)
            self._ffn(fw, blk)

    def _final(self, fw: Forward, out: torch.Tensor, row_mask: Optional[torch.Tensor]) -> None:
        """Final LayerNorm into the output, padded rows as exact zeros."""
        fin = self.weights.final
        scatter = fw.packing.scatter if fw.packing is not None else None
        ops.add_layernorm(fw.view("res"), fw.pending, fin.weight, fin.bias, fin.eps,
                          out.view(fw.batch * fw.seq, self.shape.d_model), row_mask=row_mask, row_index=scatter)

    def _forward_impl(self, x: torch.Tensor, mask: Optional[torch.Tensor], mode: int,
                      packing: Optional[Packing] = None) -> torch.Tensor:
        """Eager forward (no graph)."""
        batch, seq, d = x.shape
        fw = self._prepare(batch, seq, mode, packing, mask)
        out = torch.empty((batch, seq, d), dtype=self.dtype, device=x.device)
        self._first(fw, x)
        self._body(fw, x)
        self._final(fw, out, mask.reshape(-1) if mode == MASK_GENERAL else None)
        self._check(fw)
        return out

    def _check(self, fw: Forward) -> None:
        """With TJ_CHECK_WAITS=1: raise if the scheduled attention's error
        word counted a timed-out wait or an invalid item (a host sync)."""
        if self.check_waits and fw.use_sched:
            n = sched_mod.error_count(fw.packing.attn)
            if n:
                raise RuntimeError(f"tjkernels: scheduled attention reported {n} failed items "
                                   "(timed-out waits or invalid work items); the output holds NaN rows")

    # -- the call

    def _decode_mask(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> Tuple[Optional[torch.Tensor], MaskInfo]:
        """The hook's second argument: None, a [B, S] bool-like mask, or
        integer prefix lengths [B]."""
        batch, seq = x.shape[:2]
        if mask is None:
            return None, MaskInfo(MASK_NONE)
        if mask.dim() == 1 and not mask.dtype.is_floating_point and mask.dtype != torch.bool:
            if mask.shape[0] != batch:
                raise ValueError(f"lengths must be [B], got {tuple(mask.shape)}")
            return None, self._masks.get(mask, lambda t: lengths_info(t, seq))
        if tuple(mask.shape) != (batch, seq):
            raise ValueError(f"valid_token_mask must be [B, S], got {tuple(mask.shape)}")
        if mask.dtype != torch.bool:
            mask = mask.to(torch.bool)
        if not mask.is_contiguous():
            mask = mask.contiguous()
        return mask, self._masks.get(mask, classify_mask)

    def __call__(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError(f"tjkernels runs on ROCm GPUs only (input on {x.device}); there is no CPU path")
        if x.dim() != 3 or x.shape[-1] != self.shape.d_model:
            raise ValueError(f"expected x of shape [B, S, {self.shape.d_model}], got {tuple(x.shape)}")
        if x.dtype != self.dtype:
            raise ValueError(f"x dtype {x.dtype} != model dtype {self.dtype}")
        if not x.is_contiguous():
            x = x.contiguous()
        mask, info = self._decode_mask(x, mask)
        batch, seq, _ = x.shape
        plan = self._plans.get((batch, seq))
        if plan is None:
            shp = self.shape
            plan = select_plan(batch, seq, shp.d_model, shp.heads, shp.ffn_dim, shp.layers, shp.causal,
                               self.dtype, self.device)
            plan.validate()
            if plan.ffn == "fused" and not fused_ffn_ok(shp.d_model, shp.ffn_dim, plan.compute_dtype,
                                                        plan.ffn_splits):
                raise ValueError(f"plan {plan.label!r}: the single-launch FFN has no kernel for d={shp.d_model}, "
                                 f"f={shp.ffn_dim}, {plan.compute_dtype} (see tjk_ffn_supported)")
            self._plans[(batch, seq)] = plan
        self.plan = plan
        self._use_weights(plan)
        mode, lengths = info.mode, info.lengths
        if mode == MASK_PREFIX and not plan.pack_prefix:
            # every row computed with a per-key mask, the reference's way
            if mask is None:
                mask = torch.arange(seq, device=x.device)[None, :] < torch.tensor(lengths, device=x.device)[:, None]
            mode, lengths = MASK_GENERAL, None
        packing = self._packing(lengths, seq) if mode == MASK_PREFIX else None
        if plan.cuda_graph:
            return self._forward_graph(x, mask, mode, lengths, packing)
        return self._forward_impl(x, mask, mode, packing)

    def _forward_graph(self, x: torch.Tensor, mask: Optional[torch.Tensor], mode: int,
                       lengths: Optional[Tuple[int, ...]], packing: Optional[Packing]) -> torch.Tensor:
        """The first LayerNorm (reading the caller's x) and the final one
        (writing a fresh output) run on the stream around one replayed
        hipGraph of the layer body, on fixed workspace buffers; only a
        GENERAL mask, which the recorded attention reads, is copied into a
        static buffer.  With ``plan.whole_graph`` both LayerNorms are in the
        graph too: x is copied into a static input and the static output is
        cloned, one graph launch per forward.  A packed forward's launches
        are sized by its lengths, so the lengths are part of the key, and the
        graph keeps the row maps and schedule it reads alive."""
        batch, seq, d = x.shape
        static_mask = None
        if mode == MASK_GENERAL:
            static_mask = self._static_masks.get((batch, seq))
            if static_mask is None:
                static_mask = torch.empty((batch, seq), dtype=torch.bool, device=x.device)
                self._static_masks[(batch, seq)] = static_mask
            static_mask.copy_(mask)
        key = (batch, seq, x.dtype, mode, lengths, self.plan)
        fw = self._forwards.get(key)
        if fw is None:
            fw = self._prepare(batch, seq, mode, packing, static_mask)
            self._forwards[key] = fw
            if len(self._forwards) > 4 * self._graphs.max_entries:
                self._forwards.popitem(last=False)
        row_mask = static_mask.reshape(-1) if mode == MASK_GENERAL else None
        if self.plan.whole_graph:
            return self._forward_whole_graph(x, fw, key, packing, row_mask)
        graph = self._graphs.get(key, lambda: self._body(fw), keepalive=(packing, fw))
        self._first(fw, x)
        if graph is not None:
            graph.replay()
        else:
            self._body(fw)
        out = torch.empty((batch, seq, d), dtype=self.dtype, device=x.device)
        self._final(fw, out, row_mask)
        self._check(fw)
        return out

    def _forward_whole_graph(self, x: torch.Tensor, fw: Forward, key: Tuple, packing: Optional[Packing],
                             row_mask: Optional[torch.Tensor]) -> torch.Tensor:
        """One replay of a graph that holds both LayerNorms too: x is copied
        into the graph's static input and its static output is cloned.  The
        static buffers are part of the graph entry (its keepalive), so they
        are evicted together with the graph and never separately: a replay
        always reads and writes the buffers it was captured on."""
        found, graph = self._graphs.lookup(key)
        if found and graph is not None:
            _, fw_g, (x_in, y_out) = graph.keepalive
            x_in.copy_(x)
            graph.replay()
            self._check(fw_g)
            return y_out.clone()
        if found:  # the capture failed before: eager launches on fresh buffers
            out = torch.empty_like(x)
            self._first(fw, x)
            self._body(fw)
            self._final(fw, out, row_mask)
            self._check(fw)
            return out
        io = (torch.empty_like(x), torch.empty_like(x))
        x_in, y_out = io

        def whole() -> None:
            self._first(fw, x_in)
            self._body(fw)
            self._final(fw, y_out, row_mask)

        x_in.copy_(x)
        graph = self._graphs.get(key, whole, keepalive=(packing, fw, io))
        if graph is not None:
            graph.replay()
        else:
            whole()
        self._check(fw)
        return y_out.clone()


def get_engine(module: torch.nn.Module) -> Engine:
    """The module's engine, made on first use and again after the module
    moved to another dtype or device."""
    engine = getattr(module, "_tj_engine", None)
    first = next(module.parameters())
    if engine is None or (engine.dtype, engine.device) != (first.dtype, first.device):
        engine = Engine(module)
        object.__setattr__(module, "_tj_engine", engine)
    return engine


def reset_engines(module: torch.nn.Module) -> None:
    if hasattr(module, "_tj_engine"):
        object.__delattr__(module, "_tj_engine")


def forward(module: torch.nn.Module, x: torch.Tensor,
            valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The hook body: ``return tjkernels.forward(self, x, valid_token_mask)``
    (torch_transformer_benchmark.py:203).  ``TJ_DISABLE=1`` runs the parent
    class's forward instead (engine.py:322-323)."""
    if os.environ.get("TJ_DISABLE") == "1":
        return super(type(module), module).forward(x, valid_token_mask)
    return get_engine(module)(x, valid_token_mask)
