"""Execution engine: packs weights once, then runs the plan's HIP kernels.

Mirrors the reference engine (tjkernels/engine.py:58-324): a per-module
``Engine`` cached on the module with ``object.__setattr__`` (so the
``state_dict`` is untouched), weights packed once per (compute dtype,
device), a mask classifier memoised on tensor identity, a per-shape plan
cache, and an optional whole-forward hipGraph.

The forward (reference :205-269) is a pre-LN causal encoder with an fp32
residual stream ``res``:

    LN1(layer 0) reads x in the model dtype and writes res = fp32(x) and h
    for each layer:
        qkv  = h Wqkv^T + bqkv                    (one [3d, d] GEMM, packed q|k|v)
        ctx  = flash_attention(qkv as [B,S,3,H,hd])
        res += ctx Wo^T + bo                      (GEMM residual epilogue)
        h    = LN2(res)
        mid  = gelu_erf(h W1^T + b1)              (GEMM GELU epilogue)
        res += mid W2^T + b2                      (GEMM residual epilogue)
        h    = LN1 of the next layer (res)
    out = LN_final(res), padded rows written as exact zeros

With ``Plan.residual_epilogue=False`` the out-proj / FFN outputs are instead
written in the compute dtype and added by the following LayerNorm, which is
the reference's deferred-residual scheme (engine.py:232-264).

Masks: NONE (no mask or all valid) needs nothing.  PREFIX (every sequence
valid on a prefix of length len_b) packs the valid tokens: no valid row ever
depends on a padded one -- under causal attention a valid query never sees
a key at or beyond its sequence's length (engine.py:147-150), without it the
padded keys are masked, and every other op is row-wise -- so the first
LayerNorm gathers the sum(len_b) valid rows into consecutive rows, every
GEMM and LayerNorm runs on those rows only, attention runs on the packed
sequences (cu_seqlens), and the final LayerNorm scatters the rows back to
[B, S] order with padded rows written as exact zeros.  The reference
computes the padded rows and zeroes them at the end (engine.py:267-268);
the valid rows come out the same either way.  GENERAL (any other mask)
hands the mask to the attention kernel as a per-key mask, computes every
row and zeroes the padded ones in the final LayerNorm.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import ops, schedule as sched_mod, tiles
from .graphs import GraphCache
from .plans import Plan, select_plan

try:
    from torch.utils.weak import WeakTensorKeyDictionary as _WeakDict
except Exception:  # pragma: no cover
    _WeakDict = dict

MASK_NONE, MASK_PREFIX, MASK_GENERAL = 0, 1, 2


@dataclass
class LayerWeights:
    """Packed weights of one block; every matrix keeps nn.Linear's [out, in]
    layout, which is exactly the K-contiguous operand the GEMM wants."""

    ln1_w: torch.Tensor
    ln1_b: torch.Tensor
    ln1_eps: float
    wqkv: torch.Tensor   # [3d, d]: rows q | k | v
    bqkv: torch.Tensor   # [3d]
    wo: torch.Tensor     # [d, d]
    bo: torch.Tensor
    ln2_w: torch.Tensor
    ln2_b: torch.Tensor
    ln2_eps: float
    w1: torch.Tensor     # [f, d]
    b1: torch.Tensor
    w2: torch.Tensor     # [d, f]
    b2: torch.Tensor


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
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    gather = torch.cat([torch.arange(b * seq, b * seq + n, dtype=torch.int32)
                        for b, n in enumerate(lengths)]) if cu[-1] else torch.zeros(0, dtype=torch.int32)
    scatter = torch.full((len(lengths) * seq,), -1, dtype=torch.int32)
    scatter[gather.long()] = torch.arange(cu[-1], dtype=torch.int32)
    return Packing(lengths=tuple(lengths), tokens=cu[-1], gather=gather.to(device),
                   scatter=scatter.to(device), cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=device))


@dataclass
class _Fwd:
    """Static context of one forward shape: workspace views of the processed
    rows, tile plans, masks and the packing it runs on."""

    batch: int
    seq: int
    mode: int
    packing: Optional[Packing]
    rows: int
    gather: Optional[torch.Tensor] = None
    scatter: Optional[torch.Tensor] = None
    key_mask: Optional[torch.Tensor] = None
    row_mask: Optional[torch.Tensor] = None
    res: Optional[torch.Tensor] = None
    h: Optional[torch.Tensor] = None
    qkv: Optional[torch.Tensor] = None
    ctx: Optional[torch.Tensor] = None
    mid: Optional[torch.Tensor] = None
    delta: Optional[torch.Tensor] = None
    tp_qkv: int = -1
    tp_out: int = -1
    tp_ffn1: int = -1
    tp_ffn2: int = -1
    use_sched: bool = False


@dataclass
class Workspace:
    res: torch.Tensor    # [T, d] fp32
    h: torch.Tensor      # [T, d] compute dtype
    qkv: torch.Tensor    # [T, 3d]
    ctx: torch.Tensor    # [T, d]
    mid: torch.Tensor    # [T, f]
    delta: Optional[torch.Tensor]  # [T, d] (deferred-residual plans only)


class Engine:
    def __init__(self, module: torch.nn.Module) -> None:
        cfg = module.config
        param = next(module.parameters())
        self.device = param.device
        self.dtype = param.dtype
        self.d_model = cfg.d_model
        self.num_heads = cfg.num_heads
        self.head_dim = cfg.d_model // cfg.num_heads
        self.ffn_dim = cfg.ffn_dim
        self.num_layers = cfg.num_layers
        self.causal = cfg.causal
        self.plan: Optional[Plan] = None
        self._plan_cache: Dict[Tuple[int, int], Plan] = {}
        self._built_for: Optional[Tuple] = None
        self.layers: List[LayerWeights] = []
        self.final_ln: Optional[Tuple[torch.Tensor, torch.Tensor, float]] = None
        self._module = module
        self._graphs = GraphCache()
        self._mask_modes = _WeakDict()
        self._workspaces: Dict[Tuple, Workspace] = {}
        self._packings: "OrderedDict[Tuple[int, Tuple[int, ...]], Packing]" = OrderedDict()
        self._static_masks: Dict[Tuple[int, int], torch.Tensor] = {}
        self._fwds: Dict[Tuple, "_Fwd"] = {}

    # ------------------------------------------------------------- weights

    @torch.no_grad()
    def _build(self, plan: Plan) -> None:
        key = (plan.compute_dtype, self.dtype, self.device)
        if self._built_for == key:
            return
        cdt = plan.compute_dtype
        layers: List[LayerWeights] = []
        for block in self._module.layers:
            attn = block.attention
            wqkv = torch.cat([attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight], 0)
            bqkv = torch.cat([attn.q_proj.bias, attn.k_proj.bias, attn.v_proj.bias], 0)
            layers.append(LayerWeights(
                ln1_w=block.norm1.weight.float().contiguous(),
                ln1_b=block.norm1.bias.float().contiguous(),
                ln1_eps=block.norm1.eps,
                wqkv=wqkv.to(cdt).contiguous(),
                bqkv=bqkv.to(cdt).contiguous(),
                wo=attn.out_proj.weight.to(cdt).contiguous(),
                bo=attn.out_proj.bias.to(cdt).contiguous(),
                ln2_w=block.norm2.weight.float().contiguous(),
                ln2_b=block.norm2.bias.float().contiguous(),
                ln2_eps=block.norm2.eps,
                w1=block.ffn_in.weight.to(cdt).contiguous(),
                b1=block.ffn_in.bias.to(cdt).contiguous(),
                w2=block.ffn_out.weight.to(cdt).contiguous(),
                b2=block.ffn_out.bias.to(cdt).contiguous(),
            ))
        self.layers = layers
        fn = self._module.final_norm
        self.final_ln = (fn.weight.float().contiguous(), fn.bias.float().contiguous(), fn.eps)
        self._built_for = key
        self._graphs.clear()
        self._fwds.clear()
        self._workspaces.clear()

    def _workspace(self, batch: int, seq: int, plan: Plan) -> Workspace:
        key = (batch, seq, plan.compute_dtype, plan.residual_epilogue)
        ws = self._workspaces.get(key)
        if ws is None:
            t, d, f = batch * seq, self.d_model, self.ffn_dim
            cdt, dev = plan.compute_dtype, self.device
            ws = Workspace(
                res=torch.empty((t, d), dtype=torch.float32, device=dev),
                h=torch.empty((t, d), dtype=cdt, device=dev),
                qkv=torch.empty((t, 3 * d), dtype=cdt, device=dev),
                ctx=torch.empty((t, d), dtype=cdt, device=dev),
                mid=torch.empty((t, f), dtype=cdt, device=dev),
                delta=None if plan.residual_epilogue else torch.empty((t, d), dtype=cdt, device=dev),
            )
            self._workspaces[key] = ws
        return ws

    # ---------------------------------------------------------------- mask

    def _mask_mode(self, mask: Optional[torch.Tensor]) -> int:
        return self._mask_info(mask)[0]

    def _mask_info(self, mask: Optional[torch.Tensor]) -> Tuple[int, Optional[Tuple[int, ...]]]:
        """(NONE / PREFIX / GENERAL, prefix lengths for PREFIX) with one host
        sync per distinct mask tensor, memoised on tensor identity as
        tjkernels/engine.py:131-158 does."""
        if mask is None:
            return MASK_NONE, None
        cached = self._mask_modes.get(mask)
        if cached is not None:
            return cached
        lengths = mask.sum(dim=-1)
        positions = torch.arange(mask.shape[-1], device=mask.device)
        prefix = positions[None, :] < lengths[:, None]
        if bool(torch.equal(prefix, mask)):
            host = tuple(int(n) for n in lengths.tolist())
            info = (MASK_NONE, None) if min(host) == mask.shape[-1] else (MASK_PREFIX, host)
        else:
            info = (MASK_GENERAL, None)
        self._mask_modes[mask] = info
        return info

    def _packing(self, lengths: Tuple[int, ...], seq: int) -> Packing:
        key = (seq, lengths)
        pk = self._packings.get(key)
        if pk is None:
            pk = build_packing(lengths, seq, self.device)
            self._packings[key] = pk
            while len(self._packings) > 64:
                self._packings.popitem(last=False)
        else:
            self._packings.move_to_end(key)
        return pk

    # ------------------------------------------------------------- compute

    def _prepare(self, batch: int, seq: int, mode: int, packing: Optional[Packing],
                 mask: Optional[torch.Tensor]) -> "_Fwd":
        """Everything a forward needs besides x and the output: workspace
        views, tile plans, the attention schedule.  Launches nothing except
        the one-time tile timing / schedule build of a new shape."""
        plan = self.plan
        assert plan is not None and self.final_ln is not None
        ws = self._workspace(batch, seq, plan)
        fw = _Fwd(batch=batch, seq=seq, mode=mode, packing=packing, rows=batch * seq)
        if mode == MASK_PREFIX:
            assert packing is not None
            fw.rows, fw.gather, fw.scatter = packing.tokens, packing.gather, packing.scatter
        elif mode == MASK_GENERAL:
            fw.key_mask = mask
            fw.row_mask = mask.reshape(-1)
        rows = fw.rows
        fw.res, fw.h, fw.qkv, fw.ctx, fw.mid = (ws.res[:rows], ws.h[:rows], ws.qkv[:rows],
                                                ws.ctx[:rows], ws.mid[:rows])
        fw.delta = None if ws.delta is None else ws.delta[:rows]
        # Tile plans: forced by the Plan, else measured once per shape.
        cdt, d, f = plan.compute_dtype, self.d_model, self.ffn_dim
        epi_res = ops.EPI_BIAS_RESIDUAL if plan.residual_epilogue else ops.EPI_BIAS
        fw.tp_qkv = tiles.gemm_plan(rows, 3 * d, d, cdt, ops.EPI_BIAS, plan.gemm_qkv)
        fw.tp_out = tiles.gemm_plan(rows, d, d, cdt, epi_res, plan.gemm_out)
        fw.tp_ffn1 = tiles.gemm_plan(rows, f, d, cdt, ops.EPI_BIAS_GELU, plan.gemm_ffn1)
        fw.tp_ffn2 = tiles.gemm_plan(rows, d, f, cdt, epi_res, plan.gemm_ffn2)
        # Packed 2-byte attention below 2048 keys follows a longest-first work
        # list (tjkernels.schedule; attn_plan -1 or 4).  Longer sequences run
        # the plain plan-1 kernel, measured faster there; other plan ids
        # force the plain kernel.
        fw.use_sched = (mode == MASK_PREFIX and cdt != torch.float32 and rows > 0
                        and (plan.attn_plan == 4 or (plan.attn_plan == -1 and max(packing.lengths) < 2048)))
        if fw.use_sched and packing.attn is None:
            packing.attn = sched_mod.build_schedule(packing.lengths, self.num_heads, self.head_dim,
                                                    self.causal, cdt, self.device)
        return fw

    def _first(self, fw: "_Fwd", x: torch.Tensor) -> None:
        """Layer-0 LN1: reads x (packing it under a prefix mask), writes the
        fp32 residual and h."""
        lw = self.layers[0]
        ops.add_layernorm(x.reshape(fw.batch * fw.seq, self.d_model), None, lw.ln1_w, lw.ln1_b,
                          lw.ln1_eps, fw.h, res_out=fw.res, row_index=fw.gather)

    def _body(self, fw: "_Fwd") -> None:
        """Every layer between the first LayerNorm and the final one: the
        part the hipGraph captures (fixed buffers only)."""
        plan = self.plan
        heads, hd, rows = self.num_heads, self.head_dim, fw.rows
        res, h, qkv, ctx, mid, delta = fw.res, fw.h, fw.qkv, fw.ctx, fw.mid, fw.delta
        fused = plan.residual_epilogue
        pending = None
        for i, lw in enumerate(self.layers):
            if i > 0:
                ops.add_layernorm(res, pending, lw.ln1_w, lw.ln1_b, lw.ln1_eps, h,
                                  res_out=res if pending is not None else None)
            ops.gemm(h, lw.wqkv, lw.bqkv, qkv, ops.EPI_BIAS, fw.tp_qkv)
            if fw.use_sched:
                pk = fw.packing
                ops.flash_attention_sched(qkv.view(rows, 3, heads, hd), ctx, pk.cu_seqlens,
                                          max(pk.lengths), pk.attn, causal=self.causal)
            elif fw.mode == MASK_PREFIX:
                pk = fw.packing
                ops.flash_attention(qkv.view(rows, 3, heads, hd), ctx, causal=self.causal,
                                    plan=plan.attn_plan, cu_seqlens=pk.cu_seqlens,
                                    max_seqlen=max(pk.lengths))
            else:
                ops.flash_attention(qkv.view(fw.batch, fw.seq, 3, heads, hd), ctx, causal=self.causal,
                                    key_mask=fw.key_mask, plan=plan.attn_plan)
            if fused:
                ops.gemm(ctx, lw.wo, lw.bo, res, ops.EPI_BIAS_RESIDUAL, fw.tp_out)
                ops.add_layernorm(res, None, lw.ln2_w, lw.ln2_b, lw.ln2_eps, h)
            else:
                ops.gemm(ctx, lw.wo, lw.bo, delta, ops.EPI_BIAS, fw.tp_out)
                ops.add_layernorm(res, delta, lw.ln2_w, lw.ln2_b, lw.ln2_eps, h, res_out=res)
            ops.gemm(h, lw.w1, lw.b1, mid, ops.EPI_BIAS_GELU, fw.tp_ffn1)
            if fused:
                ops.gemm(mid, lw.w2, lw.b2, res, ops.EPI_BIAS_RESIDUAL, fw.tp_ffn2)
            else:
                ops.gemm(mid, lw.w2, lw.b2, delta, ops.EPI_BIAS, fw.tp_ffn2)
                pending = delta  # added by the next LayerNorm (deferred residual)

    def _final(self, fw: "_Fwd", out: torch.Tensor, row_mask: Optional[torch.Tensor]) -> None:
        """Final LayerNorm into the output, padded rows as exact zeros."""
        fwt, fb, feps = self.final_ln
        pending = None if self.plan.residual_epilogue else fw.delta
        ops.add_layernorm(fw.res, pending, fwt, fb, feps, out.view(fw.batch * fw.seq, self.d_model),
                          row_mask=row_mask, row_index=fw.scatter)

    def _forward_impl(self, x: torch.Tensor, mask: Optional[torch.Tensor], mode: int,
                      packing: Optional[Packing] = None) -> torch.Tensor:
        """Eager forward (no graph)."""
        batch, seq, d = x.shape
        fw = self._prepare(batch, seq, mode, packing, mask)
        out = torch.empty((batch, seq, d), dtype=self.dtype, device=x.device)
        self._first(fw, x)
        self._body(fw)
        self._final(fw, out, fw.row_mask)
        return out

    # ---------------------------------------------------------------- call

    def __call__(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("tjkernels runs on ROCm GPUs only (input on "
                               f"{x.device}); there is no CPU path")
        if x.dim() != 3 or x.shape[-1] != self.d_model:
            raise ValueError(f"expected x of shape [B, S, {self.d_model}], got {tuple(x.shape)}")
        if x.dtype != self.dtype:
            raise ValueError(f"x dtype {x.dtype} != model dtype {self.dtype}")
        if not x.is_contiguous():
            x = x.contiguous()
        host_lengths: Optional[Tuple[int, ...]] = None
        if mask is not None and mask.dim() == 1 and not mask.dtype.is_floating_point \
                and mask.dtype != torch.bool:
            # forward(x, lengths): int prefix lengths [B]; read once on the host
            # (the packed layout is sized from them) and turned into the
            # equivalent prefix mask for the graph path's static inputs.
            if mask.shape[0] != x.shape[0]:
                raise ValueError(f"lengths must be [B], got {tuple(mask.shape)}")
            host_lengths = tuple(min(max(int(n), 0), x.shape[1]) for n in mask.tolist())
            lengths = torch.tensor(host_lengths, dtype=torch.int64, device=x.device)
            mask = torch.arange(x.shape[1], device=x.device)[None, :] < lengths[:, None]
        if mask is not None:
            if tuple(mask.shape) != tuple(x.shape[:2]):
                raise ValueError(f"valid_token_mask must be [B, S], got {tuple(mask.shape)}")
            if mask.dtype != torch.bool:
                mask = mask.to(torch.bool)
            if not mask.is_contiguous():
                mask = mask.contiguous()
        batch, seq, _ = x.shape
        plan = self._plan_cache.get((batch, seq))
        if plan is None:
            plan = select_plan(batch, seq, self.d_model, self.num_heads, self.ffn_dim,
                               self.num_layers, self.causal, self.dtype, self.device)
            plan.validate()
            self._plan_cache[(batch, seq)] = plan
        self.plan = plan
        self._build(plan)
        if host_lengths is not None:
            if min(host_lengths, default=x.shape[1]) == x.shape[1]:
                mode, lens = MASK_NONE, None
            else:
                mode, lens = MASK_PREFIX, host_lengths
        else:
            mode, lens = self._mask_info(mask)
        if mode == MASK_PREFIX and not plan.pack_prefix:
            mode, lens = MASK_GENERAL, None  # every row computed, per-key mask
        packing = self._packing(lens, x.shape[1]) if mode == MASK_PREFIX else None
        if plan.cuda_graph:
            return self._forward_graph(x, mask, mode, lens, packing)
        return self._forward_impl(x, mask, mode, packing)

    def _forward_graph(self, x: torch.Tensor, mask: Optional[torch.Tensor], mode: int,
                       lens: Optional[Tuple[int, ...]], packing: Optional[Packing]) -> torch.Tensor:
        """The first LayerNorm (which reads the caller's x) and the final one
        (which writes a fresh output tensor) run eagerly; the layers between
        them replay as one hipGraph on fixed workspace buffers.  So no copy
        of x into a static input and no clone of a static output is needed
        (the reference copies in and clones out, graphs.py:57-64); only a
        GENERAL mask, which the captured attention reads, is copied into a
        static buffer.  A packed forward is specific to its lengths (its
        launches are sized by them), so they are part of the key; the graph
        keeps the row maps and schedule it reads alive."""
        batch, seq, d = x.shape
        static_mask = None
        if mode == MASK_GENERAL:
            static_mask = self._static_masks.get((batch, seq))
            if static_mask is None:
                static_mask = torch.empty((batch, seq), dtype=torch.bool, device=x.device)
                self._static_masks[(batch, seq)] = static_mask
        key = (batch, seq, x.dtype, mode, lens, self.plan)
        fw = self._fwds.get(key)
        if fw is None:
            fw = self._prepare(batch, seq, mode, packing, static_mask)
            self._fwds[key] = fw
        graph = self._graphs.get(key, lambda: self._body(fw), keepalive=(packing, fw))
        self._first(fw, x)
        if graph is not None:
            if static_mask is not None:
                static_mask.copy_(mask)
            graph.replay()
        else:
            if static_mask is not None:
                static_mask.copy_(mask)
            self._body(fw)
        out = torch.empty((batch, seq, d), dtype=self.dtype, device=x.device)
        self._final(fw, out, None if mask is None or mode != MASK_GENERAL else mask.reshape(-1))
        return out


def get_engine(module: torch.nn.Module) -> Engine:
    engine = getattr(module, "_tj_engine", None)
    param = next(module.parameters())
    if engine is None or engine.dtype != param.dtype or engine.device != param.device:
        engine = Engine(module)
        object.__setattr__(module, "_tj_engine", engine)
    return engine


def reset_engines(module: torch.nn.Module) -> None:
    if hasattr(module, "_tj_engine"):
        object.__delattr__(module, "_tj_engine")


def forward(module: torch.nn.Module, x: torch.Tensor,
            valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The hook body: ``return tjkernels.forward(self, x, valid_token_mask)``
    (torch_transformer_benchmark.py:203).  ``TJ_DISABLE=1`` calls the parent
    class's forward instead, as the reference does (engine.py:322-323)."""
    if os.environ.get("TJ_DISABLE") == "1":
        return super(type(module), module).forward(x, valid_token_mask)
    return get_engine(module)(x, valid_token_mask)
