"""Tensor-level wrappers over the tjk C-ABI.

Each op checks devices/layouts it relies on, passes raw device pointers and
``torch.cuda.current_stream().cuda_stream`` (so the launch lands on the
caller's stream, including under hipGraph capture), and raises ``TjkError``
on a non-zero status.  None of them allocates on the hot path except where
an output tensor is requested with ``out=None``.

Mirrors of the reference's kernel dispatch layer
(tjkernels/kernels/__init__.py:48-101), minus its torch fallbacks.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESIDUAL, TjkError, check  # noqa: F401


def _code(t: torch.Tensor) -> int:
    try:
        return _lib.DTYPE_CODES[t.dtype]
    except KeyError:
        raise TjkError(f"unsupported dtype {t.dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    # the raw-handle query costs ~0.1 us against ~2 us for building a Stream
    if _raw_stream is not None:
        return _raw_stream(t.device.index if t.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_gpu(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise TjkError("tjkernels ops need ROCm device tensors (no CPU path)")


def _rowmajor(t: torch.Tensor, name: str) -> int:
    if t.dim() != 2 or t.stride(1) != 1:
        raise TjkError(f"{name} must be a 2-D row-major view, got shape {tuple(t.shape)} "
                       f"strides {t.stride()}")
    return t.stride(0)


def add_layernorm(res: torch.Tensor, delta: Optional[torch.Tensor],
                  gamma: torch.Tensor, beta: torch.Tensor, eps: float,
                  out: torch.Tensor, res_out: Optional[torch.Tensor] = None,
                  row_mask: Optional[torch.Tensor] = None,
                  row_index: Optional[torch.Tensor] = None,
                  index_errors: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x = res (+ delta) in fp32; res_out <- x (optional; fp32, or rounded to
    a 2-byte res_out, the reference's residual_dtype); out <- LN(x), of the
    unrounded x (rows with row_mask == 0 written as 0).  Mirrors
    fused_add_layernorm, tjkernels/kernels/__init__.py:48-70.

    With ``row_index`` (int32, one entry per output row) the call is a
    gather / scatter: output row r is computed from input row row_index[r],
    or written as zeros when the index is negative or not below the rows
    ``res`` (and ``delta``) hold -- the latter also counted in
    ``index_errors`` (a one-element int32 device tensor) when given;
    ``out`` (and ``res_out``) then have ``row_index.numel()`` rows.

    A 3-D ``delta`` [splits, rows, n] (the fused FFN's split partials) is
    summed over its first dimension, in order, before it is added."""
    _require_gpu(res, delta, gamma, beta, out, res_out, row_mask, row_index, index_errors)
    rows, n = res.shape
    src_rows = rows if delta is None else min(rows, delta.shape[-2])
    if index_errors is not None and (index_errors.dtype != torch.int32 or index_errors.numel() < 1):
        raise TjkError("index_errors must be an int32 device tensor of at least one element")
    splits, split_stride, delta2 = 1, 0, delta
    if delta is not None and delta.dim() == 3:
        splits, split_stride, delta2 = delta.shape[0], delta.stride(0), delta[0]
        if delta.shape[2] != n or (splits > 1 and delta.stride(0) < delta.shape[1] * delta.stride(1)):
            raise TjkError(f"split delta must be [splits, rows, {n}] with non-overlapping splits")
    if row_index is not None:
        if row_index.dtype != torch.int32 or row_index.dim() != 1 or not row_index.is_contiguous():
            raise TjkError("row_index must be a contiguous int32 vector")
        rows = row_index.numel()
        if out.shape[0] < rows or (res_out is not None and res_out.shape[0] < rows):
            raise TjkError("row_index has more entries than out / res_out rows")
    elif out.shape[0] < rows or (res_out is not None and res_out.shape[0] < rows):
        raise TjkError("out / res_out have fewer rows than res")
    if gamma.dtype != torch.float32 or beta.dtype != torch.float32:
        raise TjkError("gamma/beta must be float32")
    if row_mask is not None and (row_mask.dtype not in (torch.bool, torch.uint8)
                                 or row_mask.numel() != rows or not row_mask.is_contiguous()):
        raise TjkError("row_mask must be a contiguous bool/uint8 tensor with one entry per row")
    lib = _lib.load()
    status = lib.tjk_add_layernorm(
        res.data_ptr(), _code(res), _rowmajor(res, "res"),
        _ptr(delta), _code(delta) if delta is not None else 0,
        _rowmajor(delta2, "delta") if delta is not None else 0, splits, split_stride,
        _ptr(res_out), _code(res_out) if res_out is not None else 0,
        _rowmajor(res_out, "res_out") if res_out is not None else 0,
        out.data_ptr(), _code(out), _rowmajor(out, "out"),
        gamma.data_ptr(), beta.data_ptr(), rows, n, float(eps),
        _ptr(row_index), src_rows, _ptr(index_errors), _ptr(row_mask), _stream(res))
    check(status, "tjk_add_layernorm")
    return out


def gemm(a: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], out: torch.Tensor,
         epilogue: int = EPI_BIAS, plan: int = -1) -> torch.Tensor:
    """out = epi(a @ w.T + bias); w in nn.Linear [N, K] layout.
    With EPI_BIAS_RESIDUAL, ``out`` is an fp32 residual updated in place."""
    _require_gpu(a, w, bias, out)
    m, k = a.shape
    n, k2 = w.shape
    if k != k2 or out.shape[0] != m or out.shape[1] != n:
        raise TjkError(f"gemm shape mismatch a{tuple(a.shape)} w{tuple(w.shape)} out{tuple(out.shape)}")
    if w.dtype != a.dtype or (bias is not None and bias.dtype != a.dtype):
        raise TjkError("gemm operands must share a dtype")
    if epilogue == EPI_BIAS_RESIDUAL:
        if out.dtype != torch.float32:
            raise TjkError("residual epilogue needs a float32 out")
    elif out.dtype != a.dtype:
        raise TjkError("gemm out must have the operands' dtype")
    lib = _lib.load()
    status = lib.tjk_gemm_bias(a.data_ptr(), _rowmajor(a, "a"), w.data_ptr(), _rowmajor(w, "w"),
                               _ptr(bias), out.data_ptr(), _rowmajor(out, "out"), m, n, k,
                               _code(a), epilogue, plan, _stream(a))
    check(status, "tjk_gemm_bias")
    return out


def gemm_residual_from(a: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], out: torch.Tensor,
                       x: torch.Tensor, rows: Optional[torch.Tensor] = None,
                       index_errors: Optional[torch.Tensor] = None, plan: int = -1) -> torch.Tensor:
    """out = a @ w.T + bias + x[rows] in fp32 (``out`` written, not read):
    the EPI_BIAS_RESIDUAL ``gemm`` with its residual read from the
    compute-dtype ``x`` through the int32 row map ``rows`` (identity when
    None) instead of from ``out``.  A row outside ``x`` adds zeros and is
    counted in ``index_errors``.  Bit-identical to copying x[rows] into an
    fp32 ``out`` and running the residual ``gemm``; the first layer's
    out-projection of tjkernels/engine.py:230-252."""
    _require_gpu(a, w, bias, out, x, rows, index_errors)
    m, k = a.shape
    n, k2 = w.shape
    if k != k2 or out.shape[0] != m or out.shape[1] != n:
        raise TjkError(f"gemm shape mismatch a{tuple(a.shape)} w{tuple(w.shape)} out{tuple(out.shape)}")
    if w.dtype != a.dtype or (bias is not None and bias.dtype != a.dtype) or x.dtype != a.dtype:
        raise TjkError("gemm_residual_from: a, w, bias and x share the compute dtype")
    if out.dtype != torch.float32:
        raise TjkError("residual epilogue needs a float32 out")
    if x.dim() != 2 or x.shape[1] != n:
        raise TjkError(f"x must be [rows, {n}], got {tuple(x.shape)}")
    if rows is not None:
        if rows.dtype != torch.int32 or rows.dim() != 1 or not rows.is_contiguous() or rows.numel() < m:
            raise TjkError("rows must be a contiguous int32 vector with an entry per output row")
    elif x.shape[0] < m:
        raise TjkError("x has fewer rows than out and no row map is given")
    if index_errors is not None and (index_errors.dtype != torch.int32 or index_errors.numel() < 1):
        raise TjkError("index_errors must be an int32 device tensor of at least one element")
    status = _lib.load().tjk_gemm_bias_residual_from(
        a.data_ptr(), _rowmajor(a, "a"), w.data_ptr(), _rowmajor(w, "w"), _ptr(bias), out.data_ptr(),
        _rowmajor(out, "out"), m, n, k, x.data_ptr(), _rowmajor(x, "x"), x.shape[0], _ptr(rows),
        _ptr(index_errors), _code(a), plan, _stream(a))
    check(status, "tjk_gemm_bias_residual_from")
    return out


def gemm_ln_supported(k: int, dtype: torch.dtype) -> bool:
    """Whether tjk_gemm_ln takes a K (= d_model) and compute dtype."""
    code = _lib.DTYPE_CODES.get(dtype)
    return code is not None and bool(_lib.load().tjk_gemm_ln_supported(k, code))


def gemm_ln_plan_count() -> int:
    return int(_lib.load().tjk_gemm_ln_plan_count())


def gemm_ln(res: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float, w: torch.Tensor,
            bias: Optional[torch.Tensor], out: torch.Tensor, epilogue: int = EPI_BIAS,
            plan: int = -1) -> torch.Tensor:
    """out = epi(LayerNorm(res) @ w.T + bias) in one launch: the LayerNorm of
    ``add_layernorm`` without delta (fp32 ``res``) applied inside the GEMM,
    for launch-bound row counts; the add+LayerNorm launch and the GEMM of
    tjkernels/engine.py:239-245 (LN1 + QKV) and :249-253 (LN2 + the FFN's
    first GEMM) in one.  Equals add_layernorm then a class-1 ``gemm`` bit
    for bit."""
    _require_gpu(res, gamma, beta, w, bias, out)
    m, k = res.shape
    n, k2 = w.shape
    if k != k2 or out.shape[0] != m or out.shape[1] != n:
        raise TjkError(f"gemm_ln shape mismatch res{tuple(res.shape)} w{tuple(w.shape)} out{tuple(out.shape)}")
    if res.dtype != torch.float32 or gamma.dtype != torch.float32 or beta.dtype != torch.float32:
        raise TjkError("gemm_ln reads the fp32 residual and fp32 gamma / beta")
    if out.dtype != w.dtype or (bias is not None and bias.dtype != w.dtype):
        raise TjkError("gemm_ln: w, bias and out share the compute dtype")
    status = _lib.load().tjk_gemm_ln(res.data_ptr(), _rowmajor(res, "res"), gamma.data_ptr(), beta.data_ptr(),
                                     float(eps), w.data_ptr(), _rowmajor(w, "w"), _ptr(bias), out.data_ptr(),
                                     _rowmajor(out, "out"), m, n, k, _code(w), epilogue, plan, _stream(res))
    check(status, "tjk_gemm_ln")
    return out


def flash_attention(qkv: torch.Tensor, out: torch.Tensor, causal: bool = True,
                    scale: Optional[float] = None, lengths: Optional[torch.Tensor] = None,
                    key_mask: Optional[torch.Tensor] = None, plan: int = -1,
                    cu_seqlens: Optional[torch.Tensor] = None,
                    max_seqlen: Optional[int] = None) -> torch.Tensor:
    """qkv: [B, S, 3, H, hd] (any strides with a unit hd stride) -> out [B*S, H*hd].
    Mirrors flash_attention, tjkernels/kernels/attention.py:189-226, plus the
    masked cases the reference sends to SDPA (tjkernels/engine.py:184-203).

    Packed (varlen) form: ``qkv`` is [T, 3, H, hd] holding B sequences back
    to back, ``cu_seqlens`` int32 [B+1] their row offsets and ``max_seqlen``
    an upper bound of their lengths; ``out`` is [T, H*hd]."""
    _require_gpu(qkv, out, lengths, key_mask, cu_seqlens)
    if cu_seqlens is not None:
        if qkv.dim() != 4 or qkv.shape[1] != 3 or qkv.stride(3) != 1:
            raise TjkError(f"packed qkv must be [T, 3, H, hd] with unit hd stride, got {tuple(qkv.shape)}")
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2 \
                or not cu_seqlens.is_contiguous():
            raise TjkError("cu_seqlens must be a contiguous int32 [B+1] vector")
        if key_mask is not None:
            raise TjkError("cu_seqlens and key_mask are exclusive")
        if max_seqlen is None:
            raise TjkError("packed attention needs max_seqlen")
        t = qkv.shape[0]
        if out.shape[0] < t or out.shape[1] < qkv.shape[2] * qkv.shape[3] or out.dtype != qkv.dtype:
            raise TjkError("bad attention output buffer")
        qkv = qkv.unsqueeze(0)  # stride_b is unused for packed sequences
        b, s, h, hd = cu_seqlens.numel() - 1, int(max_seqlen), qkv.shape[3], qkv.shape[4]
    else:
        if qkv.dim() != 5 or qkv.shape[2] != 3 or qkv.stride(4) != 1:
            raise TjkError(f"qkv must be [B, S, 3, H, hd] with unit hd stride, got {tuple(qkv.shape)}")
        b, s, _, h, hd = qkv.shape
        if out.shape[0] != b * s or out.shape[1] < h * hd or out.dtype != qkv.dtype:
            raise TjkError("bad attention output buffer")
    if lengths is not None and (lengths.dtype != torch.int32 or lengths.numel() != b):
        raise TjkError("lengths must be int32 [B]")
    if key_mask is not None and (key_mask.dtype not in (torch.bool, torch.uint8)
                                 or tuple(key_mask.shape) != (b, s) or not key_mask.is_contiguous()):
        raise TjkError("key_mask must be a contiguous bool/uint8 [B, S] tensor")
    sb, ss, sc, sh, _ = qkv.stride()
    lib = _lib.load()
    status = lib.tjk_flash_fwd(qkv.data_ptr(), sb, ss, sc, sh, out.data_ptr(), _rowmajor(out, "out"),
                               b, s, h, hd, float(hd ** -0.5 if scale is None else scale),
                               int(bool(causal)), _ptr(lengths), _ptr(key_mask), _ptr(cu_seqlens),
                               _code(qkv), plan, _stream(qkv))
    check(status, "tjk_flash_fwd")
    return out


def flash_attention_sched(qkv: torch.Tensor, out: torch.Tensor, cu_seqlens: torch.Tensor,
                          max_seqlen: int, schedule, causal: bool = True,
                          scale: Optional[float] = None) -> torch.Tensor:
    """Packed attention following a work list (``tjkernels.schedule``): the
    same math as ``flash_attention(..., cu_seqlens=...)``, with long query
    blocks issued first and split over their key range (the second half
    merges the first's partial).  qkv: packed [T, 3, H, hd] (bf16 / fp16);
    out: [T, H*hd].  Calls sharing one schedule must be stream-ordered."""
    _require_gpu(qkv, out, cu_seqlens, schedule.work, schedule.partials)
    if qkv.dim() != 4 or qkv.shape[1] != 3 or qkv.stride(3) != 1:
        raise TjkError(f"packed qkv must be [T, 3, H, hd] with unit hd stride, got {tuple(qkv.shape)}")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or not cu_seqlens.is_contiguous():
        raise TjkError("cu_seqlens must be a contiguous int32 [B+1] vector")
    t, _, h, hd = qkv.shape
    if out.shape[0] < t or out.shape[1] < h * hd or out.dtype != qkv.dtype:
        raise TjkError("bad attention output buffer")
    ss, sc, sh, _ = qkv.stride()
    lib = _lib.load()
    status = lib.tjk_flash_fwd_sched(
        qkv.data_ptr(), ss, sc, sh, out.data_ptr(), _rowmajor(out, "out"), cu_seqlens.numel() - 1,
        int(max_seqlen), h, hd, float(hd ** -0.5 if scale is None else scale), int(bool(causal)),
        cu_seqlens.data_ptr(), schedule.work.data_ptr(), schedule.work.shape[0],
        schedule.n_lists or schedule.work.shape[0],
        schedule.partials.data_ptr(), schedule.partials.numel() * schedule.partials.element_size(),
        schedule.n_slots, _code(qkv), _stream(qkv))
    check(status, "tjk_flash_fwd_sched")
    return out


def ffn_supported(d: int, f: int, splits: int, dtype: torch.dtype) -> bool:
    """Whether the single-launch FFN takes (d, f, splits, dtype); the
    counterpart of the reference's ffn.supports (tjkernels/kernels/ffn.py:103-110)."""
    code = _lib.DTYPE_CODES.get(dtype)
    return code is not None and bool(_lib.load().tjk_ffn_supported(d, f, splits, code))


def ffn(a: torch.Tensor, w1: torch.Tensor, b1: Optional[torch.Tensor], w2: torch.Tensor,
        b2: Optional[torch.Tensor], out: torch.Tensor, splits: int = 1,
        ln: Optional[tuple] = None, accumulate: bool = False) -> torch.Tensor:
    """The feed-forward block in one launch; mirrors fused_ffn,
    tjkernels/kernels/__init__.py:80-89.

    ``a`` is h [rows, d] in the weights' dtype, or with ``ln = (gamma, beta,
    eps)`` the fp32 residual that the kernel LayerNorms itself.  ``out`` is
    either [splits, rows, d] fp32 (slice s holds the f-slice s partial, slice
    0 with b2; ``add_layernorm`` sums them) or, with ``accumulate`` and one
    split, the [rows, d] fp32 residual the result is added into."""
    _require_gpu(a, w1, b1, w2, b2, out)
    rows, d = a.shape
    f = w1.shape[0]
    cdt = w1.dtype
    if tuple(w1.shape) != (f, d) or tuple(w2.shape) != (d, f) or w2.dtype != cdt:
        raise TjkError(f"ffn weight shapes w1{tuple(w1.shape)} w2{tuple(w2.shape)} do not match d={d}")
    if (b1 is not None and b1.dtype != cdt) or (b2 is not None and b2.dtype != cdt):
        raise TjkError("ffn biases must have the weights' dtype")
    if out.dtype != torch.float32:
        raise TjkError("ffn output must be float32")
    if ln is not None:
        gamma, beta, eps = ln
        if a.dtype != torch.float32 or gamma.dtype != torch.float32 or beta.dtype != torch.float32:
            raise TjkError("ffn with a LayerNorm reads the fp32 residual and fp32 gamma/beta")
    else:
        gamma = beta = None
        eps = 0.0
        if a.dtype != cdt:
            raise TjkError("ffn input must have the weights' dtype")
    if accumulate:
        if splits != 1 or out.dim() != 2 or out.shape[0] < rows:
            raise TjkError("accumulating ffn needs one split and a [rows, d] residual")
        ld_out, split_stride = _rowmajor(out, "out"), 0
    else:
        if out.dim() != 3 or out.shape[0] != splits or out.shape[1] < rows or out.stride(2) != 1:
            raise TjkError(f"ffn partials must be [splits={splits}, rows, d] fp32")
        ld_out, split_stride = out.stride(1), out.stride(0)
    if w1.stride(1) != 1 or w1.stride(0) != d or w2.stride(1) != 1 or w2.stride(0) != f:
        raise TjkError("ffn weights must be contiguous")
    status = _lib.load().tjk_ffn(a.data_ptr(), _code(a), _rowmajor(a, "a"), _ptr(gamma), _ptr(beta), float(eps),
                                 w1.data_ptr(), _ptr(b1), w2.data_ptr(), _ptr(b2), out.data_ptr(), ld_out,
                                 split_stride, splits, int(bool(accumulate)), rows, d, f, _code(w1), _stream(a))
    check(status, "tjk_ffn")
    return out


def attn_block_supported(d_model: int, heads: int, head_dim: int, max_seqlen: int, dtype: torch.dtype) -> bool:
    """Whether ``attn_block`` takes the shape (tjk_attn_block_supported)."""
    code = _lib.DTYPE_CODES.get(dtype)
    return code is not None and bool(_lib.load().tjk_attn_block_supported(d_model, heads, head_dim, max_seqlen, code))


def attn_block(x: torch.Tensor, w_qkv: torch.Tensor, b_qkv: Optional[torch.Tensor], w_out: torch.Tensor,
               b_out: Optional[torch.Tensor], parts: torch.Tensor, heads: int, causal: bool = True,
               scale: Optional[float] = None, batch: Optional[int] = None, seq: Optional[int] = None,
               cu_seqlens: Optional[torch.Tensor] = None, max_seqlen: Optional[int] = None,
               ctx_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """QKV projection, attention and out-projection of one layer in one
    launch, for sequences of at most 128 tokens: the addmm / flash_attention
    / addmm of tjkernels/engine.py:245-247 fused.

    ``x`` is h [rows, d]: ``batch`` sequences of ``seq`` rows, or with
    ``cu_seqlens`` (int32 [B+1]) packed sequences of at most ``max_seqlen``
    rows.  ``parts`` is [heads, rows, d] fp32: head h's share of the
    out-projection (head 0 with b_out); ``add_layernorm`` sums them.
    ``ctx_out`` [rows, d] optionally receives the attention context."""
    _require_gpu(x, w_qkv, b_qkv, w_out, b_out, parts, cu_seqlens, ctx_out)
    rows, d = x.shape
    cdt = x.dtype
    if tuple(w_qkv.shape) != (3 * d, d) or tuple(w_out.shape) != (d, d):
        raise TjkError(f"attn_block weight shapes w_qkv{tuple(w_qkv.shape)} w_out{tuple(w_out.shape)} "
                       f"do not match d={d}")
    if w_qkv.dtype != cdt or w_out.dtype != cdt or any(b is not None and b.dtype != cdt for b in (b_qkv, b_out)):
        raise TjkError("attn_block operands must share x's dtype")
    if not (w_qkv.is_contiguous() and w_out.is_contiguous()) or \
            any(b is not None and not b.is_contiguous() for b in (b_qkv, b_out)):
        raise TjkError("attn_block weights and biases must be contiguous")
    if d % heads:
        raise TjkError(f"d={d} is not a multiple of heads={heads}")
    if parts.dtype != torch.float32 or parts.dim() != 3 or parts.shape[0] != heads or parts.shape[1] < rows \
            or parts.shape[2] != d or parts.stride(2) != 1:
        raise TjkError(f"attn_block partials must be [heads={heads}, rows, {d}] fp32")
    if cu_seqlens is not None:
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2 \
                or not cu_seqlens.is_contiguous():
            raise TjkError("cu_seqlens must be a contiguous int32 [B+1] vector")
        if max_seqlen is None:
            raise TjkError("packed attn_block needs max_seqlen")
        b, s = cu_seqlens.numel() - 1, int(max_seqlen)
    else:
        if batch is None or seq is None or batch * seq != rows:
            raise TjkError("attn_block needs batch * seq == rows (or cu_seqlens)")
        b, s = int(batch), int(seq)
    if ctx_out is not None and (ctx_out.dtype != cdt or ctx_out.shape[0] < rows or ctx_out.shape[1] != d):
        raise TjkError("bad attn_block ctx_out buffer")
    hd = d // heads
    status = _lib.load().tjk_attn_block(
        x.data_ptr(), _rowmajor(x, "x"), w_qkv.data_ptr(), _ptr(b_qkv), w_out.data_ptr(), _ptr(b_out),
        parts.data_ptr(), parts.stride(1), parts.stride(0), _ptr(ctx_out),
        _rowmajor(ctx_out, "ctx_out") if ctx_out is not None else 0, _ptr(cu_seqlens), b, s, heads, hd,
        float(hd ** -0.5 if scale is None else scale), int(bool(causal)), _code(x), _stream(x))
    check(status, "tjk_attn_block")
    return parts


def gemm_plans(dtype: torch.dtype):
    """[(plan_id, block_m, block_n, waves, k_groups)] available for ``dtype``."""
    import ctypes
    lib = _lib.load()
    code = _lib.DTYPE_CODES[dtype]
    out = []
    for i in range(lib.tjk_gemm_plan_count(code)):
        bm, bn, wv, kg = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib.tjk_gemm_plan_info(code, i, ctypes.byref(bm), ctypes.byref(bn), ctypes.byref(wv),
                                     ctypes.byref(kg)), "tjk_gemm_plan_info")
        out.append((i, bm.value, bn.value, wv.value, kg.value))
    return out
