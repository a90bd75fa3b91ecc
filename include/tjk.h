/*
 * tjk.h -- C-ABI of the MI355X (gfx950) fused Transformer-forward kernels.
 *
 * Every entry point takes caller-allocated device pointers, explicit leading
 * dimensions, a dtype enum and a hipStream_t passed as `void*`, enqueues its
 * kernels on that stream and returns an int status:
 *     0              success
 *     negative       invalid argument / unsupported shape or dtype
 *                    (nothing was launched; see tjk_last_error_string())
 *     positive       a hipError_t from the launch
 * No entry point allocates memory or synchronizes the host, and all but one
 * keep no mutable global state, so they are safe inside hipGraph stream
 * capture and reentrant across streams.  The exception is
 * tjk_flash_fwd_sched_static: it keeps a per-device table of its static
 * workspace's address, filled once under a mutex, and every call on one
 * device shares that workspace, so calls that overlap on one device race.
 * Row-major layouts throughout.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   tjk_add_layernorm  <- fused_add_layernorm, tjkernels/kernels/__init__.py:48-70
 *                         (Triton kernel tjkernels/kernels/layernorm.py:30-75,
 *                         launcher :96-127) and the final masked_fill,
 *                         tjkernels/engine.py:267-268
 *   tjk_gemm_bias      <- torch.addmm(bias, h, W), tjkernels/engine.py:245 (QKV)
 *                         and :247 (out-proj); FFN fallback addmm + gelu,
 *                         tjkernels/kernels/__init__.py:88-89
 *   tjk_flash_fwd      <- flash_attention, tjkernels/kernels/attention.py:189-226
 *                         (kernel :34-125), and the SDPA masked fallback,
 *                         tjkernels/engine.py:184-203
 *   tjk_ffn            <- fused_ffn, tjkernels/kernels/__init__.py:80-89
 *                         (Triton kernel tjkernels/kernels/ffn.py:21-69,
 *                         shape gate ffn.py:103-110 -> tjk_ffn_supported)
 *   tjk_flash_fwd_sched <- the grid of (query block, b*h) programs of
 *                         tjkernels/kernels/attention.py:199-217
 *   tjk_gemm_ln        <- fused_add_layernorm without a pending delta and
 *                         the addmm after it: LN1 + QKV, tjkernels/engine.py:239-245;
 *                         LN2 + the FFN's first GEMM, engine.py:249-253 with
 *                         tjkernels/kernels/__init__.py:88
 *   tjk_attn_block     <- the QKV addmm, flash_attention and out-proj addmm
 *                         (tjkernels/engine.py:245-247) fused for sequences
 *                         of at most 128 tokens, the tiny-shape fusion of
 *                         README.md:193-196
 */
#ifndef TJK_H
#define TJK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TJK_ABI_VERSION 10

/* dtypes */
#define TJK_F32 0
#define TJK_F16 1
#define TJK_BF16 2

/* statuses */
#define TJK_OK 0
#define TJK_EINVAL (-1)
#define TJK_EUNSUPPORTED (-2)

/* GEMM epilogues */
#define TJK_EPI_BIAS 0          /* C = A W^T + b                                   */
#define TJK_EPI_BIAS_GELU 1     /* C = gelu_erf(A W^T + b)                          */
#define TJK_EPI_BIAS_RESIDUAL 2 /* R += A W^T + b, R fp32 (C is the fp32 residual) */

/* Version of this ABI (TJK_ABI_VERSION). */
int tjk_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* tjk_last_error_string(void);

/*
 * Fused residual-add + LayerNorm over rows of length n.
 *   x   = res (+ delta)                       computed in fp32
 *   res_out = x            (if res_out != NULL), stored in res_out_dtype:
 *           fp32, or rounded to fp16 / bf16 (a 2-byte residual stream, the
 *           reference's Plan.residual_dtype, tjkernels/plans.py:33-36; the
 *           LayerNorm below still normalises the unrounded fp32 x, as the
 *           reference's kernel does, tjkernels/kernels/layernorm.py:50-60).
 *           res_out may alias res only in place: same dtype and leading
 *           dimension, no row_index.
 *   out = (x - mean) * rsqrt(var + eps) * gamma + beta, biased variance,
 *         written in out_dtype; rows whose row_mask byte is 0 are written as 0
 *         (row_mask may be NULL, indexed by row).
 * row_index (may be NULL) makes the call a gather / scatter over `rows`
 * output rows: output row r reads res / delta row row_index[r]; a negative
 * index writes an all-zero output row and leaves res_out's row untouched.
 * src_rows is the number of rows res and delta hold (read only with a
 * row_index): an entry >= src_rows is treated like a negative one (zero
 * row, nothing read) and counted, once per output row, in *index_errors
 * (an int on the device, may be NULL; never reset by the call).
 * res_dtype, delta_dtype, res_out_dtype, out_dtype in
 * {TJK_F32, TJK_F16, TJK_BF16};
 * delta may be NULL.  Requires n % 4 == 0, n <= 8192, 8-byte aligned rows.
 * delta_splits > 1 (fp32 delta, n <= 1024): delta is the sum of
 * delta_splits slices delta_split_stride elements apart (the split partials
 * of tjk_ffn), in a fixed order: the slices form four consecutive groups of
 * q = ceil(delta_splits / 4), each summed in slice order (S_g), and
 * x = res + (((S_0 + S_1) + S_2) + S_3) (empty groups skipped).
 */
int tjk_add_layernorm(const void* res, int res_dtype, int64_t ld_res,
                      const void* delta, int delta_dtype, int64_t ld_delta,
                      int delta_splits, int64_t delta_split_stride,
                      void* res_out, int res_out_dtype, int64_t ld_res_out,
                      void* out, int out_dtype, int64_t ld_out,
                      const float* gamma, const float* beta,
                      int64_t rows, int64_t n, float eps,
                      const int32_t* row_index, int64_t src_rows, int* index_errors,
                      const uint8_t* row_mask, void* stream);

/*
 * C[m, n] = epilogue(sum_k A[m, k] * W[n, k] + bias[n]) -- W in nn.Linear
 * [out, in] layout, so both operands are K-contiguous.
 * A, W, bias and (for TJK_EPI_BIAS / _GELU) C are `dtype`; for
 * TJK_EPI_BIAS_RESIDUAL, C is the fp32 residual updated in place.
 * Accumulation is fp32 (IEEE fp32 MFMA for TJK_F32).  bias may be NULL.
 * Requires k % 8 == 0 (k % 4 for fp32), n % 4 == 0 and 16-byte aligned rows.
 * plan_id selects the tile shape (tjk_gemm_plan_count() of them; -1 = auto).
 */
int tjk_gemm_bias(const void* a, int64_t lda, const void* w, int64_t ldw,
                  const void* bias, void* c, int64_t ldc,
                  int64_t m, int64_t n, int64_t k,
                  int dtype, int epilogue, int plan_id, void* stream);

/*
 * C[m, n] = sum_k A[m, k] * W[n, k] + bias[n] + x[r(m), n], C fp32 and
 * written (not read): tjk_gemm_bias's TJK_EPI_BIAS_RESIDUAL with the
 * residual read from x (`dtype`, leading dimension ld_x) instead of from C.
 * r(m) = rows[m] (an int32 row map, e.g. the packing of prefix-masked
 * tokens), or m when rows is NULL; a row r(m) outside [0, x_rows) adds
 * zeros and is counted once in *index_errors (optional; x may be NULL when
 * x_rows is 0).  The sum is
 * formed exactly as tjk_gemm_bias forms it from a residual holding x's rows
 * in fp32 (the same bits).  Requires what tjk_gemm_bias requires, ld_x %
 * 4 == 0 and x aligned to 4 elements.
 * Replaces, for the first layer, the fp32 copy of x the reference makes
 * (tjkernels/engine.py:230) and writes back from the first
 * fused_add_layernorm (:239-242), and the add of the out-projection into
 * it (:247-252): the first LayerNorm then writes only h.
 */
int tjk_gemm_bias_residual_from(const void* a, int64_t lda, const void* w, int64_t ldw,
                                const void* bias, float* c, int64_t ldc,
                                int64_t m, int64_t n, int64_t k,
                                const void* x, int64_t ld_x, int64_t x_rows,
                                const int32_t* rows, int* index_errors,
                                int dtype, int plan_id, void* stream);

/* Number of GEMM tile plans for `dtype`, and the tile of plan `id`:
 * block_m x block_n outputs, `waves` waves, the K range split over
 * k_groups wave groups whose sums are added at the end.  Plans with the same
 * k_groups add up K in the same order: they give identical results. */
int tjk_gemm_plan_count(int dtype);
int tjk_gemm_plan_info(int dtype, int id, int* block_m, int* block_n, int* waves, int* k_groups);

/*
 * Flash-attention forward over a packed QKV buffer laid out [B, S, 3, H, hd]
 * with element strides (stride_b, stride_s, stride_c, stride_h) and a unit
 * stride on hd.  out[b*S + s, h*hd + i] (leading dimension ld_out).
 *   softmax(Q K^T * scale) V per (b, h), fp32 accumulation and softmax.
 *   causal     keys j > query i are excluded
 *   lengths    if non-NULL, keys j >= lengths[b] are excluded
 *   key_mask   if non-NULL ([B, S] bytes), keys with a 0 byte are excluded
 *   cu_seqlens if non-NULL ([B + 1] int32, non-decreasing, cu_seqlens[0] = 0,
 *              every cu_seqlens[b+1] - cu_seqlens[b] <= seq): packed
 *              sequences; sequence b is rows cu_seqlens[b] .. cu_seqlens[b+1]-1
 *              of both the QKV buffer (row stride stride_s; stride_b unused)
 *              and `out`; only its own rows are read or written.  Exclusive
 *              with key_mask.  The kernels bound what they read by it: a
 *              length above seq is taken as seq, a negative one as 0, a
 *              negative start as 0; the buffers must hold cu_seqlens[B] rows.
 * A query row with no admissible key is written as 0.
 * head_dim in [1, 128], head_dim % 8 == 0 (16-byte aligned rows).
 * plan_id: -1 chooses; 0 software-pipelined (2-byte types); 1 / 2 one / two
 * 32-query blocks per wave; 3 plan 1 with two key splits; 4 whole sequences
 * of at most 128 tokens, one wave per 32 queries (seq > 128 returns
 * TJK_EUNSUPPORTED).  Every plan computes the same function.
 */
int tjk_flash_fwd(const void* qkv, int64_t stride_b, int64_t stride_s,
                  int64_t stride_c, int64_t stride_h,
                  void* out, int64_t ld_out,
                  int batch, int seq, int heads, int head_dim, float scale,
                  int causal, const int32_t* lengths, const uint8_t* key_mask,
                  const int32_t* cu_seqlens, int dtype, int plan_id, void* stream);

/* Number of attention plans for `dtype`. */
int tjk_flash_plan_count(int dtype);

/*
 * Scheduled flash attention over packed sequences (bf16 / fp16): the same
 * math as tjk_flash_fwd with cu_seqlens, but the workgroups follow a work
 * list built by the caller (from the host-known lengths), so long query
 * blocks can start first and be split over their key range.  The launch
 * runs n_lists workgroups (1 <= n_lists <= n_work); workgroup w runs items
 * w, w + n_lists, w + 2*n_lists, ... (< n_work) back to back, in that order
 * (n_lists == n_work: one item per workgroup).  An item { -1, *, *, * } is
 * a hole (padding of a shorter list) and is skipped.
 *   work[4*i .. 4*i+3] = { b*heads + h, qb, t_lo | t_hi << 16, slot }
 *     query block qb (queries 128*qb .. 128*qb+127 of sequence b, head h)
 *     over key tiles t_lo .. t_hi-1 (64 keys each; t_hi is clipped to the
 *     block's last causal / in-sequence tile); slot -1 writes the output
 *     rows; a query block split over its key range is two items: the first
 *     (slot s >= 0) publishes an fp32 partial (unnormalised O, exponent
 *     offset and sum per query) in partials slot s, the second (slot -2-s)
 *     waits for it, merges it into its own ((O_hi a_hi + O_lo a_lo) /
 *     (l_hi a_hi + l_lo a_lo), in that order, so results are deterministic)
 *     and writes the output rows.  The first half must run first: with one
 *     item per workgroup, before the second in the list (workgroups are
 *     dispatched in list order); with lists, at the head of a list (index
 *     < n_lists), and all n_lists workgroups must fit on the device at once.
 *     A second half's wait is bounded: a list breaking these rules costs
 *     NaN rows and an error count, never a hang.
 * Every (query block, key tile) pair of every sequence must be covered
 * exactly once.  partials holds partials_bytes >=
 * tjk_flash_partial_bytes(head_dim, n_slots) bytes: the n_slots partials,
 * an error word and one flag per slot, zero-filled before the first call
 * (NULL is accepted with n_slots == 0, and then nothing is counted);
 * every completed call leaves the flags zero.  The error word counts
 * (never resets) items the kernel could not run as listed: a (b, h) outside
 * the launch (dropped), a slot outside [0, n_slots) (rows written as NaN),
 * and a second half whose wait for its first half timed out (rows written
 * as NaN; the late first half then clears its flag).  Calls sharing a
 * partials buffer must not overlap.  max_seqlen bounds every sequence
 * length.
 */
int tjk_flash_fwd_sched(const void* qkv, int64_t stride_s, int64_t stride_c, int64_t stride_h,
                        void* out, int64_t ld_out, int batch, int max_seqlen, int heads,
                        int head_dim, float scale, int causal, const int32_t* cu_seqlens,
                        const int32_t* work, int n_work, int n_lists, float* partials,
                        size_t partials_bytes, int n_slots, int dtype, void* stream);
size_t tjk_flash_partial_bytes(int head_dim, int n_slots);

/*
 * tjk_flash_fwd_sched without the partials argument: the workspace (split
 * partials, error word, flags) is a static device array of
 * tjk_flash_sched_static_bytes() bytes (4 MiB) that every device the
 * library runs on holds until the process ends; the entry point allocates
 * nothing.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under stream capture, tight serving loops, harnesses that
 * forbid hipMalloc).  n_slots must keep tjk_flash_partial_bytes(head_dim,
 * n_slots) within the array (TJK_EUNSUPPORTED otherwise, nothing launched).
 * Each call first clears the error word and flags with a fill kernel on
 * `stream`; calls on one device share the array, so calls that overlap
 * (unordered streams) race.  The current device must be the stream's.
 */
int tjk_flash_fwd_sched_static(const void* qkv, int64_t stride_s, int64_t stride_c, int64_t stride_h,
                               void* out, int64_t ld_out, int batch, int max_seqlen, int heads,
                               int head_dim, float scale, int causal, const int32_t* cu_seqlens,
                               const int32_t* work, int n_work, int n_lists, int n_slots, int dtype,
                               void* stream);
size_t tjk_flash_sched_static_bytes(void);
/* Workgroups of the scheduled kernel resident per CU (> 0), or a negative /
 * hipError_t status. */
int tjk_flash_sched_occupancy(int head_dim, int dtype);

/*
 * Feed-forward block in one launch, the [rows, f] GELU intermediate kept in
 * LDS.  For the f-slices s = 0 .. splits-1 (f / splits columns each):
 *   P[s] = gelu_erf(A W1[s]^T + b1[s]) W2[:, s]^T  (+ b2 for s = 0)
 * with W1 [f, d], W2 [d, f] (nn.Linear layout), the intermediate rounded to
 * `dtype` as the reference rounds its hidden activation, and
 *   A = a (`dtype`, a_dtype == dtype)                 if ln_gamma == NULL
 *   A = LayerNorm(a) * ln_gamma + ln_beta             otherwise, a the fp32
 *       residual (a_dtype == TJK_F32), biased variance, eps ln_eps; equal
 *       to tjk_add_layernorm's output on the same rows.
 * P[s] is stored as fp32 rows of `out` (leading dimension ld_out) at
 * out + s * split_stride; tjk_add_layernorm(delta_splits = splits) then adds
 * their sum to the residual.  With splits == 1 and accumulate != 0 the
 * result is added into `out` (the fp32 residual) instead.
 * Supported: f / splits in {64, 128}; d in {128, 256, 512} (fp32: 128,
 * 256); see tjk_ffn_supported.  b1 / b2 may be NULL.
 */
int tjk_ffn(const void* a, int a_dtype, int64_t lda, const float* ln_gamma, const float* ln_beta,
            float ln_eps, const void* w1, const void* b1, const void* w2, const void* b2, float* out,
            int64_t ld_out, int64_t split_stride, int splits, int accumulate, int64_t rows, int64_t d,
            int64_t f, int dtype, void* stream);
/* 1 if tjk_ffn takes (d, f, splits, dtype), else 0. */
int tjk_ffn_supported(int64_t d, int64_t f, int splits, int dtype);

/*
 * C = epilogue(LayerNorm(res) W^T + b) in one launch: the LayerNorm of a
 * tjk_add_layernorm call without delta (res fp32 [m, k], gamma / beta fp32,
 * biased variance, eps) computed inside the GEMM into its resident A
 * operand, in place of an add+LayerNorm launch followed by tjk_gemm_bias:
 * the LayerNorm applied in the next GEMM's A-load, for launch-bound row
 * counts (the tiny-shape fusion of README.md:193-196).  h equals
 * tjk_add_layernorm's output bit for bit and the K summation is one chain
 * (K-summation class 1), so C equals tjk_gemm_bias with a class-1 plan on
 * that h.  W [n, k] nn.Linear layout, bias and C in `dtype` (fp16 / bf16);
 * epilogue TJK_EPI_BIAS or TJK_EPI_BIAS_GELU; k in {256, 512, 768, 1024}
 * (tjk_gemm_ln_supported); n % 4 == 0.  plan_id 0-2: 32-row tiles of 32 /
 * 64 / 128 columns (same bits), -1: the widest giving >= 128 workgroups.
 * Each column tile recomputes its rows' LayerNorm, so large row counts
 * belong to the separate launches.
 */
int tjk_gemm_ln(const float* res, int64_t ld_res, const float* gamma, const float* beta, float eps,
                const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc, int64_t m, int64_t n,
                int64_t k, int dtype, int epilogue, int plan_id, void* stream);
/* 1 if tjk_gemm_ln takes (k, dtype), else 0. */
int tjk_gemm_ln_supported(int64_t k, int dtype);
/* Number of tjk_gemm_ln plans (column tile widths). */
int tjk_gemm_ln_plan_count(void);

/*
 * Attention block of one layer in one launch, for sequences of at most 128
 * tokens: per head h (head_dim 64),
 *   [Q | K | V] = x W_qkv[h rows]^T + b_qkv[h]     rounded to `dtype`
 *   ctx_h       = softmax(Q K^T * scale (+ causal mask)) V   rounded to `dtype`
 *   P[h]        = ctx_h W_out[:, 64h : 64h+64]^T (+ b_out for h = 0)   fp32
 * x [rows, d] (leading dimension ld_x), W_qkv [3d, d] and W_out [d, d]
 * contiguous in nn.Linear layout, b_qkv [3d] / b_out [d] (may be NULL).
 * P[h] is stored as fp32 rows of `parts` (leading dimension ld_parts) at
 * parts + h * part_stride; tjk_add_layernorm(delta_splits = heads) then adds
 * their sum -- the out-projection output -- to the residual.  ctx_out (may
 * be NULL; leading dimension ld_ctx) also receives the context [rows, d].
 * Sequences: `batch` of `seq` tokens each (rows b*seq ..), or with
 * cu_seqlens (int32 [batch+1]) packed back to back, every length <= seq
 * (longer ones taken as seq, as in tjk_flash_fwd).
 * The same Q / K / V give the same context bits as tjk_flash_fwd plan 4.
 * Supported: see tjk_attn_block_supported (bf16 / fp16, head_dim 64,
 * d_model = 64 heads in {128, 256, 384, 512}, seq <= 128).
 */
int tjk_attn_block(const void* x, int64_t ld_x, const void* w_qkv, const void* b_qkv,
                   const void* w_out, const void* b_out, float* parts, int64_t ld_parts,
                   int64_t part_stride, void* ctx_out, int64_t ld_ctx, const int32_t* cu_seqlens,
                   int batch, int seq, int heads, int head_dim, float scale, int causal, int dtype,
                   void* stream);
/* 1 if tjk_attn_block takes the shape, else 0. */
int tjk_attn_block_supported(int64_t d_model, int heads, int head_dim, int64_t max_seqlen, int dtype);

#ifdef __cplusplus
}
#endif

#endif /* TJK_H */
