// Fused residual-add + LayerNorm (HBM-bound row kernel) and the ABI's
// bookkeeping entry points (version, last error).
//
// One wave64 owns one row.  Lane l handles the 4-element chunks
// l, l+64, l+128, ... of the row, so every load/store instruction of a wave
// covers 64 consecutive chunks (fully coalesced 512 B/1 KB transactions).
// The row is held in registers: x = res (+ delta) in fp32, the fp32 residual
// is optionally written back, mean and biased variance are two wave
// reductions over the register copy (two-pass, like the reference kernel
// tjkernels/kernels/layernorm.py:63-66), then gamma/beta are applied and
// the output is written in its own dtype.  A row mask (the final-LN zeroing
// of tjkernels/engine.py:267-268) writes padded rows as exact zeros.
//
// A row index turns the kernel into a gather / scatter: output row r reads
// input row row_index[r], or is written as zeros when the index is negative
// or not below the input's row count (the latter also counted in an error
// word).
// The engine uses it to pack the valid tokens of prefix-masked sequences
// into consecutive rows (first LayerNorm) and to put them back in [B, S]
// order with zero padded rows (final LayerNorm).

#include <stdarg.h>
#include <stdio.h>

#include <type_traits>

#include "tjk_common.h"

namespace tjk {

static thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  return TJK_OK;
}

// Stores chunk c (4 elements) of the updated residual row in the residual
// stream's dtype: fp32, or a 2-byte type rounded to nearest even (the
// reference's residual_dtype knob, tjkernels/plans.py:33-36).  ro_dtype is
// the same for every lane of a launch, so the branch is uniform.
// `row` is the wave's output row (res_row); a wave's stores cover whole row
// segments.
template <typename W>
__device__ __forceinline__ void store_res_chunk(const W& row, int c, int ro_dtype, const float4& v) {
  if (ro_dtype == TJK_F32)
    row.put(c * 16, v);
  else if (ro_dtype == TJK_F16)
    row.put(c * 8, Quad<f16>::from(v));
  else
    row.put(c * 8, Quad<bf16>::from(v));
}

// Stores into row `row` (n elements) of the residual output, written
// through the L2 when WT.
template <bool WT>
__device__ __forceinline__ auto res_row(void* base, int ro_dtype, int64_t row, int64_t ld, int n) {
  const int es = ro_dtype == TJK_F32 ? 4 : 2;
  return RowOut(static_cast<char*>(base) + row * ld * es, (int64_t)n * es, WT).writer<WT>();
}

// Stores into row `row` (n elements) of the normalised output, written
// through the L2 when WT.
template <bool WT, typename TOut>
__device__ __forceinline__ auto out_row(TOut* out, int64_t row, int64_t ld, int n) {
  return RowOut(out + row * ld, (int64_t)n * (int64_t)sizeof(TOut), WT).writer<WT>();
}

// The gather / scatter map of a launch: output row r reads input row
// index[r] (index == NULL: row r).  An entry at or past src_rows (the rows
// res / delta hold) is not followed: the row is written as a hole (zeros)
// and counted in *errors (if not NULL), once per row, by the calling lane.
struct RowMap {
  const int32_t* __restrict__ index;
  int64_t src_rows;
  int* errors;
};

__device__ __forceinline__ int64_t map_row(const RowMap& rm, int64_t row, bool count) {
  if (rm.index == nullptr) return row;
  const int64_t s = rm.index[row];
  if (s < rm.src_rows) return s;
  if (count && rm.errors != nullptr) atomicAdd(rm.errors, 1);
  return -1;
}

// FULL: n == 256 * MAXCH, every lane's chunks in range (no per-chunk guards).
// ln_threads(WT) / 64 rows per workgroup: in launches that write through
// (WT, at least kWtMinBytes of output) 8 rows measured 0.3% faster than 4
// (and 2, 16) over whole C4 and C5 forwards, builds alternating on one box;
// in C2's 128-row launches 8 rows made the forward 1.4% slower, so smaller
// launches keep 4.
constexpr int ln_threads(bool wt) { return wt ? 512 : 256; }
template <typename TRes, typename TDelta, typename TOut, int MAXCH, bool FULL, bool WT>
__global__ __launch_bounds__(ln_threads(WT)) void add_layernorm_kernel(
    const TRes* res, int64_t ld_res,  // may alias res_out (in-place update)
    const TDelta* __restrict__ delta, int64_t ld_delta,
    void* res_out, int ro_dtype, int64_t ld_res_out,
    TOut* __restrict__ out, int64_t ld_out,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    int64_t rows, int n, float eps, RowMap rmap, const uint8_t* __restrict__ row_mask) {
  const int lane = threadIdx.x & 63;
  const int nch = n >> 2;
  constexpr int NT = ln_threads(WT);
  const int64_t row = (int64_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
  const bool live = row < rows;
  const int64_t src = !live ? -1 : map_row(rmap, row, lane == 0);

  // gamma / beta staged once per workgroup (NT / 64 rows), by every thread before
  // any wave leaves: read from L2 by each wave they were 8 KB per 1024-wide
  // row, more than the row itself.  In launches large enough to write
  // through (WT) and up to 2048-wide rows, their loads go out first, in
  // flight together with the row's (measured: 6.4 -> 4.9 us per C4
  // LayerNorm together with the write-through stores; in launches of a few
  // hundred rows, 0.1 us slower).
  constexpr int GPT = (64 * MAXCH + NT - 1) / NT;  // gamma / beta chunks per thread
  constexpr bool EARLY = WT && GPT <= 2;
  float4 gl[EARLY ? GPT : 1], bl[EARLY ? GPT : 1];
  if constexpr (EARLY) {
#pragma unroll
    for (int u = 0; u < GPT; ++u) {
      const int c = min((int)threadIdx.x + NT * u, nch - 1);
      gl[u] = reinterpret_cast<const float4*>(gamma)[c];
      bl[u] = reinterpret_cast<const float4*>(beta)[c];
    }
  }

  // Chunks past the row end are read at the last chunk and dropped: loads
  // under a per-lane condition are waited for one at a time.
  float4 x[MAXCH];
  if (src >= 0) {
    const TRes* rrow = res + src * ld_res;
    typename Quad<TRes>::raw rr[MAXCH];
#pragma unroll
    for (int j = 0; j < MAXCH; ++j)
      rr[j] = reinterpret_cast<const typename Quad<TRes>::raw*>(rrow)[FULL ? lane + 64 * j : min(lane + 64 * j, nch - 1)];
    if (delta != nullptr) {
      const TDelta* drow = delta + src * ld_delta;
      typename Quad<TDelta>::raw dr[MAXCH];
#pragma unroll
      for (int j = 0; j < MAXCH; ++j)
        dr[j] = reinterpret_cast<const typename Quad<TDelta>::raw*>(drow)[FULL ? lane + 64 * j
                                                                             : min(lane + 64 * j, nch - 1)];
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) {
        x[j] = Quad<TRes>::to(rr[j]);
        const float4 d = Quad<TDelta>::to(dr[j]);
        x[j].x += d.x; x[j].y += d.y; x[j].z += d.z; x[j].w += d.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) x[j] = Quad<TRes>::to(rr[j]);
    }
#pragma unroll
    for (int j = 0; j < MAXCH; ++j)
      if (!FULL && lane + 64 * j >= nch) x[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __shared__ float4 s_gamma[64 * MAXCH], s_beta[64 * MAXCH];
  if constexpr (EARLY) {
#pragma unroll
    for (int u = 0; u < GPT; ++u) {
      const int c = (int)threadIdx.x + NT * u;
      if (c < nch) {
        s_gamma[c] = gl[u];
        s_beta[c] = bl[u];
      }
    }
  } else {
    for (int c = threadIdx.x; c < nch; c += NT) {
      s_gamma[c] = reinterpret_cast<const float4*>(gamma)[c];
      s_beta[c] = reinterpret_cast<const float4*>(beta)[c];
    }
  }
  __syncthreads();
  if (!live) return;
  constexpr int OB = (int)sizeof(typename Quad<TOut>::raw);  // bytes per output chunk
  if (src < 0) {  // scatter hole: an exact zero row, nothing read
    const auto w = out_row<WT>(out, row, ld_out, n);
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) {
      const int c = lane + 64 * j;
      if (FULL || c < nch)
        w.put(c * OB, Quad<TOut>::from(make_float4(0.f, 0.f, 0.f, 0.f)));
    }
    return;
  }

  float s = 0.f;
  if (res_out != nullptr) {
    const auto w = res_row<WT>(res_out, ro_dtype, row, ld_res_out, n);
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) {
      const int c = lane + 64 * j;
      if (FULL || c < nch) store_res_chunk(w, c, ro_dtype, x[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) s += (x[j].x + x[j].y) + (x[j].z + x[j].w);
  const float inv_n = 1.0f / (float)n;
  const float mean = wave_sum(s) * inv_n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) {
    const int c = lane + 64 * j;
    if (FULL || c < nch) {
      const float a = x[j].x - mean, b = x[j].y - mean, cc = x[j].z - mean, d = x[j].w - mean;
      q += (a * a + b * b) + (cc * cc + d * d);
    }
  }
  const float var = wave_sum(q) * inv_n;
  const float rstd = 1.0f / sqrtf(var + eps);
  const bool zero = row_mask != nullptr && row_mask[row] == 0;

  const auto w = out_row<WT>(out, row, ld_out, n);
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) {
    const int c = lane + 64 * j;
    if (FULL || c < nch) {
      float4 y;
      if (zero) {
        y = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float4 g = s_gamma[c], b = s_beta[c];
        y.x = (x[j].x - mean) * rstd * g.x + b.x;
        y.y = (x[j].y - mean) * rstd * g.y + b.y;
        y.z = (x[j].z - mean) * rstd * g.z + b.z;
        y.w = (x[j].w - mean) * rstd * g.w + b.w;
      }
      w.put(c * OB, Quad<TOut>::from(y));
    }
  }
}

// Split deltas (the fused FFN's fp32 f-slice partials): one row per
// workgroup.  Wave w sums the consecutive slices [w q, (w + 1) q), q =
// ceil(n_delta / 4), in order, with all of its loads issued together; wave
// 0 then adds the four sums in wave order, x = res + (((S_0 + S_1) + S_2) +
// S_3) (waves without slices skipped), and normalises the row with the row
// kernel's arithmetic.  Spreading one row's slices over four waves keeps a
// launch of a few hundred rows from waiting out n_delta / 4 load latencies.
template <typename TRes, typename TOut, int MAXCH, bool WT>
__global__ __launch_bounds__(256) void add_layernorm_parts_kernel(
    const TRes* res, int64_t ld_res,  // may alias res_out (in-place update)
    const float* __restrict__ parts, int64_t ld_parts, int n_parts, int64_t part_stride,
    void* res_out, int ro_dtype, int64_t ld_res_out, TOut* __restrict__ out, int64_t ld_out,
    const float* __restrict__ gamma, const float* __restrict__ beta, int64_t rows, int n, float eps,
    RowMap rmap, const uint8_t* __restrict__ row_mask) {
  constexpr int PER = 32 / MAXCH;  // slices per load batch of one wave
  constexpr int OB = (int)sizeof(typename Quad<TOut>::raw);  // bytes per output chunk
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = n >> 2;
  const int64_t row = blockIdx.x;
  const int64_t src = map_row(rmap, row, threadIdx.x == 0);
  __shared__ float4 s_sum[3][MAXCH][64];
  if (src < 0) {  // scatter hole: an exact zero row
    if (wave == 0) {
      const auto w = out_row<WT>(out, row, ld_out, n);
#pragma unroll
      for (int j = 0; j < MAXCH; ++j)
        if (lane + 64 * j < nch)
          w.put((lane + 64 * j) * OB, Quad<TOut>::from(make_float4(0.f, 0.f, 0.f, 0.f)));
    }
    return;
  }
  // Every load is unconditional, chunks past the row end read at the last
  // chunk (and dropped): loads under a per-lane condition are waited for one
  // at a time.  Wave 0 also fetches gamma / beta up front.
  const int q = (n_parts + 3) / 4, p_lo = min(wave * q, n_parts), p_hi = min(p_lo + q, n_parts);
  int cl[MAXCH];  // clamped chunk index
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) cl[j] = min(lane + 64 * j, nch - 1);
  float4 x[MAXCH], gv[MAXCH], bv[MAXCH];
  if (wave == 0) {
    const TRes* rrow = res + src * ld_res;
    typename Quad<TRes>::raw rr[MAXCH];
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) rr[j] = reinterpret_cast<const typename Quad<TRes>::raw*>(rrow)[cl[j]];
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) {
      gv[j] = reinterpret_cast<const float4*>(gamma)[cl[j]];
      bv[j] = reinterpret_cast<const float4*>(beta)[cl[j]];
    }
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) x[j] = Quad<TRes>::to(rr[j]);
  }
  float4 acc[MAXCH];
  const float* prow = parts + src * ld_parts;
  for (int p0 = p_lo; p0 < p_hi; p0 += PER) {
    float4 v[PER][MAXCH];
#pragma unroll
    for (int u = 0; u < PER; ++u)
#pragma unroll
      for (int j = 0; j < MAXCH; ++j)
        v[u][j] = p0 + u < p_hi ? reinterpret_cast<const float4*>(prow + (int64_t)(p0 + u) * part_stride)[cl[j]]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      if (p0 + u == p_lo) {
#pragma unroll
        for (int j = 0; j < MAXCH; ++j) acc[j] = v[u][j];
      } else if (p0 + u < p_hi) {
#pragma unroll
        for (int j = 0; j < MAXCH; ++j) {
          acc[j].x += v[u][j].x; acc[j].y += v[u][j].y; acc[j].z += v[u][j].z; acc[j].w += v[u][j].w;
        }
      }
    }
  }
  if (wave > 0 && p_lo < p_hi) {
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) s_sum[wave - 1][j][lane] = acc[j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    if (w * q < n_parts) {
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) {
        const float4 o = s_sum[w - 1][j][lane];
        acc[j].x += o.x; acc[j].y += o.y; acc[j].z += o.z; acc[j].w += o.w;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) {
    x[j].x += acc[j].x; x[j].y += acc[j].y; x[j].z += acc[j].z; x[j].w += acc[j].w;
    if (lane + 64 * j >= nch) x[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (res_out != nullptr) {
    const auto w = res_row<WT>(res_out, ro_dtype, row, ld_res_out, n);
#pragma unroll
    for (int j = 0; j < MAXCH; ++j)
      if (lane + 64 * j < nch) store_res_chunk(w, lane + 64 * j, ro_dtype, x[j]);
  }
  float sm = 0.f;
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) sm += (x[j].x + x[j].y) + (x[j].z + x[j].w);
  const float inv_n = 1.0f / (float)n;
  const float mean = wave_sum(sm) * inv_n;
  float qq = 0.f;
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) {
    if (lane + 64 * j < nch) {
      const float a = x[j].x - mean, b = x[j].y - mean, cc = x[j].z - mean, d = x[j].w - mean;
      qq += (a * a + b * b) + (cc * cc + d * d);
    }
  }
  const float var = wave_sum(qq) * inv_n;
  const float rstd = 1.0f / sqrtf(var + eps);
  const bool zero = row_mask != nullptr && row_mask[row] == 0;
  const auto w = out_row<WT>(out, row, ld_out, n);
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) {
      float4 y;
      if (zero) {
        y = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float4 g = gv[j], b = bv[j];
        y.x = (x[j].x - mean) * rstd * g.x + b.x;
        y.y = (x[j].y - mean) * rstd * g.y + b.y;
        y.z = (x[j].z - mean) * rstd * g.z + b.z;
        y.w = (x[j].w - mean) * rstd * g.w + b.w;
      }
      w.put(c * OB, Quad<TOut>::from(y));
    }
  }
}

template <typename TRes, typename TOut>
static int launch_ln_parts(const void* res, int64_t ld_res, const float* parts, int64_t ld_parts, int n_parts,
                           int64_t part_stride, void* res_out, int ro_dtype, int64_t ld_res_out, void* out, int64_t ld_out,
                           const float* gamma, const float* beta, int64_t rows, int n, float eps,
                           const RowMap& rmap, const uint8_t* row_mask, hipStream_t stream) {
  const int nch = n / 4;
  const dim3 grid((unsigned)rows), block(256);
  const bool wt = rows * n * (int64_t)sizeof(TOut) >= kWtMinBytes;
#define TJK_LNP1(MC, WT)                                                                                      \
  hipLaunchKernelGGL((add_layernorm_parts_kernel<TRes, TOut, MC, WT>), grid, block, 0, stream, (const TRes*)res, \
                     ld_res, parts, ld_parts, n_parts, part_stride, res_out, ro_dtype, ld_res_out, (TOut*)out, ld_out, gamma, \
                     beta, rows, n, eps, rmap, row_mask)
#define TJK_LNP(MC)            \
  do {                         \
    if (wt)                    \
      TJK_LNP1(MC, true);      \
    else                       \
      TJK_LNP1(MC, false);     \
  } while (0)
  if (nch <= 64) TJK_LNP(1);
  else if (nch <= 128) TJK_LNP(2);
  else TJK_LNP(4);
#undef TJK_LNP
#undef TJK_LNP1
  return check_launch("tjk_add_layernorm");
}

template <typename TRes, typename TDelta, typename TOut>
static int launch_ln(const void* res, int64_t ld_res, const void* delta, int64_t ld_delta, int n_delta,
                     int64_t delta_stride, void* res_out, int ro_dtype, int64_t ld_res_out, void* out, int64_t ld_out,
                     const float* gamma, const float* beta, int64_t rows, int n, float eps,
                     const RowMap& rmap, const uint8_t* row_mask, hipStream_t stream) {
  if constexpr (std::is_same<TDelta, float>::value) {
    if (n_delta > 1)
      return launch_ln_parts<TRes, TOut>(res, ld_res, (const float*)delta, ld_delta, n_delta, delta_stride, res_out,
                                         ro_dtype, ld_res_out, out, ld_out, gamma, beta, rows, n, eps, rmap, row_mask,
                                         stream);
  }
  const int nch = n / 4;
  const bool wt = rows * n * (int64_t)sizeof(TOut) >= kWtMinBytes;
  const int rpw = ln_threads(wt) / 64;  // rows per workgroup
  const dim3 grid((unsigned)((rows + rpw - 1) / rpw)), block(ln_threads(wt));
#define TJK_LN_LAUNCH1(MC, FULL, WT)                                                                   \
  hipLaunchKernelGGL((add_layernorm_kernel<TRes, TDelta, TOut, MC, FULL, WT>), grid, block, 0, stream,     \
                     (const TRes*)res, ld_res, (const TDelta*)delta, ld_delta, res_out, ro_dtype, ld_res_out, \
                     (TOut*)out, ld_out, gamma, beta, rows, n, eps, rmap, row_mask)
#define TJK_LN_LAUNCH(MC, FULL)        \
  do {                                 \
    if (wt)                            \
      TJK_LN_LAUNCH1(MC, FULL, true);  \
    else                               \
      TJK_LN_LAUNCH1(MC, FULL, false); \
  } while (0)
#define TJK_LN_CASE(MC)                                   \
  if (nch <= 64 * MC) {                                   \
    if (nch == 64 * MC) TJK_LN_LAUNCH(MC, true);          \
    else TJK_LN_LAUNCH(MC, false);                        \
    return check_launch("tjk_add_layernorm");             \
  }
  // widths of 3 and 6 chunks per lane (d = 768, 1536: C3's model width) run
  // without per-chunk guards too
  if (nch == 64 * 3) {
    TJK_LN_LAUNCH(3, true);
    return check_launch("tjk_add_layernorm");
  }
  if (nch == 64 * 6) {
    TJK_LN_LAUNCH(6, true);
    return check_launch("tjk_add_layernorm");
  }
  TJK_LN_CASE(1)
  TJK_LN_CASE(2)
  TJK_LN_CASE(4)
  TJK_LN_CASE(8)
  TJK_LN_CASE(16)
  TJK_LN_CASE(32)
#undef TJK_LN_CASE
#undef TJK_LN_LAUNCH
#undef TJK_LN_LAUNCH1
  return fail(TJK_EUNSUPPORTED, "tjk_add_layernorm: n=%d exceeds 8192", n);
}

template <typename TRes, typename TDelta>
static int dispatch_out(int out_dtype, const void* res, int64_t ld_res, const void* delta,
                        int64_t ld_delta, int n_delta, int64_t delta_stride, void* res_out, int ro_dtype, int64_t ld_res_out, void* out,
                        int64_t ld_out, const float* gamma, const float* beta, int64_t rows,
                        int n, float eps, const RowMap& rmap, const uint8_t* row_mask, hipStream_t stream) {
  switch (out_dtype) {
    case TJK_F32:
      return launch_ln<TRes, TDelta, float>(res, ld_res, delta, ld_delta, n_delta, delta_stride, res_out, ro_dtype, ld_res_out, out, ld_out,
                                            gamma, beta, rows, n, eps, rmap, row_mask, stream);
    case TJK_F16:
      return launch_ln<TRes, TDelta, f16>(res, ld_res, delta, ld_delta, n_delta, delta_stride, res_out, ro_dtype, ld_res_out, out, ld_out,
                                          gamma, beta, rows, n, eps, rmap, row_mask, stream);
    case TJK_BF16:
      return launch_ln<TRes, TDelta, bf16>(res, ld_res, delta, ld_delta, n_delta, delta_stride, res_out, ro_dtype, ld_res_out, out, ld_out,
                                           gamma, beta, rows, n, eps, rmap, row_mask, stream);
  }
  return fail(TJK_EINVAL, "tjk_add_layernorm: bad out dtype %d", out_dtype);
}

template <typename TRes>
static int dispatch_delta(int delta_dtype, int out_dtype, const void* res, int64_t ld_res,
                          const void* delta, int64_t ld_delta, int n_delta, int64_t delta_stride, void* res_out, int ro_dtype, int64_t ld_res_out,
                          void* out, int64_t ld_out, const float* gamma, const float* beta,
                          int64_t rows, int n, float eps, const RowMap& rmap,
                          const uint8_t* row_mask, hipStream_t stream) {
  switch (delta_dtype) {
    case TJK_F32:
      return dispatch_out<TRes, float>(out_dtype, res, ld_res, delta, ld_delta, n_delta, delta_stride, res_out, ro_dtype, ld_res_out, out,
                                       ld_out, gamma, beta, rows, n, eps, rmap, row_mask, stream);
    case TJK_F16:
      return dispatch_out<TRes, f16>(out_dtype, res, ld_res, delta, ld_delta, n_delta, delta_stride, res_out, ro_dtype, ld_res_out, out,
                                     ld_out, gamma, beta, rows, n, eps, rmap, row_mask, stream);
    case TJK_BF16:
      return dispatch_out<TRes, bf16>(out_dtype, res, ld_res, delta, ld_delta, n_delta, delta_stride, res_out, ro_dtype, ld_res_out, out,
                                      ld_out, gamma, beta, rows, n, eps, rmap, row_mask, stream);
  }
  return fail(TJK_EINVAL, "tjk_add_layernorm: bad delta dtype %d", delta_dtype);
}

}  // namespace tjk

using namespace tjk;

extern "C" int tjk_abi_version(void) { return TJK_ABI_VERSION; }

extern "C" const char* tjk_last_error_string(void) { return g_err; }

extern "C" int tjk_add_layernorm(const void* res, int res_dtype, int64_t ld_res,
                                 const void* delta, int delta_dtype, int64_t ld_delta,
                                 int delta_splits, int64_t delta_split_stride,
                                 void* res_out, int res_out_dtype, int64_t ld_res_out,
                                 void* out, int out_dtype, int64_t ld_out,
                                 const float* gamma, const float* beta,
                                 int64_t rows, int64_t n, float eps,
                                 const int32_t* row_index, int64_t src_rows, int* index_errors,
                                 const uint8_t* row_mask, void* stream) {
  g_err[0] = 0;
  if (rows < 0 || n <= 0) return fail(TJK_EINVAL, "tjk_add_layernorm: bad shape rows=%lld n=%lld", (long long)rows, (long long)n);
  if (row_index && src_rows < 0) return fail(TJK_EINVAL, "tjk_add_layernorm: negative src_rows with a row_index");
  if (rows == 0) return TJK_OK;
  if (!res || !out || !gamma || !beta) return fail(TJK_EINVAL, "tjk_add_layernorm: null pointer");
  if (res_out && res_out_dtype != TJK_F32 && res_out_dtype != TJK_F16 && res_out_dtype != TJK_BF16)
    return fail(TJK_EINVAL, "tjk_add_layernorm: bad res_out dtype %d", res_out_dtype);
  const int ro_dtype = res_out ? res_out_dtype : TJK_F32;
  if (n % 4 != 0) return fail(TJK_EUNSUPPORTED, "tjk_add_layernorm: n=%lld not a multiple of 4", (long long)n);
  if (n > 8192) return fail(TJK_EUNSUPPORTED, "tjk_add_layernorm: n=%lld exceeds 8192", (long long)n);
  if (ld_res < n || ld_out < n || (delta && ld_delta < n) || (res_out && ld_res_out < n))
    return fail(TJK_EINVAL, "tjk_add_layernorm: leading dimension smaller than n");
  if (ld_res % 4 || ld_out % 4 || (delta && ld_delta % 4) || (res_out && ld_res_out % 4))
    return fail(TJK_EUNSUPPORTED, "tjk_add_layernorm: leading dimensions must be multiples of 4");
  {
    // Chunks are 4 elements: 8-byte aligned for 2-byte types, 16 for fp32.
    const uintptr_t need_res = 4 * dtype_size(res_dtype) - 1, need_out = 4 * dtype_size(out_dtype) - 1;
    const uintptr_t need_delta = 4 * dtype_size(delta ? delta_dtype : res_dtype) - 1;
    const uintptr_t need_ro = 4 * dtype_size(ro_dtype) - 1;
    if (((uintptr_t)res & need_res) || ((uintptr_t)out & need_out) || ((uintptr_t)delta & need_delta) ||
        ((uintptr_t)res_out & need_ro) || ((uintptr_t)gamma & 15) || ((uintptr_t)beta & 15))
      return fail(TJK_EUNSUPPORTED, "tjk_add_layernorm: misaligned pointer");
  }
  // A gather / scatter reads rows other than the one it writes, and a
  // residual written in place in another dtype overwrites bytes of other
  // rows: either would race with other rows' reads.
  if (res_out && (const void*)res_out == res && (row_index || res_out_dtype != res_dtype || ld_res_out != ld_res))
    return fail(TJK_EINVAL, "tjk_add_layernorm: res_out may alias res only in place (same dtype and leading "
                "dimension, no row_index)");
  if (delta && (delta_splits < 1 || (delta_splits > 1 && (delta_split_stride < rows * ld_delta ||
                                                          delta_split_stride % 4 != 0))))
    return fail(TJK_EINVAL, "tjk_add_layernorm: delta_splits=%d needs a split stride >= rows x ld_delta, "
                "multiple of 4", delta_splits);
  if (delta && delta_splits > 1 && (n > 1024 || delta_dtype != TJK_F32))
    return fail(TJK_EUNSUPPORTED, "tjk_add_layernorm: split deltas are fp32 rows of n <= 1024");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const RowMap rmap{row_index, row_index ? src_rows : rows, index_errors};
  const int dd = delta ? delta_dtype : res_dtype;
  const int nd = delta ? delta_splits : 0;
  switch (res_dtype) {
    case TJK_F32:
      return dispatch_delta<float>(dd, out_dtype, res, ld_res, delta, ld_delta, nd, delta_split_stride, res_out, ro_dtype, ld_res_out, out,
                                   ld_out, gamma, beta, rows, (int)n, eps, rmap, row_mask, s);
    case TJK_F16:
      return dispatch_delta<f16>(dd, out_dtype, res, ld_res, delta, ld_delta, nd, delta_split_stride, res_out, ro_dtype, ld_res_out, out,
                                 ld_out, gamma, beta, rows, (int)n, eps, rmap, row_mask, s);
    case TJK_BF16:
      return dispatch_delta<bf16>(dd, out_dtype, res, ld_res, delta, ld_delta, nd, delta_split_stride, res_out, ro_dtype, ld_res_out, out,
                                  ld_out, gamma, beta, rows, (int)n, eps, rmap, row_mask, s);
  }
  return fail(TJK_EINVAL, "tjk_add_layernorm: bad res dtype %d", res_dtype);
}
