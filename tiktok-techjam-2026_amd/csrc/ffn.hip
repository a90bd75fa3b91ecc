// Feed-forward block in one launch: LayerNorm (optional), GEMM, bias,
// exact-erf GELU, GEMM, bias.
//
//   P[s] = gelu_erf(A W1[s]^T + b1[s]) W2[:, s]^T   (+ b2 for s = 0)
//
// for the f-slices s = 0 .. splits-1 of FC = f / splits columns each, with
// A = h, or A = LayerNorm(res) computed in the kernel.  Replaces the
// reference's fused_ffn (tjkernels/kernels/__init__.py:80-89; Triton
// kernel tjkernels/kernels/ffn.py:21-69), which holds one row block's whole
// [rows, f] intermediate in registers and therefore only takes d, f <= 256
// (ffn.py:103-110).  Here a workgroup owns 32 rows and one f-slice:
//
//   1. the 32 A rows are written into LDS in the compute dtype (LayerNorm
//      computed from the fp32 residual with the arithmetic of the
//      add+LayerNorm kernel, so it equals that kernel's output bit for bit);
//   2. mid = gelu_erf(A W1[s]^T + b1[s]) -- a 32 x FC MFMA tile whose W1 rows
//      stream through an LDS DMA ring while A stays resident; the result is
//      rounded to the compute dtype (as the reference rounds its hidden
//      activation) into LDS: the [rows, f] intermediate never leaves the CU;
//   3. P[s] = mid W2[:, s]^T -- a 32 x d tile, W2's column slice streaming
//      through the same ring, mid resident as the A operand;
//   4. P[s] is stored as fp32 (split 0 adds b2), or with a single split it
//      can be added straight into the fp32 residual.
//
// The splits' partials are summed in split order by the next add+LayerNorm
// (tjk_add_layernorm's delta_splits), which is where the reference adds its
// deferred FFN output (tjkernels/engine.py:232-264): no cross-workgroup
// reduction, no waiting, and the sum order is fixed, so results are
// deterministic.  The split spreads a launch-bound shape (C2: 128 tokens,
// f = 2048) over 64 workgroups instead of 4.

#include "gemm_tiles.h"

namespace tjk {

constexpr int kFfnRows = 32;  // rows per workgroup
constexpr int kFfnWaves = 4;  // each wave owns a quarter of the tile's columns

// Physical 16-byte chunk of logical chunk c in row r of a resident operand
// (rows of >= 16 chunks): an XOR over 16-chunk groups, so the fragment reads
// of 16 consecutive rows at one logical chunk hit 16 different 16-byte bank
// groups.
__device__ __forceinline__ int res_chunk(int c, int r) { return c ^ (r & 15); }

// Geometry of one phase: W tiles of BN rows x BKB bytes of K in a ring of
// STAGES slots, the A operand resident.
template <typename T, int BN, int BKB, int STAGES>
struct FfnPhase {
  static constexpr int NW = kFfnWaves;
  static constexpr int BK = BKB / (int)sizeof(T);     // K elements per tile
  static constexpr int CPR = BKB / 16;                // chunks per ring row
  static constexpr int RPI = 64 / CPR;                // ring rows per DMA instruction
  static constexpr int KS = BK / 16;                  // 16-deep MFMA steps per tile
  static constexpr int CPS = sizeof(T) == 2 ? 2 : 4;  // chunks per 16-deep step
  static constexpr int WTN = BN / NW, FN = WTN / 32;  // wave columns, 32-column blocks
  static constexpr int STAGE = BN * BKB;
  static constexpr int NDMA = BN / (RPI * NW);        // DMA instructions per wave per tile
  static constexpr int LDS = STAGES * STAGE;
  static_assert(NDMA * RPI * NW == BN, "W tile rows must split over the waves");
  static_assert(FN >= 1 && FN * 32 == WTN, "wave columns must be whole 32-column blocks");
  static_assert(STAGES >= 2 && (STAGES - 1) * NDMA <= 63, "vmcnt range");
  static_assert(KS % 2 == 0, "fragment double buffer alternates per 16-deep step");
};

// acc += A[0:32, K] * W[0:BN, K]^T for this wave's columns, where A is
// resident in LDS (row pitch a_pitch bytes, chunks placed by res_chunk) and
// W (rows w_rows valid, leading dimension ldw elements, nk K tiles) streams
// through the ring.  The same pipeline as the GEMM's dtl_accumulate: one
// barrier per K tile, placed before the tile's last 16-deep step; after it
// the next tile's first fragments are read and its DMAs issued under the
// last step's MFMAs (spread over the earlier steps with three or more
// slots).  On return every DMA has landed and the workgroup has met at a
// barrier, so the ring may be reused.
template <typename T, int BN, int BKB, int STAGES>
__device__ __forceinline__ void resident_a_accumulate(
    char* ring, const char* sa, int a_pitch, const T* __restrict__ W, int64_t ldw, int w_rows, int nk,
    f32x16 (&acc)[FfnPhase<T, BN, BKB, STAGES>::FN][1]) {
  typedef FfnPhase<T, BN, BKB, STAGES> G;
  constexpr int NW = G::NW, KS = G::KS, CPR = G::CPR, RPI = G::RPI, CPS = G::CPS;
  constexpr int WTN = G::WTN, FN = G::FN, STAGE = G::STAGE, NDMA = G::NDMA;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;

  // W rows past w_rows and K past the slice read as zero: the descriptor
  // ends at the last valid byte of the slice.
  const int64_t span = ((int64_t)(w_rows - 1) * ldw + (int64_t)nk * G::BK) * (int64_t)sizeof(T);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)span, 0x00020000);
  uint32_t voff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int r = (i * NW + wave) * RPI + lane / CPR;
    voff[i] = (uint32_t)(r * ldw * (int64_t)sizeof(T)) + (uint32_t)(((lane % CPR) ^ swz<BKB>(r)) << 4);
  }
  auto dma = [&](int kt, int q) {
    char* sb = ring + (kt % STAGES) * STAGE;
    const uint32_t kb = kt < nk ? (uint32_t)(kt * BKB) : (uint32_t)kPastEnd;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_void*)(sb + (q * NW + wave) * 1024), 16,
                                             (uint32_t)(voff[q] + kb), 0, 0, 0);
  };
  // W fragment: ring row `row`, logical chunk c (swizzled by swz<BKB>)
  auto wfrag = [&](const char* slot, int row, int ks) -> typename Mfma<T>::frag {
    const char* rb = slot + row * BKB;
    const int sw = swz<BKB>(row);
    if constexpr (sizeof(T) == 2) {
      return *reinterpret_cast<const typename Mfma<T>::frag*>(rb + (((CPS * ks + hi) ^ sw) << 4));
    } else {
      const float4 lo = *reinterpret_cast<const float4*>(rb + (((CPS * ks + 2 * hi) ^ sw) << 4));
      const float4 up = *reinterpret_cast<const float4*>(rb + (((CPS * ks + 2 * hi + 1) ^ sw) << 4));
      typename Mfma<T>::frag f;
      f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
      f[4] = up.x; f[5] = up.y; f[6] = up.z; f[7] = up.w;
      return f;
    }
  };
  // A fragment: resident row l32, K tile kt, step ks
  const char* arow = sa + l32 * a_pitch;
  auto afrag = [&](int kt, int ks) -> typename Mfma<T>::frag {
    const int c = kt * CPR + CPS * ks;
    if constexpr (sizeof(T) == 2) {
      return *reinterpret_cast<const typename Mfma<T>::frag*>(arow + (res_chunk(c + hi, l32) << 4));
    } else {
      const float4 lo = *reinterpret_cast<const float4*>(arow + (res_chunk(c + 2 * hi, l32) << 4));
      const float4 up = *reinterpret_cast<const float4*>(arow + (res_chunk(c + 2 * hi + 1, l32) << 4));
      typename Mfma<T>::frag f;
      f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
      f[4] = up.x; f[5] = up.y; f[6] = up.z; f[7] = up.w;
      return f;
    }
  };

  constexpr bool SPREAD = STAGES >= 3;
  constexpr int PRE = SPREAD ? STAGES - 1 : STAGES;
#pragma unroll
  for (int t = 0; t < PRE; ++t)
#pragma unroll
    for (int q = 0; q < NDMA; ++q) dma(t, q);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PRE - 1) * NDMA) : "memory");
  asm volatile("s_barrier" ::: "memory");
  constexpr int NMF = FN, NDS = FN + 1;  // MFMAs and fragment reads per step
  constexpr int NSLOT = NMF > NDS ? NMF : NDS;
  typename Mfma<T>::frag fa[2], fw[2][FN];
  fa[0] = afrag(0, 0);
#pragma unroll
  for (int i = 0; i < FN; ++i) fw[0][i] = wfrag(ring, wave * WTN + 32 * i + l32, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const char* st = ring + (kt % STAGES) * STAGE;
    const char* nx = ring + ((kt + 1) % STAGES) * STAGE;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int b = ks & 1;
      const bool last = ks + 1 == KS;
      const char* rw = last ? nx : st;
      const int rks = last ? 0 : ks + 1;
      const int rkt = last ? min(kt + 1, nk - 1) : kt;  // (the last tile re-reads itself: unused)
      if (last) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((STAGES - 2) * NDMA) : "memory");
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < NSLOT; ++m) {
        if (m < NMF) Mfma<T>::mma(acc[m][0], fw[b][m], fa[b]);
        if (m == 0) fa[b ^ 1] = afrag(rkt, rks);
        else if (m < NDS) fw[b ^ 1][m - 1] = wfrag(rw, wave * WTN + 32 * (m - 1) + l32, rks);
        if constexpr (SPREAD) {
          constexpr int TOT = (KS - 1) * NSLOT;
          const int i = ks * NSLOT + m;
          if (!last) {
#pragma unroll
            for (int q = i * NDMA / TOT; q < (i + 1) * NDMA / TOT; ++q) dma(kt - 1 + STAGES, q);
          }
        } else if (last) {
#pragma unroll
          for (int q = m * NDMA / NSLOT; q < (m + 1) * NDMA / NSLOT; ++q) dma(kt + STAGES, q);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// LDS plan of one instantiation: [A rows][mid][ring], the ring shared by
// both phases (and by the epilogue staging after phase 2).
template <typename T, int D, int FC>
struct FfnLayout {
  static constexpr int ES = sizeof(T);
  static constexpr int A_PITCH = D * ES, MID_PITCH = FC * ES;
  static constexpr int A_BYTES = kFfnRows * A_PITCH, MID_BYTES = kFfnRows * MID_PITCH;
  static constexpr int BUDGET = 160 * 1024 - A_BYTES - MID_BYTES;
  // phase 2's W2 tile is D rows: 128-byte rows when two slots fit, else 64
  static constexpr int BKB2 = (2 * D * 128 <= BUDGET || ES == 4) ? 128 : 64;
  static constexpr int ST2 = (BUDGET / (D * BKB2)) < 4 ? (BUDGET / (D * BKB2)) : 4;
  static constexpr int ST1 = (BUDGET / (FC * 128)) < 4 ? (BUDGET / (FC * 128)) : 4;
  typedef FfnPhase<T, FC, 128, ST1> P1;
  typedef FfnPhase<T, D, BKB2, ST2> P2;
  static constexpr int STAGE_EPI = kFfnWaves * EpiStage<T, kEpiStoreF32, P2::FN>::BYTES;
  static constexpr int RING = P1::LDS > P2::LDS ? (P1::LDS > STAGE_EPI ? P1::LDS : STAGE_EPI)
                                                 : (P2::LDS > STAGE_EPI ? P2::LDS : STAGE_EPI);
  static constexpr int TOTAL = A_BYTES + MID_BYTES + RING;
  static_assert(A_PITCH >= 256 && MID_PITCH >= 256, "resident rows need >= 16 chunks");
  static_assert(TOTAL <= 160 * 1024, "fused FFN exceeds LDS");
};

template <typename T, int D, int FC, bool LNA>
__global__ __launch_bounds__(256) void ffn_fused_kernel(
    const void* __restrict__ Av, int64_t lda, const float* __restrict__ gamma, const float* __restrict__ beta,
    float eps, const T* __restrict__ W1, const T* __restrict__ b1, const T* __restrict__ W2,
    const T* __restrict__ b2, float* __restrict__ out, int64_t ldo, int64_t split_stride, int accumulate, int M,
    int f, int nrb, int splits) {
  typedef FfnLayout<T, D, FC> Lay;
  typedef typename Lay::P1 P1;
  typedef typename Lay::P2 P2;
  constexpr int VEC = 16 / (int)sizeof(T);
  __shared__ __attribute__((aligned(1024))) char smem[Lay::TOTAL];
  char* ring = smem;
  char* sa = smem + Lay::RING;
  char* smid = sa + Lay::A_BYTES;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  // XCD-contiguous logical order, split-major: the row blocks of one f-slice
  // (which read the same W1 / W2 slices) run on one XCD and share its L2.
  const int t = xcd_remap(blockIdx.x, nrb * splits);
  const int s = t / nrb, m0 = (t % nrb) * kFfnRows, fc0 = s * FC;

  // ---- 1. A rows into LDS (compute dtype)
  if constexpr (LNA) {
    // one row per wave at a time; lane l owns the 4-element chunks l, l+64, ...
    constexpr int NCH = D / 4, MAXCH = (NCH + 63) / 64;
    const float* res = static_cast<const float*>(Av);
    for (int r = wave; r < kFfnRows; r += kFfnWaves) {
      const int m = m0 + r;
      char* row = sa + r * Lay::A_PITCH;
      if (m >= M) {
        for (int c = lane; c < Lay::A_PITCH / 16; c += 64) *reinterpret_cast<uint4*>(row + (c << 4)) = make_uint4(0, 0, 0, 0);
        continue;
      }
      float4 x[MAXCH];
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) {
        const int c = lane + 64 * j;
        x[j] = (NCH % 64 == 0 || c < NCH) ? reinterpret_cast<const float4*>(res + (int64_t)m * lda)[c]
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      // the add+LayerNorm kernel's arithmetic, operation for operation
      float sm = 0.f;
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) sm += (x[j].x + x[j].y) + (x[j].z + x[j].w);
      const float inv_n = 1.0f / (float)D;
      const float mean = wave_sum(sm) * inv_n;
      float q = 0.f;
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) {
        const int c = lane + 64 * j;
        if (NCH % 64 == 0 || c < NCH) {
          const float a = x[j].x - mean, b = x[j].y - mean, cc = x[j].z - mean, d = x[j].w - mean;
          q += (a * a + b * b) + (cc * cc + d * d);
        }
      }
      const float var = wave_sum(q) * inv_n;
      const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
      for (int j = 0; j < MAXCH; ++j) {
        const int c = lane + 64 * j;
        if (NCH % 64 == 0 || c < NCH) {
          const float4 g = reinterpret_cast<const float4*>(gamma)[c];
          const float4 bb = reinterpret_cast<const float4*>(beta)[c];
          float4 y;
          y.x = (x[j].x - mean) * rstd * g.x + bb.x;
          y.y = (x[j].y - mean) * rstd * g.y + bb.y;
          y.z = (x[j].z - mean) * rstd * g.z + bb.z;
          y.w = (x[j].w - mean) * rstd * g.w + bb.w;
          // elements 4c .. 4c+3: chunk 4c / VEC, byte (4c % VEC) * size
          const int ch = (4 * c) / VEC, off = ((4 * c) % VEC) * (int)sizeof(T);
          *reinterpret_cast<typename Quad<T>::raw*>(row + (res_chunk(ch, r) << 4) + off) = Quad<T>::from(y);
        }
      }
    }
  } else {
    const T* A = static_cast<const T*>(Av);
    constexpr int CPRA = Lay::A_PITCH / 16;  // 16-byte chunks per row
    for (int i = tid; i < kFfnRows * CPRA; i += 256) {
      const int r = i / CPRA, c = i % CPRA, m = m0 + r;
      const uint4 v = m < M ? *reinterpret_cast<const uint4*>(A + (int64_t)m * lda + c * VEC) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(sa + r * Lay::A_PITCH + (res_chunk(c, r) << 4)) = v;
    }
  }
  __syncthreads();

  // ---- 2. mid = gelu_erf(A W1[fc0 : fc0+FC]^T + b1), rounded, into LDS
  {
    f32x16 acc[P1::FN][1];
    zero_acc<T, 1, P1::FN>(acc);
    resident_a_accumulate<T, FC, 128, Lay::ST1>(ring, sa, Lay::A_PITCH, W1 + (int64_t)fc0 * D, D, FC,
                                                D / P1::BK, acc);
#pragma unroll
    for (int i = 0; i < P1::FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = wave * P1::WTN + 32 * i + 8 * g + 4 * hi;  // column within the slice
        const float4 bv = b1 ? Quad<T>::to(*reinterpret_cast<const typename Quad<T>::raw*>(b1 + fc0 + n))
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        float4 v = make_float4(gelu_erf(acc[i][0][4 * g + 0] + bv.x), gelu_erf(acc[i][0][4 * g + 1] + bv.y),
                               gelu_erf(acc[i][0][4 * g + 2] + bv.z), gelu_erf(acc[i][0][4 * g + 3] + bv.w));
        const int ch = n / VEC, off = (n % VEC) * (int)sizeof(T);
        *reinterpret_cast<typename Quad<T>::raw*>(smid + l32 * Lay::MID_PITCH + (res_chunk(ch, l32) << 4) + off) =
            Quad<T>::from(v);
      }
  }
  __syncthreads();

  // ---- 3. P = mid W2[:, fc0 : fc0+FC]^T
  f32x16 acc[P2::FN][1];
  zero_acc<T, 1, P2::FN>(acc);
  resident_a_accumulate<T, D, Lay::BKB2, Lay::ST2>(ring, smid, Lay::MID_PITCH, W2 + fc0, f, D, FC / P2::BK, acc);

  // ---- 4. store the fp32 partial (split 0 adds b2), or add into the residual
  char* stage = ring + wave * EpiStage<T, kEpiStoreF32, P2::FN>::BYTES;
  if (accumulate) {
    epilogue<T, TJK_EPI_BIAS_RESIDUAL, 1, P2::FN>(acc, b2, out, ldo, M, D, m0, wave * P2::WTN, lane, stage);
  } else {
    epilogue<T, kEpiStoreF32, 1, P2::FN>(acc, s == 0 ? b2 : nullptr, out + (int64_t)s * split_stride, ldo, M, D, m0,
                                         wave * P2::WTN, lane, stage);
  }
}

// Instantiated (d, f-slice) pairs: d in {128, 256, 512}, slice 128.
template <typename T, int D, int FC>
static int launch_ffn_d(const void* a, int64_t lda, const float* gamma, const float* beta, float eps,
                        const void* w1, const void* b1, const void* w2, const void* b2, float* out, int64_t ldo,
                        int64_t split_stride, int accumulate, int M, int f, int splits, hipStream_t s) {
  const int nrb = (M + kFfnRows - 1) / kFfnRows;
  const dim3 grid((unsigned)(nrb * splits)), block(256);
  if (gamma != nullptr)
    hipLaunchKernelGGL((ffn_fused_kernel<T, D, FC, true>), grid, block, 0, s, a, lda, gamma, beta, eps,
                       (const T*)w1, (const T*)b1, (const T*)w2, (const T*)b2, out, ldo, split_stride, accumulate, M,
                       f, nrb, splits);
  else
    hipLaunchKernelGGL((ffn_fused_kernel<T, D, FC, false>), grid, block, 0, s, a, lda, gamma, beta, eps,
                       (const T*)w1, (const T*)b1, (const T*)w2, (const T*)b2, out, ldo, split_stride, accumulate, M,
                       f, nrb, splits);
  return check_launch("tjk_ffn");
}

constexpr int kFfnSlice = 128;

static bool ffn_shape_ok(int64_t d, int64_t f, int64_t splits, int dtype) {
  if (dtype != TJK_F32 && dtype != TJK_F16 && dtype != TJK_BF16) return false;
  if (splits < 1 || f % splits != 0 || f / splits != kFfnSlice) return false;
  if (dtype == TJK_F32) return d == 128 || d == 256;
  return d == 128 || d == 256 || d == 512;
}

template <typename T>
static int launch_ffn(int64_t d, const void* a, int64_t lda, const float* gamma, const float* beta, float eps,
                      const void* w1, const void* b1, const void* w2, const void* b2, float* out, int64_t ldo,
                      int64_t split_stride, int accumulate, int M, int f, int splits, hipStream_t s) {
  switch (d) {
    case 128:
      return launch_ffn_d<T, 128, kFfnSlice>(a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride,
                                             accumulate, M, f, splits, s);
    case 256:
      return launch_ffn_d<T, 256, kFfnSlice>(a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride,
                                             accumulate, M, f, splits, s);
    default:
      if constexpr (sizeof(T) == 2)
        return launch_ffn_d<T, 512, kFfnSlice>(a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride,
                                               accumulate, M, f, splits, s);
      return fail(TJK_EUNSUPPORTED, "tjk_ffn: d=%lld not supported for fp32", (long long)d);
  }
}

}  // namespace tjk

using namespace tjk;

extern "C" int tjk_ffn_supported(int64_t d, int64_t f, int splits, int dtype) {
  return ffn_shape_ok(d, f, splits, dtype) ? 1 : 0;
}

extern "C" int tjk_ffn(const void* a, int a_dtype, int64_t lda, const float* ln_gamma, const float* ln_beta,
                       float ln_eps, const void* w1, const void* b1, const void* w2, const void* b2, float* out,
                       int64_t ld_out, int64_t split_stride, int splits, int accumulate, int64_t rows, int64_t d,
                       int64_t f, int dtype, void* stream) {
  if (rows < 0 || d <= 0 || f <= 0) return fail(TJK_EINVAL, "tjk_ffn: bad shape rows=%lld d=%lld f=%lld",
                                                (long long)rows, (long long)d, (long long)f);
  if (!ffn_shape_ok(d, f, splits, dtype))
    return fail(TJK_EUNSUPPORTED, "tjk_ffn: unsupported d=%lld f=%lld splits=%d dtype=%d (f / splits must be %d; "
                "d in {128, 256, 512}, fp32 d <= 256)", (long long)d, (long long)f, splits, dtype, kFfnSlice);
  if (rows == 0) return TJK_OK;
  if (rows > INT32_MAX / 2 || f > INT32_MAX || d * f * dtype_size(dtype) >= kPastEnd)
    return fail(TJK_EUNSUPPORTED, "tjk_ffn: shape exceeds the 32-bit buffer range");
  if (!a || !w1 || !w2 || !out) return fail(TJK_EINVAL, "tjk_ffn: null pointer");
  const bool ln = ln_gamma != nullptr;
  if (ln != (ln_beta != nullptr)) return fail(TJK_EINVAL, "tjk_ffn: ln_gamma and ln_beta go together");
  if (ln ? a_dtype != TJK_F32 : a_dtype != dtype)
    return fail(TJK_EINVAL, "tjk_ffn: the input is the fp32 residual with a LayerNorm, else h in the compute dtype");
  if (accumulate && splits != 1) return fail(TJK_EINVAL, "tjk_ffn: accumulate needs a single split");
  const int es = dtype_size(dtype), aes = dtype_size(a_dtype);
  if (lda < d || ld_out < d) return fail(TJK_EINVAL, "tjk_ffn: leading dimension smaller than d");
  if ((lda * aes) % 16 || ld_out % 4) return fail(TJK_EUNSUPPORTED, "tjk_ffn: rows must stay 16-byte aligned");
  if (splits > 1 && split_stride < rows * ld_out)
    return fail(TJK_EINVAL, "tjk_ffn: split_stride smaller than one split's rows x ld_out");
  if (((uintptr_t)a & 15) || ((uintptr_t)w1 & 15) || ((uintptr_t)w2 & 15) || ((uintptr_t)out & 15) ||
      ((uintptr_t)b1 & (4 * es - 1)) || ((uintptr_t)b2 & (4 * es - 1)) || ((uintptr_t)ln_gamma & 15) ||
      ((uintptr_t)ln_beta & 15) || (split_stride * 4) % 16)
    return fail(TJK_EUNSUPPORTED, "tjk_ffn: misaligned pointer");
  const int M = (int)rows, fi = (int)f;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case TJK_F32:
      return launch_ffn<float>(d, a, lda, ln_gamma, ln_beta, ln_eps, w1, b1, w2, b2, out, ld_out, split_stride,
                               accumulate, M, fi, splits, s);
    case TJK_F16:
      return launch_ffn<f16>(d, a, lda, ln_gamma, ln_beta, ln_eps, w1, b1, w2, b2, out, ld_out, split_stride,
                             accumulate, M, fi, splits, s);
    default:
      return launch_ffn<bf16>(d, a, lda, ln_gamma, ln_beta, ln_eps, w1, b1, w2, b2, out, ld_out, split_stride,
                              accumulate, M, fi, splits, s);
  }
}
