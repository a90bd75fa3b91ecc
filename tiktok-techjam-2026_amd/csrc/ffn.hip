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
//   3. P[s] = mid W2[:, s]^T -- a 32 x d tile with mid resident as the A
//      operand and W2's column slice in LDS;
//   4. P[s] is stored as fp32 (split 0 adds b2), or with a single split it
//      can be added straight into the fp32 residual.
//
// The kernel is latency-bound at the shapes it serves (C2: 128 tokens), so
// the weight copies start first: when W2's slice fits in LDS beside W1's
// ring (64-column slices) all of it is in flight from the start, else its
// first tiles load during the GELU; W1's first tiles load while the
// LayerNorm runs.
//
// The splits' partials are summed by the next add+LayerNorm
// (tjk_add_layernorm's delta_splits, in a fixed order), which is where the
// reference adds its deferred FFN output (tjkernels/engine.py:232-264): no
// cross-workgroup reduction, no waiting, deterministic results.
//
// The same resident-A machinery gives tjk_gemm_ln (end of this file): one
// GEMM whose A operand is the LayerNorm of the fp32 residual, computed in the
// kernel (LayerNorm applied in the GEMM's A-load).

#include "gemm_tiles.h"

namespace tjk {

constexpr int kFfnRows = 32;  // rows per workgroup
constexpr int kFfnWaves = 4;

// Physical 16-byte chunk of logical chunk c in row r of a resident operand
// whose rows hold NCH chunks: an XOR over groups of min(NCH, 16) chunks, so
// the fragment reads of consecutive rows at one logical chunk hit different
// 16-byte bank groups.
template <int NCH>
__device__ __forceinline__ int res_chunk(int c, int r) {
  static_assert(NCH >= 8 && (NCH % 8) == 0, "resident rows need a multiple of 8 chunks");
  return c ^ (r & ((NCH >= 16 ? 16 : 8) - 1));
}

// Geometry of one phase: W tiles of BN rows x BKB bytes of K in STAGES LDS
// slots, the A operand resident.  WN waves own BN / WN columns each (the
// others only help with the copies).
template <typename T, int BN, int BKB, int STAGES, int WN>
struct FfnPhase {
  static constexpr int NW = kFfnWaves;
  static constexpr int BK = BKB / (int)sizeof(T);     // K elements per tile
  static constexpr int CPR = BKB / 16;                // chunks per ring row
  static constexpr int RPI = 64 / CPR;                // ring rows per DMA instruction
  static constexpr int KS = BK / 16;                  // 16-deep MFMA steps per tile
  static constexpr int CPS = sizeof(T) == 2 ? 2 : 4;  // chunks per 16-deep step
  static constexpr int WTN = BN / WN, FN = WTN / 32;  // wave columns, 32-column blocks
  static constexpr int STAGE = BN * BKB;
  static constexpr int NDMA = BN / (RPI * NW);        // DMA instructions per wave per tile
  static constexpr int LDS = STAGES * STAGE;
  static_assert(NDMA * RPI * NW == BN, "W tile rows must split over the waves");
  static_assert(WN >= 1 && WN <= NW && FN >= 1 && FN * 32 * WN == BN, "whole 32-column blocks per wave");
  static_assert(STAGES >= 2 && (STAGES - 1) * NDMA <= 63, "vmcnt range");
  static_assert(KS % 2 == 0, "fragment double buffer alternates per 16-deep step");
};

// The W operand of one phase streaming through LDS slots while the A
// operand (32 rows, row pitch APITCH bytes, chunks placed by res_chunk)
// stays resident:  acc += A[0:32, K] * W[0:BN, K]^T for this wave's
// columns.  W has w_rows valid rows (leading dimension ldw elements) and nk
// K tiles.  prologue() issues the first tiles' DMAs; they depend on nothing
// in LDS, so a caller issues them before preparing A.  accumulate() is the
// GEMM's dtl_accumulate pipeline: one barrier per K tile, placed before the
// tile's last 16-deep step; after it the next tile's first fragments are
// read and its DMAs issued under the last step's MFMAs (spread over the
// earlier steps with three or more slots).  On return every DMA has landed
// and the workgroup has met at a barrier, so the slots may be reused.
// DMAs of streams issued after this one's prologue must not be outstanding
// when accumulate() starts (each stream's waits count only its own).
template <typename T, int BN, int BKB, int STAGES, int WN, int APITCH>
struct WStream {
  typedef FfnPhase<T, BN, BKB, STAGES, WN> G;
  static constexpr int NW = G::NW, KS = G::KS, CPR = G::CPR, RPI = G::RPI, CPS = G::CPS;
  static constexpr int WTN = G::WTN, FN = G::FN, STAGE = G::STAGE, NDMA = G::NDMA;
  static constexpr int ACH = APITCH / 16;  // chunks per resident A row
  static constexpr bool SPREAD = STAGES >= 3;
  static constexpr int PRE = SPREAD ? STAGES - 1 : STAGES;  // tiles in flight before the loop

  char* ring;
  int nk, lane, wave, l32, hi;
  __amdgpu_buffer_rsrc_t rsw;
  uint32_t voff[NDMA];

  __device__ __forceinline__ WStream(char* ring_, const T* __restrict__ W, int64_t ldw, int w_rows, int nk_)
      : ring(ring_), nk(nk_) {
    const int tid = threadIdx.x;
    lane = tid & 63;
    wave = tid >> 6;
    l32 = lane & 31;
    hi = lane >> 5;
    // W rows past w_rows and K past the slice read as zero: the descriptor
    // ends at the last valid byte of the slice.
    const int64_t span = ((int64_t)(w_rows - 1) * ldw + (int64_t)nk * G::BK) * (int64_t)sizeof(T);
    rsw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)span, 0x00020000);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int r = (i * NW + wave) * RPI + lane / CPR;
      voff[i] = (uint32_t)(r * ldw * (int64_t)sizeof(T)) + (uint32_t)(((lane % CPR) ^ swz<BKB>(r)) << 4);
    }
  }

  __device__ __forceinline__ void dma(int kt, int q) {
    char* sb = ring + (kt % STAGES) * STAGE;
    const uint32_t kb = kt < nk ? (uint32_t)(kt * BKB) : (uint32_t)kPastEnd;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_void*)(sb + (q * NW + wave) * 1024), 16,
                                             (uint32_t)(voff[q] + kb), 0, 0, 0);
  }

  __device__ __forceinline__ void prologue() {
#pragma unroll
    for (int t = 0; t < PRE; ++t)
#pragma unroll
      for (int q = 0; q < NDMA; ++q) dma(t, q);
  }

  // W fragment: slot row `row`, step ks (chunks swizzled by swz<BKB>)
  __device__ __forceinline__ typename Mfma<T>::frag wfrag(const char* slot, int row, int ks) const {
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
  }

  // A fragment: resident row l32, K tile kt, step ks
  __device__ __forceinline__ typename Mfma<T>::frag afrag(const char* arow, int kt, int ks) const {
    const int c = kt * CPR + CPS * ks;
    if constexpr (sizeof(T) == 2) {
      return *reinterpret_cast<const typename Mfma<T>::frag*>(arow + (res_chunk<ACH>(c + hi, l32) << 4));
    } else {
      const float4 lo = *reinterpret_cast<const float4*>(arow + (res_chunk<ACH>(c + 2 * hi, l32) << 4));
      const float4 up = *reinterpret_cast<const float4*>(arow + (res_chunk<ACH>(c + 2 * hi + 1, l32) << 4));
      typename Mfma<T>::frag f;
      f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
      f[4] = up.x; f[5] = up.y; f[6] = up.z; f[7] = up.w;
      return f;
    }
  }

  // Requires prologue() before, and A complete in LDS and published by a
  // workgroup barrier.
  __device__ __forceinline__ void accumulate(const char* sa, f32x16 (&acc)[FN][1]) {
    const char* arow = sa + l32 * APITCH;
    const bool active = wave < WN;  // wave-uniform
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PRE - 1) * NDMA) : "memory");
    asm volatile("s_barrier" ::: "memory");
    constexpr int NMF = FN, NDS = FN + 1;  // MFMAs and fragment reads per step
    constexpr int NSLOT = NMF > NDS ? NMF : NDS;
    typename Mfma<T>::frag fa[2], fw[2][FN];
    if (active) {
      fa[0] = afrag(arow, 0, 0);
#pragma unroll
      for (int i = 0; i < FN; ++i) fw[0][i] = wfrag(ring, wave * WTN + 32 * i + l32, 0);
    }
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
          if (active) {
            if (m < NMF) Mfma<T>::mma(acc[m][0], fw[b][m], fa[b]);
            if (m == 0) fa[b ^ 1] = afrag(arow, rkt, rks);
            else if (m < NDS) fw[b ^ 1][m - 1] = wfrag(rw, wave * WTN + 32 * (m - 1) + l32, rks);
          }
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
};

template <int A, int B> struct Max { static constexpr int v = A > B ? A : B; };
template <int A, int B> struct Min { static constexpr int v = A < B ? A : B; };

// LDS plan of one (dtype, d, slice) instantiation.  Regions, in order:
//   W1 ring (ST1 slots of FC rows x 128 B),
//   W2 slots (SEP: the whole slice, two tiles; else the W1 ring is reused
//   for W2 after phase 1), A rows, mid rows.  The epilogue staging of phase
//   3 overlays the weight regions.
template <typename T, int D, int FC>
struct FfnLayout {
  static constexpr int ES = sizeof(T), KB = 1024;
  static constexpr int A_PITCH = D * ES, MID_PITCH = FC * ES;
  static constexpr int A_BYTES = kFfnRows * A_PITCH, MID_BYTES = kFfnRows * MID_PITCH;
  static constexpr int WN1 = Min<FC / 32, kFfnWaves>::v;  // waves computing phase 1
  static constexpr int ST1 = 4;
  typedef FfnPhase<T, FC, 128, ST1, WN1> P1;
  // W2 slice in two K tiles when it fits beside everything else
  static constexpr int BKB_SEP = FC * ES / 2;
  static constexpr bool SEP = (BKB_SEP == 64 || BKB_SEP == 128) &&
                              P1::LDS + 2 * D * BKB_SEP + A_BYTES + MID_BYTES <= 160 * KB;
  static constexpr int BUDGET_SHARED = 160 * KB - A_BYTES - MID_BYTES;
  static constexpr int BKB2 = SEP ? BKB_SEP : ((2 * D * 128 <= BUDGET_SHARED || ES == 4) ? 128 : 64);
  static constexpr int ST2 = SEP ? 2 : Min<BUDGET_SHARED / (D * BKB2), 4>::v;
  typedef FfnPhase<T, D, BKB2, ST2, kFfnWaves> P2;
  static constexpr int W2_OFF = SEP ? P1::LDS : 0;
  static constexpr int WEIGHTS = SEP ? P1::LDS + P2::LDS : Max<P1::LDS, P2::LDS>::v;
  static constexpr int STAGE_EPI = kFfnWaves * EpiStage<T, kEpiStoreF32, P2::FN>::BYTES;
  static constexpr int RING = Max<WEIGHTS, STAGE_EPI>::v;
  static constexpr int TOTAL = RING + A_BYTES + MID_BYTES;
  static_assert(TOTAL <= 160 * KB, "fused FFN exceeds LDS");
};

// Rows m0 .. m0 + 31 of LayerNorm(res) (res fp32, biased variance) written
// into LDS in the compute dtype: row r at sa + r * APITCH, its 16-byte
// chunks placed by res_chunk.  Rows wave, wave + 4, ...: every row's loads
// are issued at once, then started() runs (the caller's weight copies,
// which then land during the loads' latency), then the LayerNorm of each
// row.  Rows past M are written as zeros.
template <typename T, int D, int APITCH, typename Started>
__device__ __forceinline__ void layernorm_rows_to_lds(char* sa, const float* __restrict__ res, int64_t lda,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta, float eps, int m0, int M,
                                                      Started started) {
  constexpr int VEC = 16 / (int)sizeof(T), ACH = APITCH / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // lane l owns the 4-element chunks l, l+64, ... of a row
  constexpr int NCH = D / 4, MAXCH = (NCH + 63) / 64, RPW = kFfnRows / kFfnWaves;
  float4 x[RPW][MAXCH], gm[MAXCH], bt[MAXCH];
#pragma unroll
  for (int j = 0; j < MAXCH; ++j) {
    const int c = lane + 64 * j;
    const bool in = NCH % 64 == 0 || c < NCH;
    gm[j] = in ? reinterpret_cast<const float4*>(gamma)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    bt[j] = in ? reinterpret_cast<const float4*>(beta)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int m = m0 + wave + kFfnWaves * i;
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) {
      const int c = lane + 64 * j;
      x[i][j] = (m < M && (NCH % 64 == 0 || c < NCH)) ? reinterpret_cast<const float4*>(res + (int64_t)m * lda)[c]
                                                      : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  started();
  // the add+LayerNorm kernel's arithmetic, operation for operation, with
  // the eight rows' wave reductions interleaved
  const float inv_n = 1.0f / (float)D;
  float mean[RPW], rstd[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) sm += (x[i][j].x + x[i][j].y) + (x[i][j].z + x[i][j].w);
    mean[i] = sm;
  }
  wave_sum_n<RPW>(mean);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    mean[i] *= inv_n;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) {
      const int c = lane + 64 * j;
      if (NCH % 64 == 0 || c < NCH) {
        const float a = x[i][j].x - mean[i], b = x[i][j].y - mean[i], cc = x[i][j].z - mean[i],
                    d = x[i][j].w - mean[i];
        q += (a * a + b * b) + (cc * cc + d * d);
      }
    }
    rstd[i] = q;
  }
  wave_sum_n<RPW>(rstd);
#pragma unroll
  for (int i = 0; i < RPW; ++i) rstd[i] = 1.0f / sqrtf(rstd[i] * inv_n + eps);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = wave + kFfnWaves * i, m = m0 + r;
    char* row = sa + r * APITCH;
#pragma unroll
    for (int j = 0; j < MAXCH; ++j) {
      const int c = lane + 64 * j;
      if (NCH % 64 == 0 || c < NCH) {
        float4 y;
        if (m < M) {
          y.x = (x[i][j].x - mean[i]) * rstd[i] * gm[j].x + bt[j].x;
          y.y = (x[i][j].y - mean[i]) * rstd[i] * gm[j].y + bt[j].y;
          y.z = (x[i][j].z - mean[i]) * rstd[i] * gm[j].z + bt[j].z;
          y.w = (x[i][j].w - mean[i]) * rstd[i] * gm[j].w + bt[j].w;
        } else {
          y = make_float4(0.f, 0.f, 0.f, 0.f);  // rows past the input: zeros
        }
        // elements 4c .. 4c+3: chunk 4c / VEC, byte (4c % VEC) * size
        const int ch = (4 * c) / VEC, off = ((4 * c) % VEC) * (int)sizeof(T);
        *reinterpret_cast<typename Quad<T>::raw*>(row + (res_chunk<ACH>(ch, r) << 4) + off) = Quad<T>::from(y);
      }
    }
  }
}

// Av and out are not __restrict__: with LayerNorm 2 inside (LNA) and an
// unsplit accumulating launch they are the same fp32 residual, read into LDS
// before the barrier that precedes every store to out.
template <typename T, int D, int FC, bool LNA>
__global__ __launch_bounds__(256) void ffn_fused_kernel(
    const void* Av, int64_t lda, const float* __restrict__ gamma, const float* __restrict__ beta,
    float eps, const T* __restrict__ W1, const T* __restrict__ b1, const T* __restrict__ W2,
    const T* __restrict__ b2, float* out, int64_t ldo, int64_t split_stride, int accumulate, int M,
    int f, int nrb, int splits) {
  typedef FfnLayout<T, D, FC> Lay;
  typedef typename Lay::P1 P1;
  typedef typename Lay::P2 P2;
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int ACH = Lay::A_PITCH / 16, MCH = Lay::MID_PITCH / 16;
  __shared__ __attribute__((aligned(1024))) char smem[Lay::TOTAL];
  char* ring = smem;
  char* sa = smem + Lay::RING;
  char* smid = sa + Lay::A_BYTES;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, l32 = lane & 31;
  // XCD-contiguous logical order, split-major: the row blocks of one f-slice
  // (which read the same W1 / W2 slices) run on one XCD and share its L2.
  const int t = xcd_remap(blockIdx.x, nrb * splits);
  const int s = t / nrb, m0 = (t % nrb) * kFfnRows, fc0 = s * FC;

  // this wave's b1 columns, raw, read before any DMA so that no later wait
  // for them has to drain the weight copies.  The loads are unconditional
  // (without b1 they read W1 and the values are dropped): a load under a
  // condition is waited for on its own, one memory round trip per load.
  typedef typename Quad<T>::raw Raw;
  const T* b1p = b1 != nullptr ? b1 + fc0 : W1;
  Raw b1r[P1::FN][4];
#pragma unroll
  for (int i = 0; i < P1::FN; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = min(wave, Lay::WN1 - 1) * P1::WTN + 32 * i + 8 * g + 4 * hi;
      b1r[i][g] = *reinterpret_cast<const Raw*>(b1p + n);
    }

  WStream<T, FC, 128, Lay::ST1, Lay::WN1, Lay::A_PITCH> w1s(ring, W1 + (int64_t)fc0 * D, D, FC, D / P1::BK);
  WStream<T, D, Lay::BKB2, Lay::ST2, kFfnWaves, Lay::MID_PITCH> w2s(ring + Lay::W2_OFF, W2 + fc0, f, D,
                                                                    FC / P2::BK);
  // The streams' waits count their own copies only: W2's (when it has its
  // own slots) are issued first, so they are older than all of W1's.
  auto start_copies = [&]() {
    if constexpr (Lay::SEP) w2s.prologue();
    w1s.prologue();
  };

  // ---- 1. A rows into LDS (compute dtype)
  if constexpr (LNA) {
    layernorm_rows_to_lds<T, D, Lay::A_PITCH>(sa, static_cast<const float*>(Av), lda, gamma, beta, eps, m0, M,
                                              start_copies);
  } else {
    const T* A = static_cast<const T*>(Av);
    constexpr int PER = kFfnRows * ACH / 256;
    static_assert(PER * 256 == kFfnRows * ACH, "A rows must split over the threads");
    uint4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = tid + 256 * k, r = i / ACH, c = i % ACH, m = m0 + r;
      v[k] = m < M ? *reinterpret_cast<const uint4*>(A + (int64_t)m * lda + c * VEC) : make_uint4(0, 0, 0, 0);
    }
    start_copies();
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = tid + 256 * k, r = i / ACH, c = i % ACH;
      *reinterpret_cast<uint4*>(sa + r * Lay::A_PITCH + (res_chunk<ACH>(c, r) << 4)) = v[k];
    }
  }
  __syncthreads();

  // ---- 2. mid = gelu_erf(A W1[fc0 : fc0+FC]^T + b1), rounded, into LDS
  {
    f32x16 acc[P1::FN][1];
    zero_acc<T, 1, P1::FN>(acc);
    w1s.accumulate(sa, acc);
    if constexpr (!Lay::SEP) w2s.prologue();  // the ring is free: W2's first tiles load under the GELU
    if (wave < Lay::WN1) {
#pragma unroll
      for (int i = 0; i < P1::FN; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = wave * P1::WTN + 32 * i + 8 * g + 4 * hi;  // column within the slice
          const float4 bv = b1 != nullptr ? Quad<T>::to(b1r[i][g]) : make_float4(0.f, 0.f, 0.f, 0.f);
          float4 v = make_float4(gelu_erf(acc[i][0][4 * g + 0] + bv.x), gelu_erf(acc[i][0][4 * g + 1] + bv.y),
                                 gelu_erf(acc[i][0][4 * g + 2] + bv.z), gelu_erf(acc[i][0][4 * g + 3] + bv.w));
          const int ch = n / VEC, off = (n % VEC) * (int)sizeof(T);
          *reinterpret_cast<typename Quad<T>::raw*>(smid + l32 * Lay::MID_PITCH + (res_chunk<MCH>(ch, l32) << 4) +
                                                    off) = Quad<T>::from(v);
        }
    }
  }
  __syncthreads();

  // ---- 3. P = mid W2[:, fc0 : fc0+FC]^T
  f32x16 acc[P2::FN][1];
  zero_acc<T, 1, P2::FN>(acc);
  w2s.accumulate(smid, acc);

  // ---- 4. store the fp32 partial (split 0 adds b2), or add into the residual
  char* stage = ring + wave * EpiStage<T, kEpiStoreF32, P2::FN>::BYTES;
  if (accumulate) {
    epilogue<T, TJK_EPI_BIAS_RESIDUAL, 1, P2::FN>(acc, b2, out, ldo, M, D, m0, wave * P2::WTN, lane, stage);
  } else {
    epilogue<T, kEpiStoreF32, 1, P2::FN>(acc, s == 0 ? b2 : nullptr, out + (int64_t)s * split_stride, ldo, M, D, m0,
                                         wave * P2::WTN, lane, stage);
  }
}

// Instantiated: d in {128, 256, 512} (fp32: 128, 256), f-slices of 64 or
// 128 columns.
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

static bool ffn_shape_ok(int64_t d, int64_t f, int64_t splits, int dtype) {
  if (dtype != TJK_F32 && dtype != TJK_F16 && dtype != TJK_BF16) return false;
  if (splits < 1 || f % splits != 0 || (f / splits != 64 && f / splits != 128)) return false;
  if (dtype == TJK_F32) return d == 128 || d == 256;
  return d == 128 || d == 256 || d == 512;
}

template <typename T, int FC>
static int launch_ffn_fc(int64_t d, const void* a, int64_t lda, const float* gamma, const float* beta, float eps,
                         const void* w1, const void* b1, const void* w2, const void* b2, float* out, int64_t ldo,
                         int64_t split_stride, int accumulate, int M, int f, int splits, hipStream_t s) {
  switch (d) {
    case 128:
      return launch_ffn_d<T, 128, FC>(a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride, accumulate,
                                      M, f, splits, s);
    case 256:
      return launch_ffn_d<T, 256, FC>(a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride, accumulate,
                                      M, f, splits, s);
    default:
      if constexpr (sizeof(T) == 2)
        return launch_ffn_d<T, 512, FC>(a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride,
                                        accumulate, M, f, splits, s);
      return fail(TJK_EUNSUPPORTED, "tjk_ffn: d=%lld not supported for fp32", (long long)d);
  }
}

template <typename T>
static int launch_ffn(int64_t d, const void* a, int64_t lda, const float* gamma, const float* beta, float eps,
                      const void* w1, const void* b1, const void* w2, const void* b2, float* out, int64_t ldo,
                      int64_t split_stride, int accumulate, int M, int f, int splits, hipStream_t s) {
  if (f / splits == 64)
    return launch_ffn_fc<T, 64>(d, a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride, accumulate, M,
                                f, splits, s);
  return launch_ffn_fc<T, 128>(d, a, lda, gamma, beta, eps, w1, b1, w2, b2, out, ldo, split_stride, accumulate, M,
                               f, splits, s);
}

// ------------------------------------------------- LayerNorm-prologue GEMM
//
// C = epi(LayerNorm(res) W^T + b) for a launch of a few hundred rows (the
// QKV and FFN1 projections at C2's 128 tokens), in place of an
// add+LayerNorm launch followed by the GEMM: a workgroup owns 32 rows and
// BN columns, computes the LayerNorm of its rows into the resident A operand
// (layernorm_rows_to_lds, bit for bit the add+LayerNorm kernel's h) while
// the first W tiles load, and streams W through a 4-slot LDS ring.  Each
// column tile recomputes its rows' LayerNorm (64 KB of fp32 at d = 512, from
// L2), which is why this is for launch-bound row counts only.  The K
// summation is one chain of K tiles in order, the GEMM's K-summation class 1:
// with the same h the result equals the class-1 GEMM plans bit for bit.
template <typename T, int D, int BN, int EPI>
struct LnGemmLayout {
  static constexpr int A_PITCH = D * (int)sizeof(T), A_BYTES = kFfnRows * A_PITCH;
  static constexpr int WN = Min<BN / 32, kFfnWaves>::v;  // waves computing
  // W ring deep enough for every K tile (up to 8) to be in flight at once:
  // the launch is latency-bound, and a shallower ring waits out the DMA
  // latency again every few K tiles
  static constexpr int STAGES = Min<Min<D / 64, 8>::v, (160 * 1024 - A_BYTES) / (BN * 128)>::v;
  typedef FfnPhase<T, BN, 128, STAGES, WN> P;
  static constexpr int STAGE_EPI = kFfnWaves * EpiStage<T, EPI, P::FN>::BYTES;
  static constexpr int RING = Max<P::LDS, STAGE_EPI>::v;  // the epilogue staging overlays the ring
  static constexpr int TOTAL = RING + A_BYTES;
  static_assert(TOTAL <= 160 * 1024, "LayerNorm-prologue GEMM exceeds LDS");
};

template <typename T, int D, int BN, int EPI>
__global__ __launch_bounds__(256) void gemm_ln_kernel(
    const float* __restrict__ res, int64_t ld_res, const float* __restrict__ gamma, const float* __restrict__ beta,
    float eps, const T* __restrict__ W, int64_t ldw, const T* __restrict__ bias, T* __restrict__ C, int64_t ldc,
    int M, int N, int nrb, int ncb) {
  typedef LnGemmLayout<T, D, BN, EPI> Lay;
  typedef typename Lay::P P;
  __shared__ __attribute__((aligned(1024))) char smem[Lay::TOTAL];
  char* ring = smem;
  char* sa = smem + Lay::RING;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // XCD-contiguous logical order, column-tile-major: the row blocks of one
  // column tile (which stream the same W rows) run on one XCD
  const int t = xcd_remap(blockIdx.x, nrb * ncb);
  const int n0 = (t / nrb) * BN, m0 = (t % nrb) * kFfnRows;

  WStream<T, BN, 128, Lay::STAGES, Lay::WN, Lay::A_PITCH> ws(ring, W + (int64_t)n0 * ldw, ldw, min(BN, N - n0),
                                                             D / P::BK);
  layernorm_rows_to_lds<T, D, Lay::A_PITCH>(sa, res, ld_res, gamma, beta, eps, m0, M, [&]() { ws.prologue(); });
  __syncthreads();
  f32x16 acc[P::FN][1];
  zero_acc<T, 1, P::FN>(acc);
  ws.accumulate(sa, acc);
  if (wave < Lay::WN)
    epilogue<T, EPI, 1, P::FN>(acc, bias, C, ldc, M, N, m0, n0 + wave * P::WTN, lane,
                               ring + wave * EpiStage<T, EPI, P::FN>::BYTES);
}

// Column tiles of the plans: 32, 64 or 128 columns (1, 2 or 4 waves
// computing; all four load rows and copy W).
constexpr int kLnGemmPlans = 3;
constexpr int kLnGemmBn[kLnGemmPlans] = {32, 64, 128};

template <typename T, int D, int BN>
static int launch_gemm_ln_bn(const float* res, int64_t ld_res, const float* gamma, const float* beta, float eps,
                             const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc, int M, int N,
                             int epi, hipStream_t s) {
  const int nrb = (M + kFfnRows - 1) / kFfnRows, ncb = (N + BN - 1) / BN;
  const dim3 grid((unsigned)(nrb * ncb)), block(256);
  if (epi == TJK_EPI_BIAS_GELU)
    hipLaunchKernelGGL((gemm_ln_kernel<T, D, BN, TJK_EPI_BIAS_GELU>), grid, block, 0, s, res, ld_res, gamma, beta,
                       eps, (const T*)w, ldw, (const T*)bias, (T*)c, ldc, M, N, nrb, ncb);
  else
    hipLaunchKernelGGL((gemm_ln_kernel<T, D, BN, TJK_EPI_BIAS>), grid, block, 0, s, res, ld_res, gamma, beta, eps,
                       (const T*)w, ldw, (const T*)bias, (T*)c, ldc, M, N, nrb, ncb);
  return check_launch("tjk_gemm_ln");
}

template <typename T, int D>
static int launch_gemm_ln_d(int plan, const float* res, int64_t ld_res, const float* gamma, const float* beta,
                            float eps, const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc, int M,
                            int N, int epi, hipStream_t s) {
  switch (plan) {
    case 0:
      return launch_gemm_ln_bn<T, D, 32>(res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
    case 1:
      return launch_gemm_ln_bn<T, D, 64>(res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
    default:
      return launch_gemm_ln_bn<T, D, 128>(res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
  }
}

template <typename T>
static int launch_gemm_ln(int64_t k, int plan, const float* res, int64_t ld_res, const float* gamma,
                          const float* beta, float eps, const void* w, int64_t ldw, const void* bias, void* c,
                          int64_t ldc, int M, int N, int epi, hipStream_t s) {
  switch (k) {
    case 256:
      return launch_gemm_ln_d<T, 256>(plan, res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
    case 512:
      return launch_gemm_ln_d<T, 512>(plan, res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
    case 768:
      return launch_gemm_ln_d<T, 768>(plan, res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
    default:
      return launch_gemm_ln_d<T, 1024>(plan, res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, M, N, epi, s);
  }
}

static bool gemm_ln_shape_ok(int64_t k, int dtype) {
  return (dtype == TJK_F16 || dtype == TJK_BF16) && (k == 256 || k == 512 || k == 768 || k == 1024);
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
    return fail(TJK_EUNSUPPORTED, "tjk_ffn: unsupported d=%lld f=%lld splits=%d dtype=%d (f / splits must be 64 or "
                "128; d in {128, 256, 512}, fp32 d <= 256)", (long long)d, (long long)f, splits, dtype);
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

extern "C" int tjk_gemm_ln_supported(int64_t k, int dtype) { return gemm_ln_shape_ok(k, dtype) ? 1 : 0; }

extern "C" int tjk_gemm_ln_plan_count(void) { return kLnGemmPlans; }

extern "C" int tjk_gemm_ln(const float* res, int64_t ld_res, const float* gamma, const float* beta, float eps,
                           const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc, int64_t m, int64_t n,
                           int64_t k, int dtype, int epilogue, int plan_id, void* stream) {
  if (m < 0 || n < 0 || k <= 0) return fail(TJK_EINVAL, "tjk_gemm_ln: bad shape m=%lld n=%lld k=%lld",
                                            (long long)m, (long long)n, (long long)k);
  if (!gemm_ln_shape_ok(k, dtype))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_ln: k=%lld dtype=%d not supported (fp16 / bf16, k in {256, 512, 768, "
                "1024})", (long long)k, dtype);
  if (epilogue != TJK_EPI_BIAS && epilogue != TJK_EPI_BIAS_GELU)
    return fail(TJK_EINVAL, "tjk_gemm_ln: epilogue %d (bias or bias + GELU only)", epilogue);
  if (plan_id < -1 || plan_id >= kLnGemmPlans)
    return fail(TJK_EINVAL, "tjk_gemm_ln: plan %d out of range [-1,%d)", plan_id, kLnGemmPlans);
  if (m == 0 || n == 0) return TJK_OK;
  if (!res || !gamma || !beta || !w || !c) return fail(TJK_EINVAL, "tjk_gemm_ln: null pointer");
  if (m > INT32_MAX / 2 || n > INT32_MAX || n * ldw * dtype_size(dtype) >= kPastEnd)
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_ln: shape exceeds the 32-bit buffer range");
  if (n % 4) return fail(TJK_EUNSUPPORTED, "tjk_gemm_ln: n=%lld must be a multiple of 4", (long long)n);
  const int es = dtype_size(dtype);
  if (ld_res < k || ldw < k || ldc < n) return fail(TJK_EINVAL, "tjk_gemm_ln: leading dimension too small");
  if (ld_res % 4 || (ldw * es) % 16 || ldc % 4)
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_ln: rows must stay 16-byte aligned (ldc a multiple of 4)");
  if (((uintptr_t)res & 15) || ((uintptr_t)gamma & 15) || ((uintptr_t)beta & 15) || ((uintptr_t)w & 15) ||
      ((uintptr_t)c & (4 * es - 1)) || ((uintptr_t)bias & (4 * es - 1)))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_ln: misaligned pointer");
  int plan = plan_id;
  if (plan < 0) {
    // the widest column tile that still gives a launch of >= 128 workgroups
    const int64_t nrb = (m + kFfnRows - 1) / kFfnRows;
    plan = 0;
    for (int p = kLnGemmPlans - 1; p > 0; --p)
      if (nrb * ((n + kLnGemmBn[p] - 1) / kLnGemmBn[p]) >= 128) {
        plan = p;
        break;
      }
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == TJK_F16)
    return launch_gemm_ln<f16>(k, plan, res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, (int)m, (int)n,
                               epilogue, s);
  return launch_gemm_ln<bf16>(k, plan, res, ld_res, gamma, beta, eps, w, ldw, bias, c, ldc, (int)m, (int)n,
                              epilogue, s);
}
