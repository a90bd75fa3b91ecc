// MFMA GEMM with fused epilogues for the QKV, out-proj and FFN projections.
//
//   C[m, n] = epi( sum_k A[m, k] * W[n, k] + bias[n] )
//
// A is the [M, K] activation, W the nn.Linear [N, K] weight: both operands
// are K-contiguous, so both tiles are staged into LDS the same way and no
// transpose is needed anywhere.  This replaces torch.addmm at
// tjkernels/engine.py:245,247 and the addmm + gelu FFN fallback at
// tjkernels/kernels/__init__.py:88-89.
//
// Tiling (gfx950, wave64):
//   * a workgroup owns a BM x BN output tile; WM x WN waves each own a
//     (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks;
//   * K advances in BK steps (64 for 2-byte types = 128 B per row, 32 for
//     fp32); each step's A and W tiles live in LDS with a 16-byte row pad
//     (row pitch 144 B), which makes the ds_read_b128 fragment reads of 16
//     consecutive rows bank-conflict free;
//   * LDS is double-buffered: global loads for step k+1 are issued into
//     registers before the MFMAs of step k and written to the other buffer
//     after them, one barrier per step;
//   * the MFMA's first operand is the W fragment and the second the A
//     fragment, so the accumulator holds C^T: every lane owns four
//     consecutive n of one output row m, which turns the epilogue into 8- or
//     16-byte row stores and lets bias/GELU/residual be applied per register;
//   * workgroups are renumbered so that each XCD (the hardware deals
//     workgroup i to XCD i % 8) walks a contiguous range of a GROUP_M-grouped
//     tile order, keeping the A rows and W columns it reuses in its own L2.

#include "tjk_common.h"

namespace tjk {

constexpr int kGroupM = 8;

__device__ __forceinline__ float gelu_erf(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

// Bijection from hardware workgroup id to a tile order in which XCD x gets
// the contiguous range of ids [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
  const int per = nb / 8, rem = nb % 8;
  const int x = bid % 8, i = bid / 8;
  return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

template <typename T, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K) {
  constexpr int NT = WM * WN * 64;
  constexpr int VEC = 16 / sizeof(T);            // elements per 16-byte chunk
  constexpr int BK = 128 / sizeof(T);            // 128 bytes of K per row
  constexpr int CPR = BK / VEC;                  // chunks per row (8)
  constexpr int LDK = BK + VEC;                  // padded LDS row pitch (elements)
  constexpr int KS = BK / 16;                    // 16-deep MFMA steps per BK
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int CA = BM * CPR / NT, CW = BN * CPR / NT;
  static_assert(CA * NT == BM * CPR && CW * NT == BN * CPR, "tile/thread mismatch");
  static_assert(FM >= 1 && FN >= 1, "wave tile too small");

  __shared__ __attribute__((aligned(16))) T smem[2][(BM + BN) * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, hi = lane >> 5;

  // ---- tile coordinates: XCD-contiguous ranges of a grouped order
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int nb = tiles_m * tiles_n;
  const int t = xcd_remap(blockIdx.x, nb);
  const int group = t / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int pid_m = first_m + (t % (kGroupM * tiles_n)) % gsize;
  const int pid_n = (t % (kGroupM * tiles_n)) / gsize;
  const int m0 = pid_m * BM, n0 = pid_n * BN;

  // ---- global -> register staging
  uint4 ra[CA], rw[CW];
  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * NT, row = c / CPR, kc = c % CPR;
      const int gm = m0 + row, gk = k0 + kc * VEC;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const uint4*>(A + (int64_t)gm * lda + gk)
                                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      const int c = tid + i * NT, row = c / CPR, kc = c % CPR;
      const int gn = n0 + row, gk = k0 + kc * VEC;
      rw[i] = (gn < N && gk < K) ? *reinterpret_cast<const uint4*>(W + (int64_t)gn * ldw + gk)
                                 : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tiles = [&](int buf) {
    T* sA = smem[buf];
    T* sW = smem[buf] + BM * LDK;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * NT, row = c / CPR, kc = c % CPR;
      *reinterpret_cast<uint4*>(sA + row * LDK + kc * VEC) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      const int c = tid + i * NT, row = c / CPR, kc = c % CPR;
      *reinterpret_cast<uint4*>(sW + row * LDK + kc * VEC) = rw[i];
    }
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (K + BK - 1) / BK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles((kt + 1) * BK);
    const T* sA = smem[cur] + (wm * WTM + l32) * LDK + hi * 8;
    const T* sW = smem[cur] + BM * LDK + (wn * WTN + l32) * LDK + hi * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      typename Mfma<T>::frag af[FM], wf[FN];
#pragma unroll
      for (int j = 0; j < FM; ++j) af[j] = Mfma<T>::load(sA + j * 32 * LDK + ks * 16);
#pragma unroll
      for (int i = 0; i < FN; ++i) wf[i] = Mfma<T>::load(sW + i * 32 * LDK + ks * 16);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) Mfma<T>::mma(acc[i][j], wf[i], af[j]);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane owns C[m, n..n+3] for each (i, j, g)
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + wm * WTM + j * 32 + l32;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * WTN + i * 32 + g * 8 + hi * 4;
        if (n >= N) continue;
        float4 v = make_float4(acc[i][j][4 * g + 0], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                               acc[i][j][4 * g + 3]);
        if (bias != nullptr) {
          const float4 bv = Quad<T>::to(*reinterpret_cast<const typename Quad<T>::raw*>(bias + n));
          v.x += bv.x; v.y += bv.y; v.z += bv.z; v.w += bv.w;
        }
        if (EPI == TJK_EPI_BIAS_GELU) {
          v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
        }
        if (EPI == TJK_EPI_BIAS_RESIDUAL) {
          float4* r = reinterpret_cast<float4*>(static_cast<float*>(Cv) + (int64_t)m * ldc + n);
          float4 o = *r;
          o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
          *r = o;
        } else {
          T* c = static_cast<T*>(Cv) + (int64_t)m * ldc + n;
          *reinterpret_cast<typename Quad<T>::raw*>(c) = Quad<T>::from(v);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ plans

struct GemmPlan {
  int bm, bn, wm, wn;
};

// 2-byte types (bf16/fp16), BK = 64.
static const GemmPlan kPlans16[] = {
    {256, 256, 2, 2},  // 0: wave tile 128x128 (LDS 144 KB, 1 WG/CU)
    {256, 128, 2, 2},  // 1: wave tile 128x64
    {128, 256, 2, 2},  // 2: wave tile 64x128
    {128, 128, 2, 2},  // 3: wave tile 64x64 (2 WG/CU)
    {64, 64, 2, 2},    // 4: wave tile 32x32, small shapes
    {256, 256, 2, 4},  // 5: 8 waves, wave tile 128x64
};
// fp32, BK = 32.
static const GemmPlan kPlans32[] = {
    {128, 128, 2, 2},  // 0
    {64, 64, 2, 2},    // 1
};

template <typename T>
static const GemmPlan* plans(int* count) {
  if (sizeof(T) == 4) {
    *count = sizeof(kPlans32) / sizeof(kPlans32[0]);
    return kPlans32;
  }
  *count = sizeof(kPlans16) / sizeof(kPlans16[0]);
  return kPlans16;
}

// Picks the tile that minimises (number of full-chip rounds) x (tile cost),
// with a per-tile efficiency prior favouring the larger wave tiles.
template <typename T>
static int auto_plan(int64_t M, int64_t N) {
  int count;
  const GemmPlan* p = plans<T>(&count);
  static const double eff16[] = {1.0, 0.85, 0.85, 0.6, 0.3, 0.9};
  static const double eff32[] = {1.0, 0.6};
  const double* eff = sizeof(T) == 4 ? eff32 : eff16;
  int best = 0;
  double best_cost = 1e300;
  for (int i = 0; i < count; ++i) {
    const int64_t tiles = ((M + p[i].bm - 1) / p[i].bm) * ((N + p[i].bn - 1) / p[i].bn);
    const int64_t rounds = (tiles + 255) / 256;
    const double cost = (double)rounds * p[i].bm * p[i].bn / eff[i];
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = i;
    }
  }
  return best;
}

template <typename T, int BM, int BN, int WM, int WN>
static void launch_epi(int epi, const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                       void* c, int64_t ldc, int M, int N, int K, hipStream_t s) {
  const int nb = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  dim3 grid(nb), block(WM * WN * 64);
  switch (epi) {
    case TJK_EPI_BIAS:
      hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, TJK_EPI_BIAS>), grid, block, 0, s, (const T*)a, lda,
                         (const T*)w, ldw, (const T*)bias, c, ldc, M, N, K);
      break;
    case TJK_EPI_BIAS_GELU:
      hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, TJK_EPI_BIAS_GELU>), grid, block, 0, s, (const T*)a,
                         lda, (const T*)w, ldw, (const T*)bias, c, ldc, M, N, K);
      break;
    default:
      hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, TJK_EPI_BIAS_RESIDUAL>), grid, block, 0, s,
                         (const T*)a, lda, (const T*)w, ldw, (const T*)bias, c, ldc, M, N, K);
      break;
  }
}

template <typename T>
static int run_gemm(int plan, int epi, const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                    void* c, int64_t ldc, int M, int N, int K, hipStream_t s) {
  if constexpr (sizeof(T) == 4) {
    switch (plan) {
      case 0: launch_epi<T, 128, 128, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
      default: launch_epi<T, 64, 64, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
    }
  } else {
    switch (plan) {
      case 0: launch_epi<T, 256, 256, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
      case 1: launch_epi<T, 256, 128, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
      case 2: launch_epi<T, 128, 256, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
      case 3: launch_epi<T, 128, 128, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
      case 4: launch_epi<T, 64, 64, 2, 2>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
      default: launch_epi<T, 256, 256, 2, 4>(epi, a, lda, w, ldw, bias, c, ldc, M, N, K, s); break;
    }
  }
  return check_launch("tjk_gemm_bias");
}

template <typename T>
static int gemm_checked(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                        int64_t ldc, int64_t m, int64_t n, int64_t k, int epi, int plan, hipStream_t s) {
  int count;
  plans<T>(&count);
  if (plan < -1 || plan >= count) return fail(TJK_EINVAL, "tjk_gemm_bias: plan %d out of range [-1,%d)", plan, count);
  if (plan == -1) plan = auto_plan<T>(m, n);
  return run_gemm<T>(plan, epi, a, lda, w, ldw, bias, c, ldc, (int)m, (int)n, (int)k, s);
}

}  // namespace tjk

using namespace tjk;

extern "C" int tjk_gemm_plan_count(int dtype) {
  int count = 0;
  if (dtype == TJK_F32) plans<float>(&count);
  else if (dtype == TJK_F16 || dtype == TJK_BF16) plans<bf16>(&count);
  else return fail(TJK_EINVAL, "tjk_gemm_plan_count: bad dtype %d", dtype);
  return count;
}

extern "C" int tjk_gemm_plan_info(int dtype, int id, int* block_m, int* block_n, int* waves) {
  int count = 0;
  const GemmPlan* p;
  if (dtype == TJK_F32) p = plans<float>(&count);
  else if (dtype == TJK_F16 || dtype == TJK_BF16) p = plans<bf16>(&count);
  else return fail(TJK_EINVAL, "tjk_gemm_plan_info: bad dtype %d", dtype);
  if (id < 0 || id >= count) return fail(TJK_EINVAL, "tjk_gemm_plan_info: plan %d out of range", id);
  if (block_m) *block_m = p[id].bm;
  if (block_n) *block_n = p[id].bn;
  if (waves) *waves = p[id].wm * p[id].wn;
  return TJK_OK;
}

extern "C" int tjk_gemm_bias(const void* a, int64_t lda, const void* w, int64_t ldw,
                             const void* bias, void* c, int64_t ldc,
                             int64_t m, int64_t n, int64_t k,
                             int dtype, int epilogue, int plan_id, void* stream) {
  if (m < 0 || n < 0 || k < 0) return fail(TJK_EINVAL, "tjk_gemm_bias: negative shape");
  if (m == 0 || n == 0) return TJK_OK;
  if (!a || !w || !c) return fail(TJK_EINVAL, "tjk_gemm_bias: null pointer");
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: shape exceeds int32");
  if (epilogue < TJK_EPI_BIAS || epilogue > TJK_EPI_BIAS_RESIDUAL)
    return fail(TJK_EINVAL, "tjk_gemm_bias: bad epilogue %d", epilogue);
  if (dtype != TJK_F32 && dtype != TJK_F16 && dtype != TJK_BF16) return fail(TJK_EINVAL, "tjk_gemm_bias: bad dtype %d", dtype);
  const int es = dtype_size(dtype), vec = 16 / es;
  if (k % vec) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: k=%lld must be a multiple of %d", (long long)k, vec);
  if (n % 4) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: n=%lld must be a multiple of 4", (long long)n);
  if (lda < k || ldw < k || ldc < n) return fail(TJK_EINVAL, "tjk_gemm_bias: leading dimension too small");
  if (lda % vec || ldw % vec) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: lda/ldw must be multiples of %d", vec);
  if (ldc % 4) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: ldc must be a multiple of 4");
  const int cs = epilogue == TJK_EPI_BIAS_RESIDUAL ? 4 : es;
  if (((uintptr_t)a & 15) || ((uintptr_t)w & 15) || ((uintptr_t)c & (4 * cs - 1)) || ((uintptr_t)bias & (4 * es - 1)))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case TJK_F32: return gemm_checked<float>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, s);
    case TJK_F16: return gemm_checked<f16>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, s);
    default: return gemm_checked<bf16>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, s);
  }
}

extern "C" size_t tjk_ffn_workspace_bytes(int64_t tokens, int64_t f, int dtype) {
  if (tokens <= 0 || f <= 0) return 0;
  return (size_t)tokens * (size_t)f * (size_t)dtype_size(dtype);
}

extern "C" int tjk_ffn(const void* h, int64_t ldh, const void* w1, const void* b1,
                       const void* w2, const void* b2, void* out, int64_t ld_out,
                       void* workspace, int64_t tokens, int64_t d, int64_t f,
                       int dtype, int epilogue, int plan_ids, void* stream) {
  if (epilogue != TJK_EPI_BIAS && epilogue != TJK_EPI_BIAS_RESIDUAL)
    return fail(TJK_EINVAL, "tjk_ffn: epilogue must be TJK_EPI_BIAS or TJK_EPI_BIAS_RESIDUAL");
  if (tokens > 0 && !workspace) return fail(TJK_EINVAL, "tjk_ffn: null workspace");
  int p1 = (int8_t)(plan_ids & 0xff), p2 = (int8_t)((plan_ids >> 8) & 0xff);
  int rc = tjk_gemm_bias(h, ldh, w1, d, b1, workspace, f, tokens, f, d, dtype, TJK_EPI_BIAS_GELU, p1, stream);
  if (rc != TJK_OK) return rc;
  return tjk_gemm_bias(workspace, f, w2, f, b2, out, ld_out, tokens, d, f, dtype, epilogue, p2, stream);
}
