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


#include "gemm_tiles.h"

namespace tjk {

template <typename T, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K, ResSrc src) {
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
  int pid_m, pid_n;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, pid_m, pid_n);
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

  // The loop ends on a barrier, so the operand tiles are dead: reuse LDS.
  static_assert(NT / 64 * EpiStage<T, EPI, FN>::BYTES <= (int)sizeof(smem), "epilogue staging exceeds LDS");
  epilogue<T, EPI, FM, FN>(acc, bias, Cv, ldc, M, N, m0 + wm * WTM, n0 + wn * WTN, lane,
                           reinterpret_cast<char*>(&smem[0][0]) + wave * EpiStage<T, EPI, FN>::BYTES, NoPrefetch(),
                           nullptr, src);
}

template <typename T, int BM, int BN, int WM, int WN, int BKB, int STAGES, int EPI, int KSPLIT>
__global__ __launch_bounds__(WM * WN * KSPLIT * 64) void gemm_dtl_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K, ResSrc src) {
  typedef DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, KSPLIT> G;
  constexpr int NW = G::NW, FM = G::FM, FN = G::FN;
  __shared__ __attribute__((aligned(1024))) char smem[G::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, kg = (tid >> 6) / NW, wave = (tid >> 6) % NW;
  const int wm = wave / WN, wn = wave % WN;

  int pid_m, pid_n;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;

  // Bias and residual reads issued ahead of the operand DMAs, where their
  // registers fit beside the accumulators (plus ~144 for fragments and
  // addresses) without lowering the occupancy the LDS ring allows: their
  // round trip then overlaps the main loop instead of ending the launch,
  // which matters most for the short launches of a few hundred rows.  Wave
  // tiles above 4 blocks of 32 x 32 keep the bias loads in the epilogue and
  // prefetch only the residual, and only without a K split: there the
  // fragments already bring the wave close to its 256 architectural
  // registers (measured: 256 x 256 and 128 x 256 tiles spilled).
  constexpr int WG_PER_CU = 160 * 1024 / G::LDS;
  constexpr int WAVES_PER_SIMD = (WG_PER_CU * NW * KSPLIT + 3) / 4 > 1 ? (WG_PER_CU * NW * KSPLIT + 3) / 4 : 1;
  constexpr int BUDGET = 512 / WAVES_PER_SIMD - FM * FN * 16 - 144;
  constexpr int BIAS_REGS = FN * 4 * (int)sizeof(typename Quad<T>::raw) / 4;
  typedef ResPrefetch<FM, FN, T, EPI == kEpiResidualFrom> ResPre;
  constexpr int PRE_REGS = ResPre::REGS;
  constexpr bool SMALL = sizeof(T) == 2 && FM * FN <= 4;
  constexpr bool BIAS_PRE = SMALL && BIAS_REGS <= BUDGET;
  constexpr bool PREFETCH = epi_residual(EPI) && (KSPLIT == 1 || SMALL) &&
                            PRE_REGS + (BIAS_PRE ? BIAS_REGS : 0) <= BUDGET;
  typedef typename std::conditional<PREFETCH, ResPre, NoPrefetch>::type Pre;
  BiasRaw<T, FN> bpre;
  if constexpr (BIAS_PRE) bpre.load(bias, N, n0 + wn * G::WTN, lane);
  Pre pre;
  if constexpr (PREFETCH)
    pre.load(static_cast<const float*>(Cv), ldc, M, N, m0 + wm * G::WTM, n0 + wn * G::WTN, lane, src);

  f32x16 acc[FN][FM];
  zero_acc<T, FM, FN>(acc);
  dtl_accumulate<T, BM, BN, WM, WN, BKB, STAGES, KSPLIT>(smem, A, lda, W, ldw, M, N, m0, n0, 0, K / G::BK, acc);

  constexpr int ACCF = FN * FM * 16;                   // accumulator floats per lane
  constexpr int XCH = (KSPLIT - 1) * NW * ACCF * 64 * 4;  // exchange bytes
  static_assert(XCH + NW * EpiStage<T, EPI, FN>::BYTES <= G::LDS,
                "K-split exchange + epilogue staging exceed LDS");
  if constexpr (KSPLIT > 1) {
    // the groups' accumulators are summed (in group order) before the epilogue
    float* xch = reinterpret_cast<float*>(smem);
    if (kg > 0) {
      float* my = xch + (int64_t)((kg - 1) * NW + wave) * ACCF * 64;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) my[((i * FM + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int p = 1; p < KSPLIT; ++p) {
      const float* ot = xch + (int64_t)((p - 1) * NW + wave) * ACCF * 64;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += ot[((i * FM + j) * 16 + r) * 64 + lane];
    }
  }
  // batched residual reads except in the register-tight tiles (K-split
  // groups, more than 8 accumulator blocks), where they spilled
  constexpr int RB = KSPLIT == 1 && FM * FN <= 8 ? kResBatch : 0;
  epilogue<T, EPI, FM, FN, Pre, RB>(acc, bias, Cv, ldc, M, N, m0 + wm * G::WTM, n0 + wn * G::WTN, lane,
                                    smem + XCH + wave * EpiStage<T, EPI, FN>::BYTES, pre,
                                    BIAS_PRE ? &bpre : nullptr, src);
}


// ---------------------------------------------------- wave-specialized GEMM
//
// The direct-to-LDS main loop above issues its DMA from the waves that run
// the MFMAs.  When the per-CU DMA rate saturates (measured on MI355X:
// ~35-44 B/clk per CU for buffer_load ... lds), a wave stalls at the issue
// of its next DMA instruction and, issuing in order, its MFMAs stall with
// it: the loop then takes about the DMA-only time plus the MFMA-only time
// (1.5x the larger of the two at the packed C4 shapes).  Here the two jobs
// go to different waves of the workgroup:
//   * NW = WM x WN compute waves read fragments from the ring and issue the
//     MFMAs (the same fragment reads, MFMA order and epilogue as
//     gemm_dtl_kernel, so the results are bitwise those of the class-1
//     plans);
//   * L loader waves only issue the LDS DMA of K tile kt + STAGES - 1 and
//     wait for tile kt + 1 to land.
// One barrier per K tile (B_kt, before the compute waves' last 16-deep step
// of tile kt) orders them: after B_kt tile kt + 1 has landed and tile kt's
// slot is free.  A final barrier ends the ring before the epilogue reuses
// its LDS; the loader waves then exit.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int L, int EPI>
__global__ __launch_bounds__((WM * WN + L) * 64) void gemm_ws_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K, ResSrc src) {
  constexpr int BKB = 128;
  typedef DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, 1> G;
  constexpr int NW = G::NW, KS = G::KS, CPS = G::CPS, WTM = G::WTM, WTN = G::WTN, FM = G::FM, FN = G::FN;
  constexpr int STAGE = G::STAGE;
  constexpr int NINST = (BM + BN) / G::RPI;  // 1 KB DMA instructions per K tile
  constexpr int NL = NINST / L;              // per loader wave
  static_assert(NINST % L == 0 && BM % G::RPI == 0, "DMA rows split over the loader waves");
  static_assert(STAGES >= 2 && (STAGES - 2) * NL <= 63, "vmcnt range");
  constexpr int STG = NW * EpiStage<T, EPI, FN>::BYTES;
  constexpr int LDS = STAGES * STAGE > STG ? STAGES * STAGE : STG;
  __shared__ __attribute__((aligned(1024))) char smem[LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  int pid_m, pid_n;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;
  const int nk = K / G::BK;

  if (wave >= NW) {
    // ------------------------------------------------------------ loaders
    const int lw = wave - NW;
    const int64_t a_rows = min((int64_t)BM, (int64_t)(M - m0));
    const int64_t w_rows = min((int64_t)BN, (int64_t)(N - n0));
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A + (int64_t)m0 * lda), (short)0, (int)(a_rows * lda * (int64_t)sizeof(T)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(W + (int64_t)n0 * ldw), (short)0, (int)(w_rows * ldw * (int64_t)sizeof(T)), 0x00020000);
    // instruction q of loader lw fills rows (q L + lw) RPI .. +RPI-1 of the
    // stacked (A; W) tile; lane l lands at byte 16 l: row + l / CPR,
    // physical chunk l % CPR, so it fetches logical chunk (l % CPR) ^ swz(row)
    auto dma = [&](int t, int q) {
      char* sb = smem + (t % STAGES) * STAGE;
      const int base = (q * L + lw) * G::RPI;  // wave-uniform
      const uint32_t kb = (uint32_t)(t * BKB);
      if (base < BM) {
        const int r = base + lane / G::CPR;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsa, (lds_void*)(sb + base * BKB), 16,
            (uint32_t)(r * lda * (int64_t)sizeof(T)) + (uint32_t)(((lane % G::CPR) ^ swz<BKB>(r)) << 4) + kb, 0, 0, 0);
      } else {
        const int r = base - BM + lane / G::CPR;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsw, (lds_void*)(sb + base * BKB), 16,
            (uint32_t)(r * ldw * (int64_t)sizeof(T)) + (uint32_t)(((lane % G::CPR) ^ swz<BKB>(r)) << 4) + kb, 0, 0, 0);
      }
    };
    for (int t = 0; t < STAGES - 1 && t < nk; ++t) {
#pragma unroll
      for (int q = 0; q < NL; ++q) dma(t, q);
    }
    // tile 0 landed (the tiles issued after it may still be in flight)
    if (nk >= STAGES - 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((STAGES - 2) * NL) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // B_-1
    for (int k = 0; k < nk; ++k) {
      // tile k + STAGES - 1 into the slot tile k - 1 freed at B_{k-1};
      // then tile k + 1 landed before B_k
      const int t = k + STAGES - 1;
      if (t < nk) {
#pragma unroll
        for (int q = 0; q < NL; ++q) dma(t, q);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((STAGES - 2) * NL) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __builtin_amdgcn_s_barrier();  // B_k
    }
    __builtin_amdgcn_s_barrier();  // B_final
    return;
  }

  // ------------------------------------------------------------- compute
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, hi = lane >> 5;
  // The epilogue's bias and residual reads go out before the main loop where
  // the registers allow (accumulators, two fragment sets and address
  // registers counted against the per-wave share of the register file):
  // their round trip then overlaps the main loop.
  constexpr int WPS = (NW + L + 3) / 4;  // waves per SIMD (one workgroup per CU)
  constexpr int AVAIL = (512 / WPS) & ~7;
  // (the residual first: its read-modify-write is most of a residual
  // epilogue; 36 overhead registers, 44 with a ring whose slot count is not
  // a power of two, keeps every plan here free of spills)
  constexpr int USED = FM * FN * 16 + 2 * (FM + FN) * 4 + ((STAGES & (STAGES - 1)) ? 44 : 36);
  constexpr int BIAS_REGS = FN * 4 * (int)sizeof(typename Quad<T>::raw) / 4;
  typedef ResPrefetch<FM, FN, T, EPI == kEpiResidualFrom> ResPre;
  constexpr int PRE_REGS = ResPre::REGS;
  constexpr bool PREFETCH = epi_residual(EPI) && USED + PRE_REGS <= AVAIL;
  constexpr bool BIAS_PRE = USED + BIAS_REGS + (PREFETCH ? PRE_REGS : 0) <= AVAIL;
  typedef typename std::conditional<PREFETCH, ResPre, NoPrefetch>::type Pre;
  BiasRaw<T, FN> bpre;
  if constexpr (BIAS_PRE) bpre.load(bias, N, n0 + wn * WTN, lane);
  Pre pre;
  if constexpr (PREFETCH)
    pre.load(static_cast<const float*>(Cv), ldc, M, N, m0 + wm * WTM, n0 + wn * WTN, lane, src);
  const int sw = swz<BKB>(l32);
  typedef typename Mfma<T>::frag Frag;
  auto frag_at = [&](const char* rowbase, int ks) -> Frag {
    return *reinterpret_cast<const Frag*>(rowbase + (((CPS * ks + hi) ^ sw) << 4));
  };
  f32x16 acc[FN][FM];
  zero_acc<T, FM, FN>(acc);
  constexpr int NMF = FN * FM, NDS = FN + FM;
  constexpr int NSLOT = NMF > NDS ? NMF : NDS;
  Frag fa[2][FM], fw[2][FN];
  __builtin_amdgcn_s_barrier();  // B_-1: tile 0 landed
  __builtin_amdgcn_sched_barrier(0);
  {
    const char* sa = smem + (wm * WTM + l32) * BKB;
    const char* sw_ = smem + BM * BKB + (wn * WTN + l32) * BKB;
#pragma unroll
    for (int j = 0; j < FM; ++j) fa[0][j] = frag_at(sa + j * 32 * BKB, 0);
#pragma unroll
    for (int i = 0; i < FN; ++i) fw[0][i] = frag_at(sw_ + i * 32 * BKB, 0);
  }
  // Same schedule as dtl_accumulate: MFMA m of a step, then fragment read m
  // of the next step; the barrier precedes the last step of a tile, whose
  // fragments are in registers, and the next tile's first fragments are
  // read during the last step's MFMAs.  (The slot after the last tile is
  // read too; those fragments are never used.)
  for (int kt = 0; kt < nk; ++kt) {
    const char* st = smem + (kt % STAGES) * STAGE;
    const char* sa = st + (wm * WTM + l32) * BKB;
    const char* sw_ = st + BM * BKB + (wn * WTN + l32) * BKB;
    const char* nx = smem + ((kt + 1) % STAGES) * STAGE;
    const char* na = nx + (wm * WTM + l32) * BKB;
    const char* nw = nx + BM * BKB + (wn * WTN + l32) * BKB;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int b = ks & 1;
      const bool last = ks + 1 == KS;
      const char* ra = last ? na : sa;
      const char* rw = last ? nw : sw_;
      const int rks = last ? 0 : ks + 1;
      if (last) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // my reads of slot kt are done
        __builtin_amdgcn_s_barrier();                        // B_kt
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < NSLOT; ++m) {
        if (m < NMF) Mfma<T>::mma(acc[m / FM][m % FM], fw[b][m / FM], fa[b][m % FM]);
        if (m < FM) fa[b ^ 1][m] = frag_at(ra + m * 32 * BKB, rks);
        else if (m < NDS) fw[b ^ 1][m - FM] = frag_at(rw + (m - FM) * 32 * BKB, rks);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();  // B_final: every ring read done, every DMA landed
  // (the tiles that cannot take the prefetch are register-tight: their
  // residual pieces are read one by one, which spills nothing)
  epilogue<T, EPI, FM, FN, Pre, 0>(acc, bias, Cv, ldc, M, N, m0 + wm * WTM, n0 + wn * WTN, lane,
                                   smem + wave * EpiStage<T, EPI, FN>::BYTES, pre, BIAS_PRE ? &bpre : nullptr,
                                   src);
}

// ------------------------------------------------------------------ plans

enum { kStaged = 0, kDtl = 1, kWs = 2 };

struct GemmPlan {
  int kind, bm, bn, wm, wn, bkb, stages;
  double eff;       // prior used by auto_plan
  int ksplit = 1;   // K groups per workgroup (direct-to-LDS kernel)
  int loaders = 0;  // DMA-only waves (wave-specialized kernel)
};

// 2-byte types (bf16/fp16), BK = 64.  Measured on MI355X (bf16, C4/C5
// projections): the 64x64-wave-tile plan 7 is best while there are too few
// 256x256 tiles to fill two rounds of the 256 CUs, the 8-wave 256x256 plan 8
// beyond that.  (A 4-stage ring of 64-byte rows was tried and dropped: it
// measured 50% LDS bank-conflict cycles and no gain.)
static const GemmPlan kPlans16[] = {
    {kStaged, 256, 256, 2, 2, 128, 2, 0.50},  // 0
    {kStaged, 256, 128, 2, 2, 128, 2, 0.45},  // 1
    {kStaged, 128, 256, 2, 2, 128, 2, 0.45},  // 2
    {kStaged, 128, 128, 2, 2, 128, 2, 0.55},  // 3
    {kStaged, 64, 64, 2, 2, 128, 2, 0.40},    // 4  small shapes / K % 64 != 0
    {kStaged, 256, 256, 2, 4, 128, 2, 0.55},  // 5
    {kDtl, 256, 256, 2, 2, 128, 2, 0.85},     // 6  wave tile 128x128, 1 WG/CU
    {kDtl, 128, 128, 2, 2, 128, 2, 0.90},     // 7  wave tile 64x64, 2 WG/CU
    {kDtl, 256, 256, 2, 4, 128, 2, 1.00},     // 8  8 waves, wave tile 128x64
    {kDtl, 64, 64, 2, 2, 128, 2, 0.45},       // 9  small shapes
    {kDtl, 256, 128, 2, 2, 128, 2, 0.75},     // 10 wave tile 128x64
    {kDtl, 128, 256, 2, 2, 128, 2, 0.75},     // 11 wave tile 64x128
    {kDtl, 192, 128, 2, 2, 128, 2, 0.80},     // 12 wave tile 96x64, 1 WG/CU
    {kDtl, 192, 256, 2, 4, 128, 2, 0.90},     // 13 8 waves, wave tile 96x64
    {kDtl, 192, 384, 2, 4, 128, 2, 0.95},     // 14 8 waves, wave tile 96x96
    {kDtl, 96, 128, 1, 4, 128, 2, 0.60},      // 15 wave tile 96x32, small M
    // 16, 17: two K groups of 4 waves per workgroup (K tiles alternate between
    // the groups' LDS rings, partial sums added before the epilogue).  At the
    // packed C4 N=1024 projections they measured slower than plan 15 (FFN2
    // 60.4 vs 57.8 us): those GEMMs are partly bound by re-reading A from
    // the MALL, which splitting K does not change.
    {kDtl, 192, 128, 2, 2, 128, 2, 0.85, 2},  // 16 wave tile 96x64
    {kDtl, 128, 128, 2, 2, 128, 2, 0.85, 2},  // 17 wave tile 64x64
    // 18: a 4-slot ring (160 KB) with the spread DMA schedule, one workgroup
    // per CU.  Other deep rings measured (C4/C5 projections, residual reads
    // prefetched where registers allow) and dropped because a 2-slot plan
    // was faster on every shape: 256x256 8 waves and 4 waves with 64-byte
    // rows in 4 slots, 128x128 and 96x128 in 4 slots, 256x128 in 3 slots.
    {kDtl, 192, 128, 2, 2, 128, 4, 0.85},     // 18 wave tile 96x64, 160 KB
    // 19, 20: small tiles in deep rings (8 and 6 slots) for launches of a few
    // dozen workgroups with long K (C2's FFN2: 16 tiles, 32 K tiles each),
    // where a 2-slot ring leaves each step waiting out the DMA latency.
    {kDtl, 64, 64, 2, 2, 128, 8, 0.45},       // 19 wave tile 32x32, 128 KB
    {kDtl, 128, 64, 2, 2, 128, 6, 0.50},      // 20 wave tile 64x32, 144 KB
    // 21-23: the same small tiles with K split between 2 or 4 groups of 4
    // waves inside the workgroup (partials added through LDS), which
    // shortens the serial chain of K tiles a launch of a few dozen
    // workgroups waits out.
    {kDtl, 64, 64, 2, 2, 128, 2, 0.45, 4},    // 21 16 waves, 128 KB
    {kDtl, 64, 64, 2, 2, 128, 4, 0.45, 2},    // 22 8 waves, 128 KB
    {kDtl, 128, 64, 2, 2, 128, 3, 0.50, 2},   // 23 8 waves, 144 KB
    // 24, 25: 32-row tiles with K split between two groups of 2 / 1 waves,
    // for projections of a few hundred rows (C2: 128), whose tiles would
    // otherwise occupy a few dozen CUs each moving 128 KB of operands: at
    // 32 x 64 and 32 x 32 a launch spreads over 2x and 4x more CUs.
    {kDtl, 32, 64, 1, 2, 128, 4, 0.35, 2},    // 24 4 waves, 96 KB
    {kDtl, 32, 32, 1, 1, 128, 4, 0.30, 2},    // 25 2 waves, 64 KB
    // 26, 27: the 32-row tiles with K split between four groups, for a
    // launch of a few dozen tiles with long K (C2's FFN2, K = 2048): each
    // group streams every 4th K tile, so a workgroup has four rings' worth
    // of K tiles in flight and the serial chain is a quarter of K.
    {kDtl, 32, 32, 1, 1, 128, 4, 0.30, 4},    // 26 4 waves, 128 KB
    {kDtl, 32, 64, 1, 2, 128, 3, 0.35, 4},    // 27 8 waves, 144 KB
    // 28-32: wave-specialized (gemm_ws_kernel): WM x WN compute waves plus 4
    // DMA-only loader waves.  Measured on the packed C4 projections against
    // the best plan above: FFN2 (5430 x 1024 x 4096) 51 against 55.5 us,
    // out-proj 20.6 against 22.0 us, FFN1 59.7 against 60.2 us; QKV no gain.
    {kWs, 192, 128, 2, 2, 128, 4, 0.85, 1, 4},  // 28 wave tile 96x64, 160 KB
    {kWs, 192, 128, 2, 4, 128, 3, 0.85, 1, 4},  // 29 wave tile 96x32, 120 KB
    {kWs, 192, 128, 2, 4, 128, 4, 0.85, 1, 4},  // 30 wave tile 96x32, 160 KB
    {kWs, 192, 256, 2, 4, 128, 2, 0.85, 1, 4},  // 31 wave tile 96x64, 112 KB
    {kWs, 128, 256, 2, 4, 128, 3, 0.85, 1, 4},  // 32 wave tile 64x64, 144 KB
};
// fp32.
static const GemmPlan kPlans32[] = {
    {kStaged, 128, 128, 2, 2, 128, 2, 0.6},  // 0
    {kStaged, 64, 64, 2, 2, 128, 2, 0.4},    // 1
    {kDtl, 128, 128, 2, 2, 128, 2, 1.0},     // 2
    {kDtl, 256, 128, 2, 2, 128, 2, 1.0},     // 3
    {kDtl, 64, 64, 2, 2, 128, 2, 0.5},       // 4
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

static bool dtl_ok(const GemmPlan& p, int64_t k, int64_t lda, int64_t ldw, int es) {
  return k % (p.bkb / es) == 0 && (lda * es) % 16 == 0 && (ldw * es) % 16 == 0;
}

// Default tile choice.  For shapes the direct-to-LDS kernel takes, the
// measured rule above; otherwise (odd K, misaligned rows) the staged plan
// minimising (full-chip rounds of 256 workgroups) x (tile area / prior).
template <typename T>
static int auto_plan(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  int count;
  const GemmPlan* p = plans<T>(&count);
  if (sizeof(T) == 2 && dtl_ok(p[7], K, lda, ldw, sizeof(T))) {
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (t256 >= 512) return 8;
    if (t128 >= 128) return 7;
    return 9;
  }
  int best = 0;
  double best_cost = 1e300;
  for (int i = 0; i < count; ++i) {
    if (p[i].kind != kStaged && !dtl_ok(p[i], K, lda, ldw, sizeof(T))) continue;
    const int64_t tiles = ((M + p[i].bm - 1) / p[i].bm) * ((N + p[i].bn - 1) / p[i].bn);
    const int64_t rounds = (tiles + 255) / 256;
    const double cost = (double)rounds * p[i].bm * p[i].bn / p[i].eff;
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = i;
    }
  }
  return best;
}

// Kernel selection by plan kind through a specialised struct (the host stub
// of a kernel launched under `if constexpr` is not always emitted).
struct GemmArgs {
  const void* a; int64_t lda; const void* w; int64_t ldw; const void* bias; void* c; int64_t ldc;
  int M, N, K; hipStream_t s;
  ResSrc src;  // kEpiResidualFrom's residual source (unused by the other epilogues)
};
template <int KIND> struct Launcher;
template <> struct Launcher<kStaged> {
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    const dim3 grid(((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN));
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, EPI>), grid, dim3(WM * WN * 64), 0, g.s, (const T*)g.a,
                       g.lda, (const T*)g.w, g.ldw, (const T*)g.bias, g.c, g.ldc, g.M, g.N, g.K, g.src);
    return TJK_OK;
  }
};
template <int BKB, int STAGES, int KSPLIT = 1> struct DtlLauncher {
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    const dim3 grid(((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN));
    hipLaunchKernelGGL((gemm_dtl_kernel<T, BM, BN, WM, WN, BKB, STAGES, EPI, KSPLIT>), grid,
                       dim3(WM * WN * KSPLIT * 64), 0, g.s, (const T*)g.a, g.lda, (const T*)g.w, g.ldw,
                       (const T*)g.bias, g.c, g.ldc, g.M, g.N, g.K, g.src);
    return TJK_OK;
  }
};

template <typename L, typename T, int BM, int BN, int WM, int WN>
static int launch_epi(int epi, const GemmArgs& g) {
  switch (epi) {
    case TJK_EPI_BIAS: return L::template go<T, BM, BN, WM, WN, TJK_EPI_BIAS>(g);
    case TJK_EPI_BIAS_GELU: return L::template go<T, BM, BN, WM, WN, TJK_EPI_BIAS_GELU>(g);
    case kEpiResidualFrom: return L::template go<T, BM, BN, WM, WN, kEpiResidualFrom>(g);
    default: return L::template go<T, BM, BN, WM, WN, TJK_EPI_BIAS_RESIDUAL>(g);
  }
}

template <int STAGES, int L> struct WsLauncher {
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    const dim3 grid(((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN));
    hipLaunchKernelGGL((gemm_ws_kernel<T, BM, BN, WM, WN, STAGES, L, EPI>), grid, dim3((WM * WN + L) * 64), 0,
                       g.s, (const T*)g.a, g.lda, (const T*)g.w, g.ldw, (const T*)g.bias, g.c, g.ldc, g.M, g.N,
                       g.K, g.src);
    return TJK_OK;
  }
};

typedef Launcher<kStaged> St;
typedef DtlLauncher<128, 2> D2;
typedef DtlLauncher<128, 2, 2> D2K2;
typedef DtlLauncher<128, 2, 4> D2K4;
typedef DtlLauncher<128, 4, 2> D4K2;
typedef DtlLauncher<128, 3, 2> D3K2;
typedef DtlLauncher<128, 4, 4> D4K4;
typedef DtlLauncher<128, 3, 4> D3K4;
typedef DtlLauncher<128, 4> D4;
typedef DtlLauncher<128, 6> D6;
typedef DtlLauncher<128, 8> D8;
typedef WsLauncher<4, 4> W4;
typedef WsLauncher<3, 4> W3;
typedef WsLauncher<2, 4> W2;

template <typename T>
static int run_gemm(int plan, int epi, const GemmArgs& g) {
  int rc = TJK_OK;
#define TJK_GEMM_CASE(ID, L, BM, BN, WM, WN) \
  case ID: rc = launch_epi<L, T, BM, BN, WM, WN>(epi, g); break;
  if constexpr (sizeof(T) == 4) {
    switch (plan) {
      TJK_GEMM_CASE(0, St, 128, 128, 2, 2)
      TJK_GEMM_CASE(1, St, 64, 64, 2, 2)
      TJK_GEMM_CASE(2, D2, 128, 128, 2, 2)
      TJK_GEMM_CASE(3, D2, 256, 128, 2, 2)
      TJK_GEMM_CASE(4, D2, 64, 64, 2, 2)
    }
  } else {
    switch (plan) {
      TJK_GEMM_CASE(0, St, 256, 256, 2, 2)
      TJK_GEMM_CASE(1, St, 256, 128, 2, 2)
      TJK_GEMM_CASE(2, St, 128, 256, 2, 2)
      TJK_GEMM_CASE(3, St, 128, 128, 2, 2)
      TJK_GEMM_CASE(4, St, 64, 64, 2, 2)
      TJK_GEMM_CASE(5, St, 256, 256, 2, 4)
      TJK_GEMM_CASE(6, D2, 256, 256, 2, 2)
      TJK_GEMM_CASE(7, D2, 128, 128, 2, 2)
      TJK_GEMM_CASE(8, D2, 256, 256, 2, 4)
      TJK_GEMM_CASE(9, D2, 64, 64, 2, 2)
      TJK_GEMM_CASE(10, D2, 256, 128, 2, 2)
      TJK_GEMM_CASE(11, D2, 128, 256, 2, 2)
      TJK_GEMM_CASE(12, D2, 192, 128, 2, 2)
      TJK_GEMM_CASE(13, D2, 192, 256, 2, 4)
      TJK_GEMM_CASE(14, D2, 192, 384, 2, 4)
      TJK_GEMM_CASE(15, D2, 96, 128, 1, 4)
      TJK_GEMM_CASE(16, D2K2, 192, 128, 2, 2)
      TJK_GEMM_CASE(17, D2K2, 128, 128, 2, 2)
      TJK_GEMM_CASE(18, D4, 192, 128, 2, 2)
      TJK_GEMM_CASE(19, D8, 64, 64, 2, 2)
      TJK_GEMM_CASE(20, D6, 128, 64, 2, 2)
      TJK_GEMM_CASE(21, D2K4, 64, 64, 2, 2)
      TJK_GEMM_CASE(22, D4K2, 64, 64, 2, 2)
      TJK_GEMM_CASE(23, D3K2, 128, 64, 2, 2)
      TJK_GEMM_CASE(24, D4K2, 32, 64, 1, 2)
      TJK_GEMM_CASE(25, D4K2, 32, 32, 1, 1)
      TJK_GEMM_CASE(26, D4K4, 32, 32, 1, 1)
      TJK_GEMM_CASE(27, D3K4, 32, 64, 1, 2)
      TJK_GEMM_CASE(28, W4, 192, 128, 2, 2)
      TJK_GEMM_CASE(29, W3, 192, 128, 2, 4)
      TJK_GEMM_CASE(30, W4, 192, 128, 2, 4)
      TJK_GEMM_CASE(31, W2, 192, 256, 2, 4)
      TJK_GEMM_CASE(32, W3, 128, 256, 2, 4)
    }
  }
#undef TJK_GEMM_CASE
  if (rc != TJK_OK) return rc;
  return check_launch("tjk_gemm_bias");
}

template <typename T>
static int gemm_checked(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                        int64_t ldc, int64_t m, int64_t n, int64_t k, int epi, int plan, hipStream_t s,
                        const ResSrc& src = ResSrc{nullptr, 0, nullptr, 0, nullptr}) {
  int count;
  const GemmPlan* p = plans<T>(&count);
  if (plan < -1 || plan >= count) return fail(TJK_EINVAL, "tjk_gemm_bias: plan %d out of range [-1,%d)", plan, count);
  if (plan == -1) plan = auto_plan<T>(m, n, k, lda, ldw);
  if (p[plan].kind != kStaged && !dtl_ok(p[plan], k, lda, ldw, sizeof(T)))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: plan %d needs k %% %d == 0", plan, (int)(p[plan].bkb / sizeof(T)));
  if (p[plan].kind != kStaged && ((int64_t)p[plan].bm * lda * (int64_t)sizeof(T) > INT32_MAX ||
                                  (int64_t)p[plan].bn * ldw * (int64_t)sizeof(T) > INT32_MAX))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: leading dimension too large for plan %d", plan);
  const GemmArgs g{a, lda, w, ldw, bias, c, ldc, (int)m, (int)n, (int)k, s, src};
  return run_gemm<T>(plan, epi, g);
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

extern "C" int tjk_gemm_plan_info(int dtype, int id, int* block_m, int* block_n, int* waves, int* k_groups) {
  int count = 0;
  const GemmPlan* p;
  if (dtype == TJK_F32) p = plans<float>(&count);
  else if (dtype == TJK_F16 || dtype == TJK_BF16) p = plans<bf16>(&count);
  else return fail(TJK_EINVAL, "tjk_gemm_plan_info: bad dtype %d", dtype);
  if (id < 0 || id >= count) return fail(TJK_EINVAL, "tjk_gemm_plan_info: plan %d out of range", id);
  if (block_m) *block_m = p[id].bm;
  if (block_n) *block_n = p[id].bn;
  if (waves) *waves = p[id].wm * p[id].wn * p[id].ksplit + p[id].loaders;
  if (k_groups) *k_groups = p[id].ksplit;
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
    case TJK_F32:
      return gemm_checked<float>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, s);
    case TJK_F16:
      return gemm_checked<f16>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, s);
    default:
      return gemm_checked<bf16>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, s);
  }
}

extern "C" int tjk_gemm_bias_residual_from(const void* a, int64_t lda, const void* w, int64_t ldw,
                                           const void* bias, float* c, int64_t ldc,
                                           int64_t m, int64_t n, int64_t k,
                                           const void* x, int64_t ld_x, int64_t x_rows,
                                           const int32_t* rows, int* index_errors,
                                           int dtype, int plan_id, void* stream) {
  if (m < 0 || n < 0 || k < 0 || x_rows < 0) return fail(TJK_EINVAL, "tjk_gemm_bias_residual_from: negative shape");
  if (m == 0 || n == 0) return TJK_OK;
  // x is read only at rows below x_rows: it may be NULL when there are none
  if (!a || !w || !c || (!x && x_rows > 0)) return fail(TJK_EINVAL, "tjk_gemm_bias_residual_from: null pointer");
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias_residual_from: shape exceeds int32");
  if (dtype != TJK_F32 && dtype != TJK_F16 && dtype != TJK_BF16)
    return fail(TJK_EINVAL, "tjk_gemm_bias_residual_from: bad dtype %d", dtype);
  const int es = dtype_size(dtype), vec = 16 / es;
  if (k % vec) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias_residual_from: k=%lld must be a multiple of %d", (long long)k, vec);
  if (n % 4) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias_residual_from: n=%lld must be a multiple of 4", (long long)n);
  if (lda < k || ldw < k || ldc < n || ld_x < n)
    return fail(TJK_EINVAL, "tjk_gemm_bias_residual_from: leading dimension too small");
  if (lda % vec || ldw % vec) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias_residual_from: lda/ldw must be multiples of %d", vec);
  if (ldc % 4 || ld_x % 4) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias_residual_from: ldc/ld_x must be multiples of 4");
  if (((uintptr_t)a & 15) || ((uintptr_t)w & 15) || ((uintptr_t)c & 15) || ((uintptr_t)bias & (4 * es - 1)) ||
      ((uintptr_t)x & (4 * es - 1)) || ((uintptr_t)rows & 3) || ((uintptr_t)index_errors & 3))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias_residual_from: misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const ResSrc src{x, ld_x, rows, x_rows, index_errors};
  switch (dtype) {
    case TJK_F32:
      return gemm_checked<float>(a, lda, w, ldw, bias, c, ldc, m, n, k, kEpiResidualFrom, plan_id, s, src);
    case TJK_F16:
      return gemm_checked<f16>(a, lda, w, ldw, bias, c, ldc, m, n, k, kEpiResidualFrom, plan_id, s, src);
    default:
      return gemm_checked<bf16>(a, lda, w, ldw, bias, c, ldc, m, n, k, kEpiResidualFrom, plan_id, s, src);
  }
}
