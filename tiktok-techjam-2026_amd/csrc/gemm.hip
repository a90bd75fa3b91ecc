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

#include <type_traits>

#include "tjk_common.h"

namespace tjk {

constexpr int kGroupM = 8;

// GELU(v) = 0.5 v (1 + erf(v / sqrt 2)) with erf from Abramowitz & Stegun,
// Handbook of Mathematical Functions, eq. 7.1.26 (|error| <= 1.5e-7): for
// z >= 0, erf z = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2) with
// t = 1 / (1 + p z), and erf(-z) = -erf(z).  Branch-free (one reciprocal, one
// exp2) -- the library erff branches on |z| and measured ~35 VALU
// instructions per value with divergent lanes, most of the FFN1 epilogue.
__device__ __forceinline__ float gelu_erf(float v) {
  const float z = fabsf(v) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  poly *= t;
  const float e = __builtin_amdgcn_exp2f(-(z * z) * 1.4426950408889634f);  // exp(-z^2)
  const float erf_v = copysignf(fmaf(-poly, e, 1.0f), v);
  const float hv = 0.5f * v;
  return fmaf(hv, erf_v, hv);
}

// Bijection from hardware workgroup id to a tile order in which XCD x gets
// the contiguous range of ids [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
  const int per = nb / 8, rem = nb % 8;
  const int x = bid % 8, i = bid / 8;
  return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}


// Epilogue shared by both GEMM kernels.  The accumulators hold C^T blocks:
// for block (i, j), lane (l32, hi) owns output row m = mw + 32 j + l32 and,
// for g = 0..3, the four consecutive columns n = nw + 32 i + 8 g + 4 hi.
// Stored straight from that layout, every store instruction would scatter
// 8-16 byte pieces over 32 rows (32 L2 requests per instruction), which
// measured slower than the whole K=1024 main loop.  Instead each wave
// applies bias / GELU in registers, transposes one 32-row block at a time
// through a private LDS region (row pitch padded by one 16-byte piece) and
// writes whole row segments: 16 bytes per lane, WTN contiguous elements per
// row.  The residual epilogue stages fp32 and does its read-modify-write of
// the fp32 residual with the same row-contiguous pieces.
template <typename T, int EPI, int FN>
struct EpiStage {
  typedef typename std::conditional<EPI == TJK_EPI_BIAS_RESIDUAL, float, T>::type S;  // staged type
  static constexpr int WTN = FN * 32;
  static constexpr int SV = 16 / (int)sizeof(S);  // elements per 16-byte piece
  static constexpr int PITCH = WTN + SV;          // staged row pitch (elements)
  static constexpr int BYTES = 32 * PITCH * (int)sizeof(S);  // LDS bytes per wave
};

//
// `parts` (stream-K finishers only) supplies parts.n fp32 partial tiles of
// the same output tile, laid out like the accumulators; they are added in
// order to acc + bias before the activation.
// Cache-policy bits of buffer loads / stores on gfx950 (sc0 = 1, sc1 = 16):
// sc1 makes an access device-coherent, sc0 sc1 on a store writes through.
constexpr int kCpolSc1 = 16, kCpolSc0Sc1 = 17;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Access policy of the residual read-modify-write (TJK_EPI_BIAS_RESIDUAL):
// plain, or write-through stores / device-coherent loads for a residual
// tile that two workgroups update one after the other.
enum { kResPlain = 0, kResWriteThrough = 1, kResCoherentLoad = 2 };

struct NoParts {
  static constexpr int n = 0;
  __device__ f32x4 get(int, int) const { return f32x4{0.f, 0.f, 0.f, 0.f}; }
};

// The residual pieces (TJK_EPI_BIAS_RESIDUAL, plain policy) a wave's
// epilogue will update, read into registers before the main loop.  A launch
// whose tiles all run in one round otherwise starts every residual read at
// the same moment, after the last MFMA; read early, they overlap the main
// loop and the epilogue only writes.  Piece (j, it) is the one the
// epilogue's store loop handles for 32-row block j, iteration it.
struct NoPrefetch {
  static constexpr bool on = false;
  __device__ float4 get(int, int) const { return make_float4(0.f, 0.f, 0.f, 0.f); }
};
template <int FM, int FN>
struct ResPrefetch {
  static constexpr bool on = true;
  static constexpr int WTN = FN * 32, LPR = WTN / 4, NPC = 32 * LPR, NIT = (NPC + 63) / 64;
  float4 r[FM][NIT];
  __device__ __forceinline__ void load(const float* __restrict__ C, int64_t ldc, int M, int N, int mw, int nw,
                                       int lane) {
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int pc = lane + 64 * it;
        const int m = mw + 32 * j + pc / LPR, n = nw + (pc % LPR) * 4;
        r[j][it] = ((NPC % 64 == 0 || pc < NPC) && m < M && n < N)
                       ? *reinterpret_cast<const float4*>(C + (int64_t)m * ldc + n)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  }
  __device__ __forceinline__ float4 get(int j, int it) const { return r[j][it]; }
};

template <typename T, int EPI, int FM, int FN, typename Parts = NoParts, int RPOL = kResPlain,
          typename Pre = NoPrefetch>
__device__ __forceinline__ void epilogue(const f32x16 (&acc)[FN][FM], const T* __restrict__ bias,
                                         void* __restrict__ Cv, int64_t ldc, int M, int N, int mw, int nw,
                                         int lane, char* __restrict__ stage, const Parts& parts = Parts(),
                                         const Pre& pre = Pre()) {
  typedef EpiStage<T, EPI, FN> E;
  typedef typename E::S S;
  constexpr int LPR = E::WTN / E::SV;  // 16-byte pieces per staged row
  constexpr int NPC = 32 * LPR;        // pieces per 32-row block
  constexpr int NIT = (NPC + 63) / 64; // read instructions per block
  S* st = reinterpret_cast<S*>(stage);
  const int l32 = lane & 31, hi = lane >> 5;
  // 16-byte output pieces need a 16-byte aligned C and a leading dimension
  // that keeps every row 16-byte aligned; otherwise pieces go out as halves.
  const bool a16 = ((uintptr_t)Cv & 15) == 0 && (ldc % E::SV) == 0;

  float4 bv[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = nw + i * 32 + g * 8 + hi * 4;
      bv[i][g] = (bias != nullptr && n < N)
                     ? Quad<T>::to(*reinterpret_cast<const typename Quad<T>::raw*>(bias + n))
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }

#pragma unroll
  for (int j = 0; j < FM; ++j) {
    // this row block's partials, all loads of one partial in flight at once
    f32x4 ps[FN][4];
    if (parts.n > 0) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) ps[i][g] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int q = 0; q < parts.n; ++q) {
        f32x4 ld[FN][4];
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) ld[i][g] = parts.get(q, (i * FM + j) * 4 + g);
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) ps[i][g] += ld[i][g];
      }
    }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4 v = make_float4(acc[i][j][4 * g + 0] + bv[i][g].x, acc[i][j][4 * g + 1] + bv[i][g].y,
                               acc[i][j][4 * g + 2] + bv[i][g].z, acc[i][j][4 * g + 3] + bv[i][g].w);
        if (parts.n > 0) {
          v.x += ps[i][g][0]; v.y += ps[i][g][1]; v.z += ps[i][g][2]; v.w += ps[i][g][3];
        }
        if (EPI == TJK_EPI_BIAS_GELU) {
          v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
        }
        S* dst = st + l32 * E::PITCH + i * 32 + g * 8 + hi * 4;
        if constexpr (EPI == TJK_EPI_BIAS_RESIDUAL)
          *reinterpret_cast<float4*>(dst) = v;
        else
          *reinterpret_cast<typename Quad<T>::raw*>(dst) = Quad<T>::from(v);
      }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int pc = lane + 64 * it;  // piece index: row pc / LPR, piece pc % LPR
      if (NPC % 64 != 0 && pc >= NPC) break;
      const int rr = pc / LPR, cc = (pc % LPR) * E::SV;
      const int m = mw + 32 * j + rr, n = nw + cc;
      const uint4 piece = *reinterpret_cast<const uint4*>(st + rr * E::PITCH + cc);
      if (m < M && n < N) {
        if constexpr (EPI == TJK_EPI_BIAS_RESIDUAL) {
          // fp32 pieces never straddle N (N % 4 == 0)
          const float4 a = __builtin_bit_cast(float4, piece);
          if constexpr (RPOL == kResPlain) {
            float4* r = reinterpret_cast<float4*>(static_cast<float*>(Cv) + (int64_t)m * ldc + n);
            float4 o = Pre::on ? pre.get(j, it) : *r;
            o.x += a.x; o.y += a.y; o.z += a.z; o.w += a.w;
            *r = o;
          } else {  // the caller keeps M * ldc * 4 below 2^31
            const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(Cv, (short)0, 0x7fffffff, 0x00020000);
            const int off = (int)(((int64_t)m * ldc + n) * 4);
            float4 o = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, RPOL == kResCoherentLoad ? kCpolSc1 : 0));
            o.x += a.x; o.y += a.y; o.z += a.z; o.w += a.w;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), rc, off, 0,
                                                   RPOL == kResWriteThrough ? kCpolSc0Sc1 : 0);
          }
        } else {
          T* c = static_cast<T*>(Cv) + (int64_t)m * ldc + n;
          if (E::SV == 4 || (a16 && n + E::SV <= N)) {
            *reinterpret_cast<uint4*>(c) = piece;
          } else {  // 2-byte types: halves of 4 elements (N % 4 == 0)
            *reinterpret_cast<uint2*>(c) = make_uint2(piece.x, piece.y);
            if (n + 4 < N) *reinterpret_cast<uint2*>(c + 4) = make_uint2(piece.z, piece.w);
          }
        }
      }
    }
  }
}

// Tile coordinates of workgroup `bid`: XCD-contiguous ranges of a
// GROUP_M-grouped raster over (tiles_m x tiles_n).
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& pid_m, int& pid_n) {
  const int t = xcd_remap(bid, tiles_m * tiles_n);
  const int group = t / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  pid_m = first_m + (t % (kGroupM * tiles_n)) % gsize;
  pid_n = (t % (kGroupM * tiles_n)) / gsize;
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
                           reinterpret_cast<char*>(&smem[0][0]) + wave * EpiStage<T, EPI, FN>::BYTES);
}

// ------------------------------------------------------- direct-to-LDS GEMM
//
// Same math and epilogue as gemm_kernel, with the operand tiles moved by
// gfx950's LDS DMA (buffer_load_dwordx4 ... lds): each wave instruction
// copies 64 x 16 B straight from global memory into 1 KB of LDS, so tiles
// never pass through VGPRs.  Rows beyond M (or N) fall outside the buffer
// descriptor's range and arrive as zeros, which removes every bounds branch
// from the main loop.
//
// LDS holds STAGES tiles in a ring; a tile row is BKB bytes of K (64 or
// 128) with no padding.  The 16-byte chunk c of row r is stored at chunk
// c ^ swz(r), which spreads the ds_read_b128 fragment reads of 16
// consecutive rows over all banks (for 32- and 64-bank LDS alike).
//
// Pipeline, one barrier per tile, placed before the tile's last 16-deep
// step: by then every fragment of tile k is in registers, so after the
// barrier (which also certifies that tile k+1 has landed) a wave issues the
// DMA of tile k+STAGES into tile k's slot and reads tile k+1's first
// fragments while the last step's MFMAs run.  Every DMA has STAGES-1 tiles
// of MFMA work to land, and no wave waits for LDS right after the barrier.
// With a ring of three or more slots the DMA of tile k-1+STAGES (into the
// slot tile k-1 freed at the previous barrier) is instead spread over the
// MFMAs of tile k's steps before the last: the vector memory unit then gets
// a few instructions per step rather than a burst after each barrier, and
// every DMA still has at least one tile of MFMA work to land.  Measured on
// MI355X (wall-clock probes of one launch, bias epilogue): 192x128 tiles in
// a 4-slot ring (160 KB) run the C4 FFN2 main loop (5430x1024x4096) at 67%
// of the clock-limited MFMA rate, against 62% for 3 slots with the spread
// schedule, 55% for 3 slots issuing after the barrier and 52% for 2 slots.
// Removing the W operand's LDS reads did not change the 2-slot loop's
// speed; removing its DMA made it 25% faster: the loops are bound by the
// DMA traffic per CU, not by LDS reads.
// The DMA is issued on every iteration, past the end pointed outside the
// buffer range (it moves nothing), which keeps the body one basic block;
// scheduling directives interleave the MFMAs with the next step's ds_reads.
// Requires K % (BKB / sizeof(T)) == 0 and 16-byte aligned rows.

template <int BKB> __device__ __forceinline__ int swz(int r);
template <> __device__ __forceinline__ int swz<128>(int r) { return (r & 7) ^ ((r >> 3) & 1); }
template <> __device__ __forceinline__ int swz<64>(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

typedef __attribute__((address_space(3))) void lds_void;

// Byte offset that lies beyond any buffer descriptor range used here.
constexpr int kPastEnd = 0x7fff0000;

// Tile geometry shared by the direct-to-LDS kernels.
template <typename T, int BM, int BN, int WM, int WN, int BKB, int STAGES, int KSPLIT>
struct DtlGeom {
  static constexpr int NW = WM * WN;
  static constexpr int BK = BKB / sizeof(T);          // K elements per tile
  static constexpr int CPR = BKB / 16;                // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;                // rows per DMA instruction
  static constexpr int KS = BK / 16;                  // 16-deep MFMA steps per tile
  static constexpr int CPS = sizeof(T) == 2 ? 2 : 4;  // chunks per 16-deep step
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int STAGE = (BM + BN) * BKB;       // bytes per LDS stage
  static constexpr int DA = BM / (RPI * NW), DW = BN / (RPI * NW);
  static constexpr int NDMA = DA + DW;                // DMA instructions per wave per tile
  static constexpr int LDS = KSPLIT * STAGES * STAGE; // ring bytes
  static_assert(DA * RPI * NW == BM && DW * RPI * NW == BN, "tile rows must split over the waves");
  static_assert(STAGES >= 2 && (STAGES - 1) * NDMA <= 63, "vmcnt range");
  static_assert(KS % 2 == 0, "fragment double buffer alternates per 16-deep step");
};

// acc += A[m0 : m0+BM, K tiles kt0..kt1) * W[n0 : n0+BN, same]^T for this
// wave's sub-tile (K-split group kg takes K tiles kt0 + kg, kt0 + kg +
// KSPLIT, ...).  On return every DMA has landed and the workgroup has met at
// a barrier, so the LDS ring may be reused.  (smem is deliberately not
// __restrict__: with it the compiler stops telling the LDS DMA writes and
// the fragment reads of different ring slots apart and waits for every DMA
// before each ds_read.)
template <typename T, int BM, int BN, int WM, int WN, int BKB, int STAGES, int KSPLIT>
__device__ __forceinline__ void dtl_accumulate(
    char* smem, const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    int M, int N, int m0, int n0, int kt0, int kt1,
    f32x16 (&acc)[DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, KSPLIT>::FN][DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, KSPLIT>::FM]) {
  typedef DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, KSPLIT> G;
  constexpr int NW = G::NW, KS = G::KS, CPR = G::CPR, RPI = G::RPI, CPS = G::CPS;
  constexpr int WTM = G::WTM, WTN = G::WTN, FM = G::FM, FN = G::FN, STAGE = G::STAGE;
  constexpr int DA = G::DA, NDMA = G::NDMA;
  constexpr int DW = G::DW;

  // K split inside the workgroup: KSPLIT groups of WM x WN waves, group kg
  // streaming its K tiles through its own LDS ring.  The thread id passes an
  // empty asm so that, inside a persistent kernel's tile loop, nothing
  // derived from it is hoisted out of that loop (which keeps the per-lane
  // DMA and fragment addresses of every call live at once).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, kg = (tid >> 6) / NW, wave = (tid >> 6) % NW;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, hi = lane >> 5;
  char* const gsm = smem + kg * (STAGES * STAGE);

  // Buffer descriptors over this tile's rows; reads past row M (N) return 0.
  const int64_t a_rows = min((int64_t)BM, (int64_t)(M - m0));
  const int64_t w_rows = min((int64_t)BN, (int64_t)(N - n0));
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + (int64_t)m0 * lda), (short)0, (int)(a_rows * lda * (int64_t)sizeof(T)), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (int64_t)n0 * ldw), (short)0, (int)(w_rows * ldw * (int64_t)sizeof(T)), 0x00020000);

  // DMA instruction i of this wave fills LDS rows (i*NW + wave)*RPI + 0..RPI-1;
  // lane l lands at byte 16*l of that 1 KB: row +l/CPR, physical chunk l%CPR,
  // so it fetches logical chunk (l%CPR) ^ swz(row).
  uint32_t voff_a[DA], voff_w[DW];
#pragma unroll
  for (int i = 0; i < DA; ++i) {
    const int r = (i * NW + wave) * RPI + lane / CPR;
    voff_a[i] = (uint32_t)(r * lda * (int64_t)sizeof(T)) + (uint32_t)(((lane % CPR) ^ swz<BKB>(r)) << 4);
  }
#pragma unroll
  for (int i = 0; i < DW; ++i) {
    const int r = (i * NW + wave) * RPI + lane / CPR;
    voff_w[i] = (uint32_t)(r * ldw * (int64_t)sizeof(T)) + (uint32_t)(((lane % CPR) ^ swz<BKB>(r)) << 4);
  }
  const int nit = (kt1 - kt0 + KSPLIT - 1) / KSPLIT;  // ring steps per group
  // DMA instruction q (q < DA: A rows, else W rows) of this group's step it
  // into its slot; past the segment it points outside the range and moves
  // nothing.
  auto dma = [&](int it, int q) {
    char* sb = gsm + (it % STAGES) * STAGE;
    const int kt = kt0 + it * KSPLIT + kg;
    const uint32_t kb = kt < kt1 ? (uint32_t)(kt * BKB) : (uint32_t)kPastEnd;
    if (q < DA)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_void*)(sb + (q * NW + wave) * 1024), 16,
                                               (uint32_t)(voff_a[q] + kb), 0, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_void*)(sb + BM * BKB + ((q - DA) * NW + wave) * 1024),
                                               16, (uint32_t)(voff_w[q - DA] + kb), 0, 0, 0);
  };

  // Fragment reads: row (base + l32), logical chunk c at physical c ^ swz(l32).
  const int sw = swz<BKB>(l32);
  auto frag_at = [&](const char* rowbase, int ks) -> typename Mfma<T>::frag {
    if constexpr (sizeof(T) == 2) {
      return *reinterpret_cast<const typename Mfma<T>::frag*>(rowbase + (((CPS * ks + hi) ^ sw) << 4));
    } else {
      const float4 lo = *reinterpret_cast<const float4*>(rowbase + (((CPS * ks + 2 * hi) ^ sw) << 4));
      const float4 up = *reinterpret_cast<const float4*>(rowbase + (((CPS * ks + 2 * hi + 1) ^ sw) << 4));
      typename Mfma<T>::frag f;
      f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
      f[4] = up.x; f[5] = up.y; f[6] = up.z; f[7] = up.w;
      return f;
    }
  };

  // Prologue: tiles 0 .. STAGES-1 in flight (STAGES-2 with the spread
  // schedule, whose loop issues tile kt-1+STAGES during tile kt); tile 0
  // landed everywhere.
  constexpr bool SPREAD = STAGES >= 3;
  constexpr int PRE = SPREAD ? STAGES - 1 : STAGES;
#pragma unroll
  for (int t = 0; t < PRE; ++t)
#pragma unroll
    for (int q = 0; q < NDMA; ++q) dma(t, q);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PRE - 1) * NDMA) : "memory");
  asm volatile("s_barrier" ::: "memory");
  constexpr int NMF = FN * FM, NDS = FN + FM;  // MFMAs and fragment reads per step
  constexpr int NSLOT = NMF > NDS ? NMF : NDS;
  typename Mfma<T>::frag fa[2][FM], fw[2][FN];
  {
    const char* sa = gsm + (wm * WTM + l32) * BKB;
    const char* sw_ = gsm + BM * BKB + (wn * WTN + l32) * BKB;
#pragma unroll
    for (int j = 0; j < FM; ++j) fa[0][j] = frag_at(sa + j * 32 * BKB, 0);
#pragma unroll
    for (int i = 0; i < FN; ++i) fw[0][i] = frag_at(sw_ + i * 32 * BKB, 0);
  }
  // The loop body is emitted in source order (scheduling fences between the
  // pieces): MFMA m of a step is followed by fragment read m of the next
  // step (m < FM + FN), and after the barrier by DMA instructions, so the
  // LDS reads and DMA issues hide under the MFMAs of the step before the
  // one that needs them.
  for (int kt = 0; kt < nit; ++kt) {
    const char* st = gsm + (kt % STAGES) * STAGE;
    const char* sa = st + (wm * WTM + l32) * BKB;
    const char* sw_ = st + BM * BKB + (wn * WTN + l32) * BKB;
    const char* nx = gsm + ((kt + 1) % STAGES) * STAGE;
    const char* na = nx + (wm * WTM + l32) * BKB;
    const char* nw = nx + BM * BKB + (wn * WTN + l32) * BKB;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int b = ks & 1;
      const bool last = ks + 1 == KS;
      // fragments of the next step: this tile's step ks+1, or after the
      // barrier the next tile's step 0
      const char* ra = last ? na : sa;
      const char* rw = last ? nw : sw_;
      const int rks = last ? 0 : ks + 1;
      if (last) {
        // Before the last step's MFMAs (its fragments are in registers): my
        // reads of this slot are complete and my DMAs of step kt+1 have
        // landed, then everyone's.  The slot is then free for step
        // kt+STAGES.  Inline asm with a memory clobber keeps the compiler
        // from moving LDS accesses across either instruction.
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((STAGES - 2) * NDMA) : "memory");  // tile kt+1 landed
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < NSLOT; ++m) {
        if (m < NMF) Mfma<T>::mma(acc[m / FM][m % FM], fw[b][m / FM], fa[b][m % FM]);
        if (m < FM) fa[b ^ 1][m] = frag_at(ra + m * 32 * BKB, rks);
        else if (m < NDS) fw[b ^ 1][m - FM] = frag_at(rw + (m - FM) * 32 * BKB, rks);
        if constexpr (SPREAD) {
          // DMA instructions of tile kt-1+STAGES over slots 0 .. (KS-1)*NSLOT-1
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

  // Reuse LDS once every DMA (including the ones issued past the last
  // tile) has landed and every wave is done reading.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

template <typename T, int FM, int FN>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[FN][FM]) {
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

template <typename T, int BM, int BN, int WM, int WN, int BKB, int STAGES, int EPI, int KSPLIT>
__global__ __launch_bounds__(WM * WN * KSPLIT * 64) void gemm_dtl_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K) {
  typedef DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, KSPLIT> G;
  constexpr int NW = G::NW, FM = G::FM, FN = G::FN;
  __shared__ __attribute__((aligned(1024))) char smem[G::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, kg = (tid >> 6) / NW, wave = (tid >> 6) % NW;
  const int wm = wave / WN, wn = wave % WN;

  int pid_m, pid_n;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;

  // Residual reads issued ahead of the operand DMAs, where their registers
  // fit beside the accumulators (plus ~144 for fragments and addresses)
  // without lowering the occupancy the LDS ring allows.
  constexpr int WAVES_PER_SIMD = (NW * KSPLIT / 4) * (160 * 1024 / G::LDS);
  constexpr int PRE_REGS = FM * ResPrefetch<FM, FN>::NIT * 4;
  constexpr bool PREFETCH = EPI == TJK_EPI_BIAS_RESIDUAL && KSPLIT == 1 &&
                            FM * FN * 16 + PRE_REGS + 144 <= 512 / WAVES_PER_SIMD;
  typedef typename std::conditional<PREFETCH, ResPrefetch<FM, FN>, NoPrefetch>::type Pre;
  Pre pre;
  if constexpr (PREFETCH)
    pre.load(static_cast<const float*>(Cv), ldc, M, N, m0 + wm * G::WTM, n0 + wn * G::WTN, lane);

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
  epilogue<T, EPI, FM, FN, NoParts, kResPlain, Pre>(acc, bias, Cv, ldc, M, N, m0 + wm * G::WTM,
                                                    n0 + wn * G::WTN, lane,
                                                    smem + XCH + wave * EpiStage<T, EPI, FN>::BYTES, NoParts(), pre);
}

// ------------------------------------------------------------ stream-K GEMM
//
// Persistent variant for shapes whose tile count fills the CUs badly.  The
// grid is one resident wave of G workgroups (CUs x occupancy).  The tiles of
// the GROUP_M raster are split in two parts:
//   * the first dp_tiles are whole tiles dealt round-robin over the grid;
//   * the rest are cut into units of one K tile (BK deep), and the units
//     (tile-major) are divided into G contiguous ranges of equal length.
// A workgroup walks its range from the end backwards, one segment (the
// part of its range inside one tile) at a time:
//   * a segment that is a whole tile goes straight to the epilogue;
//   * a segment that ends before the tile's last K tile (always the first
//     one a workgroup meets) writes its fp32 partial accumulators through to
//     memory in its workspace slot, waits for the stores, and raises its
//     flag;
//   * the segment that holds the tile's last K tile (always the last one a
//     workgroup meets) polls the flags of the lower workgroups that hold the
//     rest of the tile, and its epilogue adds their partials (device-coherent
//     loads, nearest first) before clearing their flags.
// Producers never wait, and a finisher only waits for workgroups with lower
// logical ids that publish before doing anything else, so every wait ends
// while the grid is resident; each wait is still bounded (kSkSpinLimit
// polls) and a timeout is counted in the workspace's error word instead of
// hanging.  Results are deterministic for a given grid size: the partition
// and the summation order depend only on (M, N, K, G).  Flags are left at
// zero for the next call.  Calls sharing one workspace must not overlap.
//
// Measured on MI355X at the packed C4 projections these plans are slower
// than the best direct-to-LDS tile (e.g. FFN2 5430x1024x4096: 67.7 us vs
// 55 us): a CU moves ~50 GB/s, so publishing a 192-256 KB partial costs
// 3-5 us and a finisher's epilogue with two partials 7-18 us, which eats
// the quantization gain.  They win where the data-parallel rounds dominate
// (8192^3: 1337 TFLOP/s vs 1300 for plan 8).

constexpr int kMaxSkGrid = 2048;
constexpr int kSkSpinLimit = 1 << 22;

struct SkParams {
  int tiles_m, tiles_n;
  int dp_tiles;   // whole tiles dealt round-robin over the grid
  int sk_units;   // K-tile units of the remaining tiles
  int nk;         // K tiles per output tile
};

// Workspace: int flags[kMaxSkGrid], int error, the split-K flags
// (kK2FlagOffset .. kSkHeader), then one BM x BN fp32 partial per workgroup.
constexpr size_t kSkHeader = 32768;
constexpr int kK2FlagOffset = 12288;
constexpr int kMaxK2Tiles = (int)(kSkHeader - kK2FlagOffset) / 4;
static_assert((kMaxSkGrid + 1) * 4 <= kK2FlagOffset, "flag area");

__device__ __forceinline__ void raster_coords(int t, int tiles_m, int tiles_n, int& pid_m, int& pid_n) {
  const int group = t / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  pid_m = first_m + (t % (kGroupM * tiles_n)) % gsize;
  pid_n = (t % (kGroupM * tiles_n)) / gsize;
}

template <typename T, int BM, int BN, int WM, int WN, int BKB, int STAGES, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_sk_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, SkParams p,
    char* __restrict__ workspace) {
  typedef DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, 1> G;
  constexpr int NW = G::NW, FM = G::FM, FN = G::FN;
  static_assert(NW * EpiStage<T, EPI, FN>::BYTES <= G::LDS, "epilogue staging exceeds LDS");
  __shared__ __attribute__((aligned(1024))) char smem[G::LDS];

  const int tid = threadIdx.x;
  // Logical workgroup id: XCD-contiguous (the hardware deals workgroup ids
  // round-robin over the 8 XCDs), so each XCD walks a contiguous range of
  // units -- neighbouring tiles that share operand rows and columns in its
  // L2 -- and a producer / finisher pair is mostly on one XCD.  Correctness
  // does not depend on the placement: partials move write-through and are
  // read device-coherent.
  const int grid = gridDim.x, c = xcd_remap(blockIdx.x, grid);
  int* const flags = reinterpret_cast<int*>(workspace);
  float* const partials = reinterpret_cast<float*>(workspace + kSkHeader);
  constexpr int TILE_F4 = BM * BN / 4;  // float4s per partial
  // this wave's part of a partial: [i][j][r / 4][lane] float4s
  // Partials move through the device-coherent path instead of whole-cache
  // maintenance: stores write through to memory (sc0 sc1), loads are
  // device-coherent (sc1), so no L2 writeback or invalidate is needed
  // around the flags (a cache-wide invalidate per finisher would evict the
  // operand tiles of every workgroup on its XCD).  Byte offset of float4
  // `idx` of this wave / lane in owner's slot:
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(partials, (short)0, 0x7fffffff, 0x00020000);
  auto part_off = [&](int owner, int wave, int lane) {
    return (owner * TILE_F4 + wave * (FN * FM * 4 * 64) + lane) * 16;
  };
  struct SkParts {
    __amdgpu_buffer_rsrc_t r;
    int base, stride, n;
    __device__ f32x4 get(int q, int idx) const {
      return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, base + q * stride + idx * 64 * 16,
                                                                             0, kCpolSc1));
    }
  };

  // Work items, one call site each for the main loop and the epilogue (so
  // the accumulators stay in registers): first this workgroup's
  // data-parallel tiles, then its stream-K segments from the range end
  // backwards.
  const int dp_first = c;
  const int n_dp = dp_first < p.dp_tiles ? (p.dp_tiles - dp_first + grid - 1) / grid : 0;
  const int base = p.sk_units / grid, rem = p.sk_units % grid;
  const int u_begin = c * base + min(c, rem);
  const int u_end = u_begin + base + (c < rem ? 1 : 0);
  const int big = rem * (base + 1);  // units held by the workgroups with base + 1 of them

  f32x16 acc[FN][FM];
  int u = u_end;
  for (int item = 0;; ++item) {
    int t, kt0, kt1, lo = 0, first_owner = c;
    if (item < n_dp) {
      t = dp_first + item * grid;
      kt0 = 0;
      kt1 = p.nk;
    } else {
      if (u <= u_begin) break;
      const int tl = (u - 1) / p.nk, tu0 = tl * p.nk;
      lo = max(u_begin, tu0);
      t = p.dp_tiles + tl;
      kt0 = lo - tu0;
      kt1 = u - tu0;
      // owner of the tile's first unit: the lowest workgroup holding a part
      first_owner = tu0 < big ? tu0 / (base + 1) : rem + (tu0 - big) / base;
      u = lo;
    }
    if (item > 0) __syncthreads();  // the previous epilogue's staging reads are done
    int ltid = threadIdx.x;          // per-item copy, not hoisted (see dtl_accumulate)
    asm volatile("" : "+v"(ltid));
    const int lane = ltid & 63, wave = ltid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    int pid_m, pid_n;
    raster_coords(t, p.tiles_m, p.tiles_n, pid_m, pid_n);
    zero_acc<T, FM, FN>(acc);
    dtl_accumulate<T, BM, BN, WM, WN, BKB, STAGES, 1>(smem, A, lda, W, ldw, M, N, pid_m * BM, pid_n * BN, kt0,
                                                      kt1, acc);
    if (kt1 < p.nk) {
      // producer: publish the partial
      const int dst = part_off(c, wave, lane);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * r4 + e];
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                   dst + ((i * FM + j) * 4 + r4) * 64 * 16, 0, kCpolSc0Sc1);
          }
      // every wave's write-through stores have completed, then the flag
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) __hip_atomic_store(&flags[c], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    // Finisher (holds the tile's last K tile but not its first): the lower
    // workgroups holding the rest published their partials as their first
    // item, so by now the waits are normally over.  The epilogue adds the
    // partials nearest first.
    // The polls are relaxed device-coherent loads; the partials are then
    // read with device-coherent loads as well.
    const int nparts = (kt0 > 0) ? c - first_owner : 0;
    for (int o = c - 1; o >= c - nparts; --o) {
      int spins = 0;
      while (__hip_atomic_load(&flags[o], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        if (++spins > kSkSpinLimit) {
          if (tid == 0) __hip_atomic_fetch_add(&flags[kMaxSkGrid], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    const SkParts parts{prs, nparts > 0 ? part_off(c - 1, wave, lane) : 0, -TILE_F4 * 16, nparts};
    epilogue<T, EPI, FM, FN>(acc, bias, Cv, ldc, M, N, pid_m * BM + wm * G::WTM, pid_n * BN + wn * G::WTN, lane,
                             smem + wave * EpiStage<T, EPI, FN>::BYTES, parts);
    if (nparts > 0) {
      __syncthreads();  // every wave has read the partials
      for (int q = tid; q < nparts; q += WM * WN * 64)
        __hip_atomic_store(&flags[c - 1 - q], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------- split-K residual GEMM
//
// For the residual projections (out-proj, FFN2: N = 1024) a tile size that
// keeps the LDS traffic per MFMA low (192x128) gives only ~232 tiles for
// 256 CUs, one 4-wave workgroup each, which leaves the MFMA pipes waiting on
// LDS latency.  Here every tile is computed by two workgroups, one per half
// of K, all resident at once (2 per CU): the first half adds its partial
// and the bias into the fp32 residual with write-through stores and raises
// the tile's flag; the second half waits for the flag (bounded polls), then
// adds its partial reading the residual device-coherently, and clears the
// flag.  out = (out + acc_lo + bias) + acc_hi, in that order every time, so
// results are deterministic.  The second half's workgroups have the higher
// ids, so they are dispatched after the ones they wait for.
template <typename T, int BM, int BN, int WM, int WN, int BKB, int STAGES>
__global__ __launch_bounds__(WM * WN * 64) void gemm_k2_residual_kernel(
    const T* __restrict__ A, int64_t lda, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, float* __restrict__ C, int64_t ldc, int M, int N, int K,
    int* __restrict__ flags) {
  typedef DtlGeom<T, BM, BN, WM, WN, BKB, STAGES, 1> G;
  constexpr int FM = G::FM, FN = G::FN;
  constexpr int EPI = TJK_EPI_BIAS_RESIDUAL;
  static_assert(G::NW * EpiStage<T, EPI, FN>::BYTES <= G::LDS, "epilogue staging exceeds LDS");
  __shared__ __attribute__((aligned(1024))) char smem[G::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles = gridDim.x / 2;
  const int hi_half = blockIdx.x >= tiles;
  const int b = blockIdx.x - hi_half * tiles;
  int pid_m, pid_n;
  tile_coords(b, (M + BM - 1) / BM, (N + BN - 1) / BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;
  const int nk = K / G::BK, kmid = nk / 2;

  f32x16 acc[FN][FM];
  zero_acc<T, FM, FN>(acc);
  dtl_accumulate<T, BM, BN, WM, WN, BKB, STAGES, 1>(smem, A, lda, W, ldw, M, N, m0, n0, hi_half ? kmid : 0,
                                                    hi_half ? nk : kmid, acc);
  char* const stage = smem + wave * EpiStage<T, EPI, FN>::BYTES;
  if (!hi_half) {
    epilogue<T, EPI, FM, FN, NoParts, kResWriteThrough>(acc, bias, C, ldc, M, N, m0 + wm * G::WTM,
                                                        n0 + wn * G::WTN, lane, stage);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the tile is in memory
    __syncthreads();
    if (tid == 0) __hip_atomic_store(&flags[b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    int spins = 0;
    while (__hip_atomic_load(&flags[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
      if (++spins > kSkSpinLimit) {
        if (tid == 0) __hip_atomic_fetch_add(&flags[-1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    epilogue<T, EPI, FM, FN, NoParts, kResCoherentLoad>(acc, nullptr, C, ldc, M, N, m0 + wm * G::WTM,
                                                        n0 + wn * G::WTN, lane, stage);
    __syncthreads();
    if (tid == 0) __hip_atomic_store(&flags[b], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------------ plans

enum { kStaged = 0, kDtl = 1, kSk = 2, kK2 = 3 };

struct GemmPlan {
  int kind, bm, bn, wm, wn, bkb, stages;
  double eff;      // prior used by auto_plan
  int ksplit = 1;  // K groups per workgroup (direct-to-LDS kernel)
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
    // 18-23: stream-K (persistent grid, K-split partial tiles; need a
    // workspace of tjk_gemm_workspace_bytes()).
    {kSk, 256, 256, 2, 4, 128, 2, 1.00},      // 18 8 waves, wave tile 128x64
    {kSk, 256, 256, 2, 2, 128, 2, 1.00},      // 19 wave tile 128x128
    {kSk, 192, 256, 2, 4, 128, 2, 1.00},      // 20 8 waves, wave tile 96x64
    {kSk, 192, 384, 2, 4, 128, 2, 1.00},      // 21 8 waves, wave tile 96x96
    {kSk, 192, 128, 2, 2, 128, 2, 1.00},      // 22 wave tile 96x64
    {kSk, 128, 128, 2, 2, 128, 2, 1.00},      // 23 wave tile 64x64
    // 24, 25: split-K residual (TJK_EPI_BIAS_RESIDUAL only; workspace).
    {kK2, 192, 128, 2, 2, 128, 2, 1.00},      // 24 wave tile 96x64, 2 WGs per tile
    {kK2, 128, 128, 2, 2, 128, 2, 1.00},      // 25 wave tile 64x64, 2 WGs per tile
    // 26: a 4-slot ring (160 KB) with the spread DMA schedule, one workgroup
    // per CU.  Other deep rings measured (C4/C5 projections, residual reads
    // prefetched where registers allow) and dropped because a 2-slot plan
    // was faster on every shape: 256x256 8 waves and 4 waves with 64-byte
    // rows in 4 slots, 128x128 and 96x128 in 4 slots, 256x128 in 3 slots.
    {kDtl, 192, 128, 2, 2, 128, 4, 0.85},     // 26 wave tile 96x64, 160 KB
    // 27, 28: small tiles in deep rings (8 and 6 slots) for launches of a few
    // dozen workgroups with long K (C2's FFN2: 16 tiles, 32 K tiles each),
    // where a 2-slot ring leaves each step waiting out the DMA latency.
    {kDtl, 64, 64, 2, 2, 128, 8, 0.45},       // 27 wave tile 32x32, 128 KB
    {kDtl, 128, 64, 2, 2, 128, 6, 0.50},      // 28 wave tile 64x32, 144 KB
    // 29-31: the same small tiles with K split between 2 or 4 groups of 4
    // waves inside the workgroup (partials added through LDS), which
    // shortens the serial chain of K tiles a launch of a few dozen
    // workgroups waits out.
    {kDtl, 64, 64, 2, 2, 128, 2, 0.45, 4},    // 29 16 waves, 128 KB
    {kDtl, 64, 64, 2, 2, 128, 4, 0.45, 2},    // 30 8 waves, 128 KB
    {kDtl, 128, 64, 2, 2, 128, 3, 0.50, 2},   // 31 8 waves, 144 KB
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
    if (p[i].kind == kSk || p[i].kind == kK2) continue;
    if (p[i].kind == kDtl && !dtl_ok(p[i], K, lda, ldw, sizeof(T))) continue;
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
  int M, N, K; void* ws; size_t ws_bytes; hipStream_t s;
};
template <int KIND> struct Launcher;
template <> struct Launcher<kStaged> {
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    const dim3 grid(((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN));
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, EPI>), grid, dim3(WM * WN * 64), 0, g.s, (const T*)g.a,
                       g.lda, (const T*)g.w, g.ldw, (const T*)g.bias, g.c, g.ldc, g.M, g.N, g.K);
    return TJK_OK;
  }
};
template <int BKB, int STAGES, int KSPLIT = 1> struct DtlLauncher {
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    const dim3 grid(((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN));
    hipLaunchKernelGGL((gemm_dtl_kernel<T, BM, BN, WM, WN, BKB, STAGES, EPI, KSPLIT>), grid,
                       dim3(WM * WN * KSPLIT * 64), 0, g.s, (const T*)g.a, g.lda, (const T*)g.w, g.ldw,
                       (const T*)g.bias, g.c, g.ldc, g.M, g.N, g.K);
    return TJK_OK;
  }
};

// Resident grid of a persistent kernel on the current device: CUs x
// workgroups per CU (queried once per kernel and device), at most kMaxSkGrid.
template <typename F>
static int resident_grid(F kernel, int threads) {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel), threads, 0) !=
      hipSuccess)
    return 0;
  const int g = min(max(cus * per_cu, 1), kMaxSkGrid);
  if (dev < 64) cached[dev] = g;
  return g;
}

template <int BKB, int STAGES> struct SkLauncher {
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int grid() {
    return resident_grid(gemm_sk_kernel<T, BM, BN, WM, WN, BKB, STAGES, EPI>, WM * WN * 64);
  }
  template <typename T, int BM, int BN, int WM, int WN>
  static size_t workspace_bytes() {
    const int g = max(max(grid<T, BM, BN, WM, WN, TJK_EPI_BIAS>(), grid<T, BM, BN, WM, WN, TJK_EPI_BIAS_GELU>()),
                      grid<T, BM, BN, WM, WN, TJK_EPI_BIAS_RESIDUAL>());
    return g > 0 ? kSkHeader + (size_t)g * BM * BN * sizeof(float) : 0;
  }
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    const int G = grid<T, BM, BN, WM, WN, EPI>();
    if (G <= 0) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: no resident grid for the stream-K plan");
    if (!g.ws) return fail(TJK_EINVAL, "tjk_gemm_bias: stream-K plan needs a workspace (tjk_gemm_bias_ws)");
    const size_t need = kSkHeader + (size_t)G * BM * BN * sizeof(float);
    if (g.ws_bytes < need || ((uintptr_t)g.ws & 255))
      return fail(TJK_EINVAL, "tjk_gemm_bias: stream-K workspace needs %zu bytes, 256-byte aligned (got %zu)", need,
                  g.ws_bytes);
    constexpr int BK = BKB / sizeof(T);
    SkParams p;
    p.tiles_m = (g.M + BM - 1) / BM;
    p.tiles_n = (g.N + BN - 1) / BN;
    p.nk = g.K / BK;
    const int tiles = p.tiles_m * p.tiles_n;
    // whole rounds stay data-parallel except the last full one, which joins
    // the partial round in the stream-K part (no K segment shorter than
    // about a tile's worth per workgroup)
    if (tiles % G == 0) p.dp_tiles = tiles;
    else if (tiles < G) p.dp_tiles = 0;
    else p.dp_tiles = (tiles / G - 1) * G;
    const int64_t units = (int64_t)(tiles - p.dp_tiles) * p.nk;
    if (units > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: too many stream-K units");
    p.sk_units = (int)units;
    hipLaunchKernelGGL((gemm_sk_kernel<T, BM, BN, WM, WN, BKB, STAGES, EPI>), dim3(G), dim3(WM * WN * 64), 0, g.s,
                       (const T*)g.a, g.lda, (const T*)g.w, g.ldw, (const T*)g.bias, g.c, g.ldc, g.M, g.N, p,
                       (char*)g.ws);
    return TJK_OK;
  }
};

template <int BKB, int STAGES> struct K2Launcher {
  template <typename T, int BM, int BN, int WM, int WN>
  static size_t workspace_bytes() { return kSkHeader; }
  template <typename T, int BM, int BN, int WM, int WN, int EPI>
  static int go(const GemmArgs& g) {
    if constexpr (EPI != TJK_EPI_BIAS_RESIDUAL) {
      return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: split-K plans take only the residual epilogue");
    } else {
      if (!g.ws) return fail(TJK_EINVAL, "tjk_gemm_bias: split-K plan needs a workspace (tjk_gemm_bias_ws)");
      if (g.ws_bytes < kSkHeader || ((uintptr_t)g.ws & 255))
        return fail(TJK_EINVAL, "tjk_gemm_bias: split-K workspace needs %zu bytes, 256-byte aligned (got %zu)",
                    kSkHeader, g.ws_bytes);
      const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
      if (tiles > kMaxK2Tiles - 1 || (int64_t)g.M * g.ldc * 4 >= INT32_MAX)
        return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: shape too large for the split-K plan");
      int* flags = reinterpret_cast<int*>(static_cast<char*>(g.ws) + kK2FlagOffset) + 1;  // [-1]: timeouts
      hipLaunchKernelGGL((gemm_k2_residual_kernel<T, BM, BN, WM, WN, BKB, STAGES>), dim3(2 * tiles),
                         dim3(WM * WN * 64), 0, g.s, (const T*)g.a, g.lda, (const T*)g.w, g.ldw, (const T*)g.bias,
                         (float*)g.c, g.ldc, g.M, g.N, g.K, flags);
      return TJK_OK;
    }
  }
};

template <typename L, typename T, int BM, int BN, int WM, int WN>
static int launch_epi(int epi, const GemmArgs& g) {
  switch (epi) {
    case TJK_EPI_BIAS: return L::template go<T, BM, BN, WM, WN, TJK_EPI_BIAS>(g);
    case TJK_EPI_BIAS_GELU: return L::template go<T, BM, BN, WM, WN, TJK_EPI_BIAS_GELU>(g);
    default: return L::template go<T, BM, BN, WM, WN, TJK_EPI_BIAS_RESIDUAL>(g);
  }
}

typedef Launcher<kStaged> St;
typedef DtlLauncher<128, 2> D2;
typedef DtlLauncher<128, 2, 2> D2K2;
typedef DtlLauncher<128, 2, 4> D2K4;
typedef DtlLauncher<128, 4, 2> D4K2;
typedef DtlLauncher<128, 3, 2> D3K2;
typedef DtlLauncher<128, 4> D4;
typedef DtlLauncher<128, 6> D6;
typedef DtlLauncher<128, 8> D8;
typedef SkLauncher<128, 2> SK2;
typedef K2Launcher<128, 2> K22;

// Plans of the 2-byte table that need a workspace (stream-K, split-K):
// (id, launcher, BM, BN, WM, WN).
#define TJK_WS_PLANS(X)      \
  X(18, SK2, 256, 256, 2, 4) \
  X(19, SK2, 256, 256, 2, 2) \
  X(20, SK2, 192, 256, 2, 4) \
  X(21, SK2, 192, 384, 2, 4) \
  X(22, SK2, 192, 128, 2, 2) \
  X(23, SK2, 128, 128, 2, 2) \
  X(24, K22, 192, 128, 2, 2) \
  X(25, K22, 128, 128, 2, 2)

template <typename T>
static size_t sk_workspace_bytes(int plan) {
  if constexpr (sizeof(T) == 4) {
    return 0;
  } else {
    switch (plan) {
#define TJK_SK_WS(ID, L, BM, BN, WM, WN) \
  case ID: return L::template workspace_bytes<T, BM, BN, WM, WN>();
      TJK_WS_PLANS(TJK_SK_WS)
#undef TJK_SK_WS
    }
    return 0;
  }
}

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
      TJK_WS_PLANS(TJK_GEMM_CASE)
      TJK_GEMM_CASE(26, D4, 192, 128, 2, 2)
      TJK_GEMM_CASE(27, D8, 64, 64, 2, 2)
      TJK_GEMM_CASE(28, D6, 128, 64, 2, 2)
      TJK_GEMM_CASE(29, D2K4, 64, 64, 2, 2)
      TJK_GEMM_CASE(30, D4K2, 64, 64, 2, 2)
      TJK_GEMM_CASE(31, D3K2, 128, 64, 2, 2)
    }
  }
#undef TJK_GEMM_CASE
  if (rc != TJK_OK) return rc;
  return check_launch("tjk_gemm_bias");
}

template <typename T>
static int gemm_checked(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                        int64_t ldc, int64_t m, int64_t n, int64_t k, int epi, int plan, void* ws,
                        size_t ws_bytes, hipStream_t s) {
  int count;
  const GemmPlan* p = plans<T>(&count);
  if (plan < -1 || plan >= count) return fail(TJK_EINVAL, "tjk_gemm_bias: plan %d out of range [-1,%d)", plan, count);
  if (plan == -1) plan = auto_plan<T>(m, n, k, lda, ldw);
  if (p[plan].kind != kStaged && !dtl_ok(p[plan], k, lda, ldw, sizeof(T)))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: plan %d needs k %% %d == 0", plan, (int)(p[plan].bkb / sizeof(T)));
  if (p[plan].kind != kStaged && ((int64_t)p[plan].bm * lda * (int64_t)sizeof(T) > INT32_MAX ||
                                  (int64_t)p[plan].bn * ldw * (int64_t)sizeof(T) > INT32_MAX))
    return fail(TJK_EUNSUPPORTED, "tjk_gemm_bias: leading dimension too large for plan %d", plan);
  const GemmArgs g{a, lda, w, ldw, bias, c, ldc, (int)m, (int)n, (int)k, ws, ws_bytes, s};
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

extern "C" int tjk_gemm_plan_info(int dtype, int id, int* block_m, int* block_n, int* waves) {
  int count = 0;
  const GemmPlan* p;
  if (dtype == TJK_F32) p = plans<float>(&count);
  else if (dtype == TJK_F16 || dtype == TJK_BF16) p = plans<bf16>(&count);
  else return fail(TJK_EINVAL, "tjk_gemm_plan_info: bad dtype %d", dtype);
  if (id < 0 || id >= count) return fail(TJK_EINVAL, "tjk_gemm_plan_info: plan %d out of range", id);
  if (block_m) *block_m = p[id].bm;
  if (block_n) *block_n = p[id].bn;
  if (waves) *waves = p[id].wm * p[id].wn * p[id].ksplit;
  return TJK_OK;
}

extern "C" size_t tjk_gemm_workspace_bytes(int dtype, int plan_id) {
  switch (dtype) {
    case TJK_F16: return sk_workspace_bytes<f16>(plan_id);
    case TJK_BF16: return sk_workspace_bytes<bf16>(plan_id);
    default: return 0;
  }
}

extern "C" int tjk_gemm_bias(const void* a, int64_t lda, const void* w, int64_t ldw,
                             const void* bias, void* c, int64_t ldc,
                             int64_t m, int64_t n, int64_t k,
                             int dtype, int epilogue, int plan_id, void* stream) {
  return tjk_gemm_bias_ws(a, lda, w, ldw, bias, c, ldc, m, n, k, dtype, epilogue, plan_id, nullptr, 0, stream);
}

extern "C" int tjk_gemm_bias_ws(const void* a, int64_t lda, const void* w, int64_t ldw,
                                const void* bias, void* c, int64_t ldc,
                                int64_t m, int64_t n, int64_t k,
                                int dtype, int epilogue, int plan_id,
                                void* workspace, size_t workspace_bytes, void* stream) {
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
      return gemm_checked<float>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, workspace,
                                 workspace_bytes, s);
    case TJK_F16:
      return gemm_checked<f16>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, workspace,
                               workspace_bytes, s);
    default:
      return gemm_checked<bf16>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, plan_id, workspace,
                                workspace_bytes, s);
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
