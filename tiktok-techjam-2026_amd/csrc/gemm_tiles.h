// Device building blocks shared by the GEMM and fused-FFN kernels: the
// erf GELU, the XCD-aware tile order, the LDS-staged epilogue and the
// direct-to-LDS (buffer_load ... lds) MFMA main loop.
#pragma once

#include <type_traits>

#include "tjk_common.h"

namespace tjk {

// Row tiles per group of the tile raster (tile_coords).  Whole forwards,
// five builds alternating on one box: 4 ran C4 / C5 0.27% / 0.22% faster
// than 8, 2 and 1 slower at C5, 16 1.6% slower at C4.
constexpr int kGroupM = 4;

// GELU(v) = v Phi(v) with erf from Abramowitz & Stegun, Handbook of
// Mathematical Functions, eq. 7.1.28 (|error| <= 3e-7): for z >= 0,
// erfc z = (1 + a1 z + a2 z^2 + ... + a6 z^6)^-16.  With u = |v| and
// h = erfc(u / sqrt 2) / 2, Phi(v) = 1 - h for v >= 0 and h for v < 0, so
// GELU(v) = max(v, 0) - u h: one FMA after the reciprocal, exact in the
// negative tail (no 1 - erf cancellation).  The polynomial is taken in u
// (coefficients a_i / sqrt(2)^i) and scaled by 2^(1/16), so that its 16th
// power (four squarings) is 2 (1 + ...)^16 and its reciprocal is h: one
// reciprocal and no exponential, where eq. 7.1.26 needs both (the
// transcendental instructions run at a quarter of the VALU rate, and the
// epilogue of an FFN1 tile is VALU-bound).  Branch-free -- the library
// erff branches on |z| and measured ~35 VALU instructions per value with
// divergent lanes.
__device__ __forceinline__ float gelu_erf(float v) {
  const float u = fabsf(v);
  // 2^(1/16) x (1, a1 / sqrt 2, ..., a6 / sqrt(2)^6), a1..a6 = 0.0705230784,
  // 0.0422820123, 0.0092705272, 0.0001520143, 0.0002765672, 0.0000430638
  float p = fmaf(u, 5.62129981e-06f, 5.1055209e-05f);
  p = fmaf(p, u, 3.9686136e-05f);
  p = fmaf(p, u, 3.42273922e-03f);
  p = fmaf(p, u, 2.20769979e-02f);
  p = fmaf(p, u, 5.20751625e-02f);
  p = fmaf(p, u, 1.04427373f);
  p *= p;
  p *= p;
  p *= p;
  p *= p;  // 2 (1 + ...)^16 (inf for large |v|: the reciprocal is then 0)
  const float h = __builtin_amdgcn_rcpf(p);
  return fmaf(-u, h, fmaxf(v, 0.0f));
}

// Bijection from hardware workgroup id to a tile order in which XCD x gets
// the contiguous range of ids [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
  const int per = nb / 8, rem = nb % 8;
  const int x = bid % 8, i = bid / 8;
  return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}


// Internal epilogue mode beside the ABI's TJK_EPI_*: store the fp32 sum
// (acc + bias) as is, no read-modify-write (the fused FFN's split partials).
constexpr int kEpiStoreF32 = 3;
// Internal epilogue mode: TJK_EPI_BIAS_RESIDUAL with the residual read from
// a ResSrc (below) instead of from C.
constexpr int kEpiResidualFrom = 4;
// Residual pieces a residual epilogue without a prefetch reads per batch
// (four VGPRs each; from a ResSrc at most four, whose x rows take more
// registers: eight spilled the 256 x 256 tiles there).  Eight against four
// measured C5 -0.24%, C4 unchanged (one process, interleaved rounds).
constexpr int kResBatch = 8;
__host__ __device__ constexpr bool epi_residual(int epi) {
  return epi == TJK_EPI_BIAS_RESIDUAL || epi == kEpiResidualFrom;
}

// Epilogue shared by the GEMM and fused-FFN kernels.  The accumulators hold
// C^T blocks: for block (i, j), lane (l32, hi) owns output row
// m = mw + 32 j + l32 and, for g = 0..3, the four consecutive columns
// n = nw + 32 i + 8 g + 4 hi.  Stored straight from that layout, every store
// instruction would scatter 8-16 byte pieces over 32 rows (32 L2 requests
// per instruction), which measured slower than the whole K=1024 main loop.
// Instead each wave applies bias / GELU in registers, transposes one 32-row
// block at a time through a private LDS region and writes whole row
// segments: 16 bytes per lane, WTN contiguous elements per row.  The
// residual epilogue stages fp32 and does its read-modify-write of the fp32
// residual with the same row-contiguous pieces; kEpiStoreF32 stages fp32
// and stores it.
//
// The staging is written and read in 16-byte pieces.  Measured on MI355X
// (SQ_LDS_BANK_CONFLICT of probe kernels), a 16-byte LDS write serves 8
// lanes per cycle over 32 banks and a 16-byte read 32 lanes per cycle over
// 128 banks.  A staged row holds LPR pieces (a multiple of 4) with no
// padding, and piece p of row r sits at slot r LPR + (p ^ x(r)), x(r) =
// r & 7 if LPR % 8 == 0, else (r >> 1) & 3.  A write puts one piece of each
// of 8 consecutive rows per cycle, which the XOR spreads over the 8 bank
// groups; a read takes 32 consecutive pieces in row-major order, and the
// XOR only permutes pieces within aligned groups of 8 (or 4) that every
// such window covers whole.  In fp32 each lane's four columns are one
// piece.  In a 2-byte type a piece's two halves sit in lanes l32 and
// l32 + 32, so pieces g = 2k, 2k + 1 trade halves (v_permlane32_swap) and
// each lane writes a whole piece.  (8-byte writes from rows padded by one
// piece counted ~7 conflict cycles per write and ~4 per read in the probe.)
template <typename T, int EPI, int FN>
struct EpiStage {
  static constexpr bool F32OUT = epi_residual(EPI) || EPI == kEpiStoreF32;
  typedef typename std::conditional<F32OUT, float, T>::type S;  // staged type
  static constexpr int WTN = FN * 32;
  static constexpr int SV = 16 / (int)sizeof(S);  // elements per 16-byte piece
  static constexpr int LPR = WTN / SV;            // pieces per staged row
  static constexpr int BYTES = 32 * LPR * 16;     // LDS bytes per wave
  static_assert(LPR % 4 == 0, "staged rows of whole 4-piece groups");
  static constexpr int G = LPR % 8 == 0 ? 8 : 4;  // pieces per XOR group
  static __device__ __forceinline__ int x(int r) { return G == 8 ? (r & 7) : ((r >> 1) & 3); }
  // byte offset of piece p of staged row r
  static __device__ __forceinline__ int at(int r, int p) { return (r * LPR + (p ^ x(r))) * 16; }
};

// Where kEpiResidualFrom reads the residual it adds: a matrix x in the
// compute dtype, leading dimension ld, with an optional row map -- output
// row m reads x row rows[m] (row m without a map).  A row outside
// [0, nrows) reads as zeros and is counted once in *errors (when given).
// C is written, not read: the first layer's out-projection adds the packed
// input rows straight from x, so the first LayerNorm need not materialize
// the fp32 residual.  (TJK_EPI_BIAS_RESIDUAL reads C and ignores it.)
// Where there is no map entry or x row to read, the reads go to C's first
// 16 bytes instead and their value is not used: a read from a selected
// address needs no branch, and a branch whose paths join after reads waits
// for them there, and for every store in flight with them.
struct ResSrc {
  const void* x;
  int64_t ld;
  const int32_t* rows;
  int64_t nrows;
  int* errors;
};

// The residual pieces (TJK_EPI_BIAS_RESIDUAL, kEpiResidualFrom) a wave's
// epilogue will update, read into registers before the main loop.  A launch
// whose tiles all run in one round otherwise starts every residual read at
// the same moment, after the last MFMA; read early, they overlap the main
// loop and the epilogue only writes.  Piece (j, it) is the one the
// epilogue's store loop handles for 32-row block j, iteration it.  Pieces
// from a ResSrc stay raw (half the registers of fp32 for a 2-byte x) until
// the epilogue converts them.
struct NoPrefetch {
  static constexpr bool on = false;
  __device__ float4 get(int, int) const { return make_float4(0.f, 0.f, 0.f, 0.f); }
};
template <int FM, int FN, typename T = float, bool FROM = false>
struct ResPrefetch {
  static constexpr bool on = true;
  static constexpr int WTN = FN * 32, LPR = WTN / 4, NPC = 32 * LPR, NIT = (NPC + 63) / 64;
  typedef typename std::conditional<FROM, typename Quad<T>::raw, float4>::type Piece;
  // VGPRs per lane counted against a kernel's budget: four per piece in
  // either form (a raw piece and its x row take three)
  static constexpr int REGS = FM * NIT * 4;
  Piece r[FM][NIT];
  int xrow[FROM ? FM : 1][FROM ? NIT : 1];
  int64_t nrows = 0;
  // From a ResSrc every read is from a clamped (always valid) address,
  // none under a per-lane condition, so all of them go out before any
  // returns (the row map first, then x); a clamped piece is never used.
  __device__ __forceinline__ void load(const float* __restrict__ C, int64_t ldc, int M, int N, int mw, int nw,
                                       int lane, const ResSrc& s) {
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if constexpr (FROM) {
          const int pc = min(lane + 64 * it, NPC - 1);
          const int m = min(mw + 32 * j + pc / LPR, M - 1);
          const int v = *(s.rows != nullptr ? s.rows + m : reinterpret_cast<const int32_t*>(C));
          xrow[j][it] = s.rows != nullptr ? v : m;
        } else {
          const int pc = lane + 64 * it;
          const int m = mw + 32 * j + pc / LPR, n = nw + (pc % LPR) * 4;
          const bool in = (NPC % 64 == 0 || pc < NPC) && m < M && n < N;
          r[j][it] = in ? *reinterpret_cast<const float4*>(C + (int64_t)m * ldc + n) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    if constexpr (FROM) {
      nrows = s.nrows;
#pragma unroll
      for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int pc = min(lane + 64 * it, NPC - 1);
          const int n = min(nw + (pc % LPR) * 4, N - 4);
          r[j][it] = *(valid(j, it) ? reinterpret_cast<const Piece*>(static_cast<const T*>(s.x) +
                                                                     (int64_t)xrow[j][it] * s.ld + n)
                                    : reinterpret_cast<const Piece*>(C));
        }
    }
  }
  // whether piece (j, it)'s x row lies inside x (ResSrc only)
  __device__ __forceinline__ bool valid(int j, int it) const {
    return xrow[FROM ? j : 0][FROM ? it : 0] >= 0 && xrow[FROM ? j : 0][FROM ? it : 0] < nrows;
  }
  __device__ __forceinline__ float4 get(int j, int it) const {
    if constexpr (FROM) return valid(j, it) ? Quad<T>::to(r[j][it]) : make_float4(0.f, 0.f, 0.f, 0.f);
    else return r[j][it];
  }
};

// The bias pieces of a wave's columns nw.. (the epilogue's layout: lane
// (l32, hi) needs columns nw + 32 i + 8 g + 4 hi .. +3), raw.  All loads go
// out before any is used -- one memory round trip; a load under a per-lane
// condition would be waited for on its own, one round trip per load -- with
// columns past N clamped into range (N % 4 == 0, N >= 4) and zeroed when
// converted.  A kernel whose registers allow it loads them before its main
// loop, which takes that round trip off the end of the launch.
template <typename T, int FN>
struct BiasRaw {
  typedef typename Quad<T>::raw Raw;
  Raw r[FN][4];
  __device__ __forceinline__ void load(const T* __restrict__ bias, int N, int nw, int lane) {
    const int hi = lane >> 5;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) r[i][g] = Raw{};
    if (bias != nullptr) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          r[i][g] = *reinterpret_cast<const Raw*>(bias + min(nw + i * 32 + g * 8 + hi * 4, N - 4));
    }
  }
};

// Stores this wave's (32 FM) x (32 FN) block at rows mw.., columns nw.. of
// C (rows >= M and columns >= N dropped).  `stage` is the wave's private
// EpiStage<T, EPI, FN>::BYTES of LDS.  `bpre`, when given, holds the bias
// pieces already loaded (BiasRaw::load with the same bias, N, nw, lane).
// RB_: residual pieces per batched read (0: read one by one).
template <typename T, int EPI, int FM, int FN, typename Pre = NoPrefetch, int RB_ = kResBatch>
__device__ __forceinline__ void epilogue(const f32x16 (&acc)[FN][FM], const T* __restrict__ bias,
                                         void* __restrict__ Cv, int64_t ldc, int M, int N, int mw, int nw,
                                         int lane, char* __restrict__ stage, const Pre& pre = Pre(),
                                         const BiasRaw<T, FN>* bpre = nullptr,
                                         const ResSrc& src = ResSrc{nullptr, 0, nullptr, 0, nullptr}) {
  typedef EpiStage<T, EPI, FN> E;
  constexpr int LPR = E::LPR;          // 16-byte pieces per staged row
  constexpr int NPC = 32 * LPR;        // pieces per 32-row block
  constexpr int NIT = (NPC + 63) / 64; // read instructions per block
  const int l32 = lane & 31, hi = lane >> 5;
  // 16-byte output pieces need a 16-byte aligned C and a leading dimension
  // that keeps every row 16-byte aligned; otherwise pieces go out as halves.
  const bool a16 = ((uintptr_t)Cv & 15) == 0 && (ldc % E::SV) == 0;
  constexpr int OB = E::F32OUT ? 4 : (int)sizeof(T);  // output bytes per element
  const bool wt = (int64_t)M * N * OB >= kWtMinBytes;

  // bias of this wave's columns (loaded here unless the caller did)
  BiasRaw<T, FN> own;
  if (bpre == nullptr) own.load(bias, N, nw, lane);
  const BiasRaw<T, FN>& braw = bpre != nullptr ? *bpre : own;
  float4 bv[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = nw + i * 32 + g * 8 + hi * 4;
      bv[i][g] = n < N ? Quad<T>::to(braw.r[i][g]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }

  // columns 32 i + 8 g + 4 hi .. +3 of this lane's row, bias / GELU applied
  auto value = [&](int j, int i, int g) __attribute__((always_inline)) {
    float4 v = make_float4(acc[i][j][4 * g + 0] + bv[i][g].x, acc[i][j][4 * g + 1] + bv[i][g].y,
                           acc[i][j][4 * g + 2] + bv[i][g].z, acc[i][j][4 * g + 3] + bv[i][g].w);
    if (EPI == TJK_EPI_BIAS_GELU) {
      v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
    }
    return v;
  };

  // Staging offsets, the same for every 32-row block.  Writes: piece C + hi
  // of row l32 (C even, a compile-time value) sits at C ^ wx with
  // wx = x(l32) ^ hi, i.e. at the constant C & ~(G - 1) plus one of G / 2
  // per-lane offsets.  Reads: one offset per read instruction.
  char* const wrow = stage + l32 * LPR * 16;
  const int wx = E::x(l32) ^ hi;
  auto wslot = [&](int c) __attribute__((always_inline)) {
    return wrow + 16 * ((c & ~(E::G - 1)) + ((c & (E::G - 1)) ^ wx));
  };
  int roff[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int pc = min(lane + 64 * it, NPC - 1);
    roff[it] = E::at(pc / LPR, pc % LPR);
  }

  // kEpiResidualFrom with batched reads: lane (l32, *) holds the x row of
  // output row mw + 32 j + l32, read from the row map one block ahead (a
  // wait for a read issued after the previous block's stores would also
  // wait for those stores); without a map (identity) the read goes to a
  // word of C and is not used (see ResSrc).
  constexpr bool XMAP = EPI == kEpiResidualFrom && !Pre::on && RB_ > 0;
  const bool has_map = src.rows != nullptr;
  auto map_read = [&](int j) __attribute__((always_inline)) {
    const int m = min(mw + 32 * j + l32, M - 1);
    return *(has_map ? src.rows + m : static_cast<const int32_t*>(Cv));
  };
  int map_next = XMAP ? map_read(0) : 0;

#pragma unroll
  for (int j = 0; j < FM; ++j) {
    // Without a prefetch, the block's residual pieces are read ahead of
    // their use, RB_ at a time from clamped (always valid) addresses: the
    // first batch before the block's staging, each further one when the
    // store loop starts the batch before it.  Read inside the store loop
    // (RB_ == 0: the register-tight tiles, which the batches spilled), under
    // each lane's bounds check, every piece waits for its own round trip.
    // A clamped piece is never used.
    constexpr bool RES_LOAD = epi_residual(EPI) && !Pre::on && RB_ > 0;
    constexpr int NRL = RES_LOAD ? NIT : 1;
    constexpr int RBE = EPI == kEpiResidualFrom && RB_ > 4 ? 4 : RB_;
    constexpr int RB = RBE < 1 ? 1 : RBE < NIT ? RBE : NIT;
    typedef typename std::conditional<EPI == kEpiResidualFrom, typename Quad<T>::raw, float4>::type ResPiece;
    ResPiece rl[NRL];
    int xrow[EPI == kEpiResidualFrom ? NRL : 1];
    if constexpr (XMAP) {
      const int map = map_next;
      if (j + 1 < FM) map_next = map_read(j + 1);
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int pc = min(lane + 64 * it, NPC - 1);
        const int mrow = __shfl(map, pc / LPR);  // lanes r and r + 32 hold row r's entry
        xrow[it] = has_map ? mrow : min(mw + 32 * j + pc / LPR, M - 1);
      }
    }
    auto res_read = [&](int b) __attribute__((always_inline)) {
      if constexpr (RES_LOAD) {
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int it = RB * b + q;
          if (it >= NIT) break;
          const int pc = min(lane + 64 * it, NPC - 1);
          const int m = min(mw + 32 * j + pc / LPR, M - 1), n = min(nw + (pc % LPR) * 4, N - 4);
          if constexpr (EPI == kEpiResidualFrom) {
            const int xr = xrow[it];
            const bool ok = xr >= 0 && xr < src.nrows;
            rl[it] = *(ok ? reinterpret_cast<const ResPiece*>(static_cast<const T*>(src.x) + (int64_t)xr * src.ld + n)
                          : static_cast<const ResPiece*>(Cv));
          } else {
            rl[it] = *reinterpret_cast<const float4*>(static_cast<const float*>(Cv) + (int64_t)m * ldc + n);
          }
        }
      }
    };
    res_read(0);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      if constexpr (E::SV == 4) {  // fp32 staged: a lane's four columns are one piece
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<float4*>(wslot(8 * i + 2 * g)) = value(j, i, g);
      } else {
        static_assert(sizeof(typename Quad<T>::raw) == 8, "2-byte staged type");
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          // lane (l32, 0) ends with piece 4 i + 2 k of row l32, lane (l32, 1)
          // with piece 4 i + 2 k + 1: the swap trades the upper lanes' half
          // of the first for the lower lanes' half of the second
          const typename Quad<T>::raw x = Quad<T>::from(value(j, i, 2 * k));
          const typename Quad<T>::raw y = Quad<T>::from(value(j, i, 2 * k + 1));
          const auto s0 = __builtin_amdgcn_permlane32_swap(x.x, y.x, false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(x.y, y.y, false, false);
          *reinterpret_cast<uint4*>(wslot(4 * i + 2 * k)) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
        }
      }
    }
    // rows mw + 32 j .. of this block, from column nw
    const int64_t rb0 = (int64_t)(mw + 32 * j) * ldc + nw;
    const RowOut rows(static_cast<char*>(Cv) + rb0 * OB, ((int64_t)M * ldc - rb0) * OB, wt);
    with_wt(rows.wt, [&](auto wt_tag) {
      const auto wr = rows.writer<decltype(wt_tag)::value>();
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if (RES_LOAD && it % RB == 0 && it + RB < NIT) res_read(it / RB + 1);
        const int pc = lane + 64 * it;  // piece index: row pc / LPR, piece pc % LPR
        if (NPC % 64 != 0 && pc >= NPC) break;
        const int rr = pc / LPR, cc = (pc % LPR) * E::SV;
        const int m = mw + 32 * j + rr, n = nw + cc;
        const uint4 piece = *reinterpret_cast<const uint4*>(stage + roff[it]);
        const int off = (int)(((int64_t)rr * ldc + cc) * OB);
        if (m < M && n < N) {
          if constexpr (epi_residual(EPI)) {
            // fp32 pieces never straddle N (N % 4 == 0)
            const float4 a = __builtin_bit_cast(float4, piece);
            float4 o;
            int xr = 0;  // x row (ResSrc)
            if constexpr (Pre::on) {
              o = pre.get(j, it);
            } else if constexpr (RES_LOAD) {
              if constexpr (EPI == kEpiResidualFrom) {
                xr = xrow[it];
                o = xr >= 0 && xr < src.nrows ? Quad<T>::to(rl[it]) : make_float4(0.f, 0.f, 0.f, 0.f);
              } else {
                o = rl[it];
              }
            } else if constexpr (EPI == kEpiResidualFrom) {
              xr = src.rows != nullptr ? src.rows[m] : m;
              o = xr >= 0 && xr < src.nrows
                      ? Quad<T>::to(*reinterpret_cast<const typename Quad<T>::raw*>(
                            static_cast<const T*>(src.x) + (int64_t)xr * src.ld + n))
                      : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
              o = *reinterpret_cast<const float4*>(rows.p + off);
            }
            if constexpr (EPI == kEpiResidualFrom) {
              bool bad;
              if constexpr (Pre::on) bad = !pre.valid(j, it);
              else bad = !(xr >= 0 && xr < src.nrows);
              if (bad && n == 0 && src.errors != nullptr)
                atomicAdd(src.errors, 1);  // once per row: column 0 is one lane of one tile
            }
            o.x += a.x; o.y += a.y; o.z += a.z; o.w += a.w;
            wr.put(off, o);
          } else if constexpr (EPI == kEpiStoreF32) {
            wr.put(off, piece);
          } else {
            if (E::SV == 4 || (a16 && n + E::SV <= N)) {
              wr.put(off, piece);
            } else {  // 2-byte types: halves of 4 elements (N % 4 == 0)
              T* c = static_cast<T*>(Cv) + (int64_t)m * ldc + n;
              *reinterpret_cast<uint2*>(c) = make_uint2(piece.x, piece.y);
              if (n + 4 < N) *reinterpret_cast<uint2*>(c + 4) = make_uint2(piece.z, piece.w);
            }
          }
        }
      }
    });
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
  static_assert(STAGES >= 2 && 2 * (STAGES - 1) * NDMA <= 63, "vmcnt range");
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
  // Eight-wave tiles with 96 x 96 (or larger) wave tiles issue every DMA
  // instruction from waves 0-3 (one per SIMD), twice their share, and none
  // from waves 4-7: a wave whose DMA cannot issue yet stalls its own in-order
  // MFMAs, and with the issue on one wave of each SIMD the other keeps the
  // matrix pipe busy meanwhile.  Measured (A/B of two builds, one box):
  // 192 x 384 tiles 37.3 -> 36.85 us on the packed C4 QKV, 79.3 -> 78.0 us
  // at 5430 x 4096 x 1024 with GELU, 898 -> 886 us at 8192^3; the 8-wave
  // 256 x 256 tile (128 x 64 wave tiles) got 1-2.5% slower with it and 192 x 128
  // / 192 x 256 ones no faster, so they keep the even split.  The math is
  // untouched.
  constexpr bool ASYM = NW == 8 && KSPLIT == 1 && FM * FN >= 9;
  constexpr int NDW = ASYM ? 2 * NDMA : NDMA;  // DMA instructions per issuing wave per tile
  const bool issuer = !ASYM || wave < NW / 2;
  // DMA instruction q (q < DA: A rows, else W rows) of this group's step it
  // into its slot; past the segment it points outside the range and moves
  // nothing.
  auto dma1 = [&](int it, int q) {
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
  // asymmetric issue: instruction q' of issuing wave w covers rows
  // (q' NW/2 + w) RPI .. +RPI-1 of the stacked (A; W) tile, q' < 2 NDMA
  auto dma2 = [&](int it, int q2) {
    char* sb = gsm + (it % STAGES) * STAGE;
    const int kt = kt0 + it * KSPLIT + kg;
    const uint32_t kb = kt < kt1 ? (uint32_t)(kt * BKB) : (uint32_t)kPastEnd;
    const int base = (q2 * (NW / 2) + wave) * RPI;  // wave-uniform
    if (base < BM) {
      const int r = base + lane / CPR;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsa, (lds_void*)(sb + base * BKB), 16,
          (uint32_t)(r * lda * (int64_t)sizeof(T)) + (uint32_t)(((lane % CPR) ^ swz<BKB>(r)) << 4) + kb, 0, 0, 0);
    } else {
      const int r = base - BM + lane / CPR;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsw, (lds_void*)(sb + BM * BKB + (base - BM) * BKB), 16,
          (uint32_t)(r * ldw * (int64_t)sizeof(T)) + (uint32_t)(((lane % CPR) ^ swz<BKB>(r)) << 4) + kb, 0, 0, 0);
    }
  };
  auto dma = [&](int it, int q) {
    if constexpr (ASYM) {
      if (issuer) {
        dma2(it, 2 * q);
        dma2(it, 2 * q + 1);
      }
    } else {
      dma1(it, q);
    }
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
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PRE - 1) * NDW) : "memory");
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
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((STAGES - 2) * NDW) : "memory");  // tile kt+1 landed
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

}  // namespace tjk
