// FlashAttention-2 forward on the packed [B, S, 3, H, hd] QKV buffer.
//
// Computes softmax(Q K^T * scale) V per (batch, head) with an fp32 online
// softmax in base 2, reading Q/K/V in place through strides and writing the
// context as [B*S, H*hd] (head h at columns h*hd ...), the layout the
// out-projection consumes.  Replaces the Triton kernel
// tjkernels/kernels/attention.py:34-125 (launcher :189-226) and, through
// the `lengths` / `key_mask` arguments, the SDPA fallback used for padded
// non-causal and general masks (tjkernels/engine.py:184-203,216-228).
// With `cu_seqlens` the sequences are packed back to back (varlen): batch b
// owns rows cu_seqlens[b] .. cu_seqlens[b+1]-1 of the QKV and output
// buffers, and workgroups past the end of their sequence exit at once.
//
// CDNA4 mapping.  A workgroup is 4 waves; each wave owns NQ blocks of 32
// queries.  Both products are computed transposed so that every per-query
// quantity lives in a single lane:
//     S^T = K Q^T       (MFMA A = K rows from LDS, B = Q held in registers)
//     O^T += V^T P^T    (MFMA A = V^T rows from LDS, B = P from registers)
// In the 32x32 accumulator layout lane l owns column l%32, i.e. one query,
// so the row max/sum of the softmax are in-lane reductions plus a single
// exchange with lane l^32, and the O rescale by exp2(m_old - m_new) is a
// per-lane scalar.  The K rows of each 32-key block are read in an order
// that swaps bits 2 and 3 of the key index; with that order, the eight S^T
// registers a lane feeds into one 16-key PV step cover 8 consecutive keys,
// so the matching V^T fragment is one 16-byte LDS read.  V is transposed
// while it is staged into LDS (pairs of keys packed per 32-bit word).
//
// K/V tiles are 64 keys, double-buffered in LDS with a 16-byte row pad;
// global loads for tile t+1 are issued before the math of tile t.  Causal
// workgroups only visit key tiles up to their last query, and a wave skips
// the math of tiles entirely above its own diagonal.  Workgroups are issued
// longest-first (the last query blocks have the most key tiles).

#include <algorithm>
#include <mutex>

#include "attn_short.h"

namespace tjk {

template <typename T> struct PairPack;
template <> struct PairPack<bf16> {
  // two 8-element rows (keys k, k+1) -> 8 words {row0[e], row1[e]}
  static __device__ __forceinline__ void write(bf16* dst, int ld, uint4 r0, uint4 r1) {
    const uint32_t a[4] = {r0.x, r0.y, r0.z, r0.w};
    const uint32_t b[4] = {r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      // one v_perm_b32 per word: bytes 0-3 select from a, 4-7 from b
      const uint32_t lo = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);  // {a.lo, b.lo}
      const uint32_t hi = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);  // {a.hi, b.hi}
      *reinterpret_cast<uint32_t*>(dst + (2 * w) * ld) = lo;
      *reinterpret_cast<uint32_t*>(dst + (2 * w + 1) * ld) = hi;
    }
  }
};
template <> struct PairPack<f16> {
  static __device__ __forceinline__ void write(f16* dst, int ld, uint4 r0, uint4 r1) {
    PairPack<bf16>::write(reinterpret_cast<bf16*>(dst), ld, r0, r1);
  }
};
template <> struct PairPack<float> {
  static __device__ __forceinline__ void write(float* dst, int ld, uint4 r0, uint4 r1) {
    const uint32_t a[4] = {r0.x, r0.y, r0.z, r0.w};
    const uint32_t b[4] = {r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) *reinterpret_cast<uint2*>(dst + e * ld) = make_uint2(a[e], b[e]);
  }
};

template <typename T, int HDP, int NQ, int KS, bool KEYMASK>
__global__ __launch_bounds__(256 * KS) void flash_fwd_kernel(
    const T* __restrict__ qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh,
    T* __restrict__ out, int64_t ld_out, int B, int S, int H, int hd, float scale_log2,
    int causal, const int32_t* __restrict__ lengths, const uint8_t* __restrict__ key_mask,
    const int32_t* __restrict__ cu_seqlens, int nqb) {
  constexpr int NQW = 4;                // waves per key split (one query group each)
  constexpr int BMQ = NQW * NQ * 32;    // queries per workgroup
  constexpr int BNK = 64;               // keys per tile
  constexpr int VEC = 16 / sizeof(T);   // elements per 16-byte chunk
  constexpr int LDK = HDP + VEC;        // K tile row pitch (elements)
  constexpr int LDV = BNK + VEC;        // V^T tile row pitch (elements)
  constexpr int KC = HDP / 16;          // 16-deep steps along hd
  constexpr int HB = HDP / 32;          // 32-row blocks of hd in O^T
  constexpr int CH = HDP / VEC;         // 16-byte chunks per K/V row
  constexpr int KITEMS = BNK * CH;      // K chunks per tile
  constexpr int VITEMS = (BNK / 2) * CH;  // (key pair, chunk) items per tile
  static_assert(KITEMS % 256 == 0, "K tile must split evenly over 256 threads");

  __shared__ __attribute__((aligned(16))) T sK[2][KS][BNK * LDK];
  __shared__ __attribute__((aligned(16))) T sV[2][KS][HDP * LDV];

  const int BH = B * H;
  const int rank = blockIdx.x / BH, bh = blockIdx.x % BH;
  const int qb = causal ? nqb - 1 - rank : rank;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  // Key split: waves qw and qw + NQW*p share query group qw; split p takes
  // key tiles p, p + KS, p + 2 KS, ...; the ltid-th thread of each split
  // stages that split's tiles.
  const int qw = wave % NQW, par = wave / NQW, ltid = tid & 255;

  // Sequence b: its tokens are rows row0 .. row0 + Sb - 1 (packed varlen
  // layout when cu_seqlens is given, else b*S .. b*S + S - 1).
  int Sb = S;
  int64_t row0 = (int64_t)b * S, boff = (int64_t)b * sb;
  if (cu_seqlens != nullptr) {
    row0 = max(cu_seqlens[b], 0);
    Sb = min(max(cu_seqlens[b + 1] - cu_seqlens[b], 0), S);  // bounded by the launch's sequence length
    boff = row0 * ss;
  }
  const T* qbase = qkv + boff + (int64_t)h * sh;
  const T* kbase = qbase + sc;
  const T* vbase = qbase + 2 * sc;

  int kv_len = Sb;
  if (lengths != nullptr) kv_len = min(kv_len, max(lengths[b], 0));
  const int q0 = qb * BMQ;
  const int wq0 = q0 + qw * NQ * 32;
  if (q0 >= Sb) return;  // the whole workgroup: past this sequence's end
  int kend = causal ? min(q0 + BMQ, Sb) : Sb;
  kend = min(kend, kv_len);
  const int nkt = (kend + BNK - 1) / BNK;
  const int nit = (nkt + KS - 1) / KS;  // iterations of KS tiles

  // ---- Q fragments (B operand of S^T): lane holds Q[q][16c + 8*hi + 0..7]
  typename Mfma<T>::frag qf[NQ][KC];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int q = wq0 + j * 32 + l32;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int col = 16 * c + 8 * hi;
      if (q < Sb && col < hd) {
        qf[j][c] = Mfma<T>::load(qbase + (int64_t)q * ss + col);
      } else {
        float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        qf[j][c] = Mfma<T>::pack(z);
      }
    }
  }

  // ---- staging of one K/V tile through registers
  constexpr int KPT = KITEMS / 256;
  constexpr int VPT = (VITEMS + 255) / 256;
  uint4 rk[KPT], rv0[VPT], rv1[VPT];
  auto load_kv = [&](int it) {
    const int k0 = (it * KS + par) * BNK;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int it = ltid + i * 256, key = it / CH, c = it % CH;
      const int gk = k0 + key, col = c * VEC;
      rk[i] = (gk < Sb && col < hd) ? *reinterpret_cast<const uint4*>(kbase + (int64_t)gk * ss + col)
                                  : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int it = ltid + i * 256;
      const int p = it % (BNK / 2), c = it / (BNK / 2);
      const int gk = k0 + 2 * p, col = c * VEC;
      const bool ok = it < VITEMS && col < hd;
      rv0[i] = (ok && gk < Sb) ? *reinterpret_cast<const uint4*>(vbase + (int64_t)gk * ss + col)
                              : make_uint4(0, 0, 0, 0);
      rv1[i] = (ok && gk + 1 < Sb) ? *reinterpret_cast<const uint4*>(vbase + (int64_t)(gk + 1) * ss + col)
                                  : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int it = ltid + i * 256, key = it / CH, c = it % CH;
      *reinterpret_cast<uint4*>(&sK[buf][par][key * LDK + c * VEC]) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int it = ltid + i * 256;
      if (it < VITEMS) {
        const int p = it % (BNK / 2), c = it / (BNK / 2);
        PairPack<T>::write(&sV[buf][par][(c * VEC) * LDV + 2 * p], LDV, rv0[i], rv1[i]);
      }
    }
  };

  f32x16 o[NQ][HB];
  float m_run[NQ], l_run[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[j][hb][r] = 0.f;
  }

  if (nit > 0) {
    load_kv(0);
    store_kv(0);
  }
  __syncthreads();

  const int krow = swap_bits_2_3(l32);  // K row this lane feeds into S^T
  for (int itr = 0; itr < nit; ++itr) {
    const int cur = itr & 1;
    if (itr + 1 < nit) load_kv(itr + 1);
    const int kt = itr * KS + par;
    const int k0 = kt * BNK;
    const bool wave_active = kt < nkt && (!causal || k0 <= wq0 + NQ * 32 - 1);
    if (wave_active) {
      // ---- S^T = K Q^T for two 32-key blocks
      f32x16 s[NQ][2];
#pragma unroll
      for (int j = 0; j < NQ; ++j)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[j][kb][r] = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const T* kp = &sK[cur][par][(kb * 32 + krow) * LDK + 8 * hi];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const typename Mfma<T>::frag kf = Mfma<T>::load(kp + 16 * c);
#pragma unroll
          for (int j = 0; j < NQ; ++j) Mfma<T>::mma(s[j][kb], kf, qf[j][c]);
        }
      }

      // ---- masking: register r of block kb is key k0 + kb*32 + 16*(r/8) + 8*hi + r%8.
      // Selects, not branches; only tiles that straddle the causal diagonal
      // or the end of the keys pay for them (a wave-uniform test).
      const bool tail = k0 + BNK > kend;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int q = wq0 + j * 32 + l32;
        const bool diag = causal && k0 + BNK - 1 > wq0 + j * 32;
        if (tail || diag) {
          const int lim = causal ? min(q + 1, kend) : kend;  // keys < lim are admissible
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = k0 + kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7);
              s[j][kb][r] = key < lim ? s[j][kb][r] : -INFINITY;
            }
        }
        if constexpr (KEYMASK) {
          // every mask byte loaded before any is used (a load under the
          // key < kend condition would be waited for on its own)
          uint8_t km[2][16];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              km[kb][r] = key_mask[(int64_t)b * S + min(k0 + kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7), S - 1)];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = k0 + kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7);
              const bool keep = key < kend && km[kb][r] != 0;
              s[j][kb][r] = keep ? s[j][kb][r] : -INFINITY;
            }
        }
      }

      // ---- online softmax (base 2) and P fragments.  The O rescale is
      // skipped when no lane's running max moved (alpha == 1 everywhere),
      // which is the common case once a row has seen its largest scores.
      typename Mfma<T>::frag pf[NQ][4];
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[j][kb][r]);
        {  // lanes l and l^32 hold the two halves of a query's keys
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
          mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const float m_new = fmaxf(m_run[j], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new * scale_log2;
        const float alpha = __builtin_amdgcn_exp2f(m_run[j] * scale_log2 - m_use);
        float rs = 0.f;
        float p[2][16];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            p[kb][r] = __builtin_amdgcn_exp2f(fmaf(s[j][kb][r], scale_log2, -m_use));
            rs += p[kb][r];
          }
        l_run[j] = l_run[j] * alpha + rs;
        m_run[j] = m_new;
        if (__any(alpha != 1.0f)) {
#pragma unroll
          for (int hb = 0; hb < HB; ++hb)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][hb][r] *= alpha;
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) pf[j][st] = Mfma<T>::pack(&p[st >> 1][8 * (st & 1)]);
      }

      // ---- O^T += V^T P^T: 16-key step st covers keys 16*st + 8*hi + 0..7
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        const T* vp = &sV[cur][par][(hb * 32 + l32) * LDV + 8 * hi];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const typename Mfma<T>::frag vf = Mfma<T>::load(vp + 16 * st);
#pragma unroll
          for (int j = 0; j < NQ; ++j) Mfma<T>::mma(o[j][hb], vf, pf[j][st]);
        }
      }
    }
    if (itr + 1 < nit) store_kv(cur ^ 1);
    __syncthreads();
  }

  // ---- merge the key splits: split p > 0 leaves its running max, partial
  // sums and O^T in LDS (the tiles are dead after the loop's last barrier);
  // split 0 rescales both to the common max and adds.
  if constexpr (KS > 1) {
    constexpr int OW = NQ * HB * 16 * 64;  // O^T floats per wave
    constexpr int SW = OW + 2 * NQ * 64;   // + running max and sum
    static_assert(NQW * (KS - 1) * SW * 4 <= (int)sizeof(sK), "split merge exceeds the K tiles' LDS");
    float* xo = reinterpret_cast<float*>(&sK[0][0][0]);
    if (par > 0) {
      float* my = xo + ((par - 1) * NQW + qw) * SW;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
#pragma unroll
        for (int hb = 0; hb < HB; ++hb)
#pragma unroll
          for (int r = 0; r < 16; ++r) my[((j * HB + hb) * 16 + r) * 64 + lane] = o[j][hb][r];
        my[OW + j * 64 + lane] = m_run[j];
        my[OW + NQ * 64 + j * 64 + lane] = l_run[j];
      }
    }
    __syncthreads();
    if (par > 0) return;
#pragma unroll
    for (int p = 1; p < KS; ++p) {
      const float* ot = xo + ((p - 1) * NQW + qw) * SW;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const float m2 = ot[OW + j * 64 + lane], l2 = ot[OW + NQ * 64 + j * 64 + lane];
        const float m = fmaxf(m_run[j], m2);
        const float a1 = m_run[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_run[j] - m) * scale_log2);
        const float a2 = m2 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m2 - m) * scale_log2);
        l_run[j] = l_run[j] * a1 + l2 * a2;
        m_run[j] = m;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            o[j][hb][r] = o[j][hb][r] * a1 + ot[((j * HB + hb) * 16 + r) * 64 + lane] * a2;
      }
    }
  }

  // ---- normalise and store: register r of block hb is hd row hb*32 + 8*(r/4) + 4*hi + r%4
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int q = wq0 + j * 32 + l32;
    const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run[j]), __float_as_uint(l_run[j]), false, false);
    const float l = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    if (q >= Sb) continue;
    T* orow = out + (row0 + q) * ld_out + (int64_t)h * hd;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = hb * 32 + 8 * g + 4 * hi;
        if (col < hd) {
          const float4 v = make_float4(o[j][hb][4 * g] * inv, o[j][hb][4 * g + 1] * inv,
                                       o[j][hb][4 * g + 2] * inv, o[j][hb][4 * g + 3] * inv);
          *reinterpret_cast<typename Quad<T>::raw*>(orow + col) = Quad<T>::from(v);
        }
      }
  }
}

// ------------------------------------------------ short sequences (plan 4)
//
// Every key of a sequence of at most 128 tokens fits one workgroup: a
// one-wave workgroup takes 32 queries of one (b, h), stages the K rows it
// needs and their V rows (transposed) into LDS in one round of loads, and
// computes S^T = K Q^T over all of its keys at once, an exact softmax (one
// row max, no running rescale) and O^T = V^T P^T.  The grid is
// B * H * ceil(S / 32) workgroups -- four times plan 1's at S = 128 -- and
// each workgroup waits for memory once before its math; plan 1 at C2's
// 1 x 128 x 8 heads spends ~2 us loading and ~2.6 us in two masked
// key-tile iterations on 8 workgroups.
template <typename T, int HDP, bool KEYMASK>
__global__ __launch_bounds__(64) void flash_short_kernel(
    const T* __restrict__ qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh,
    T* __restrict__ out, int64_t ld_out, int B, int S, int H, int hd, float scale_log2,
    int causal, const int32_t* __restrict__ lengths, const uint8_t* __restrict__ key_mask,
    const int32_t* __restrict__ cu_seqlens, int nqb) {
  constexpr int MAXK = 128;                // keys per sequence
  constexpr int VEC = 16 / sizeof(T);      // elements per 16-byte chunk
  constexpr int LDK = HDP + VEC;           // K row pitch (elements)
  constexpr int LDV = MAXK + VEC;          // V^T row pitch (elements)
  constexpr int KC = HDP / 16, HB = HDP / 32, CH = HDP / VEC;
  constexpr int KPL = MAXK * CH / 64;      // K chunks per lane
  constexpr int VPL = (MAXK / 2) * CH / 64;  // (key pair, chunk) items per lane
  typedef typename Mfma<T>::frag Frag;

  __shared__ __attribute__((aligned(16))) T sK[MAXK * LDK];
  __shared__ __attribute__((aligned(16))) T sV[HDP * LDV];

  const int BH = B * H;
  const int rank = blockIdx.x / BH, bh = blockIdx.x % BH;
  const int qb = causal ? nqb - 1 - rank : rank;  // causal: most keys first
  const int b = bh / H, h = bh % H;
  const int lane = threadIdx.x, l32 = lane & 31, hi = lane >> 5;

  int Sb = S;
  int64_t row0 = (int64_t)b * S, boff = (int64_t)b * sb;
  if (cu_seqlens != nullptr) {
    row0 = max(cu_seqlens[b], 0);
    Sb = min(max(cu_seqlens[b + 1] - cu_seqlens[b], 0), S);  // bounded by the launch's sequence length
    boff = row0 * ss;
  }
  const T* qbase = qkv + boff + (int64_t)h * sh;
  const T* kbase = qbase + sc;
  const T* vbase = qbase + 2 * sc;
  int kv_len = Sb;
  if (lengths != nullptr) kv_len = min(kv_len, max(lengths[b], 0));
  const int q0 = qb * 32;
  if (q0 >= Sb) return;
  int kend = causal ? min(q0 + 32, Sb) : Sb;
  kend = min(kend, kv_len);  // keys >= kend are never admissible (and never read)
  const int nkb = (kend + 31) / 32;

  // Every load below is unconditional, at an index clamped into the
  // sequence (row 0 exists: q0 < Sb), and its value replaced by zeros where
  // it lies outside: a load under a per-lane condition is waited for on its
  // own, one memory round trip per load.
  // Q fragments (B operand of S^T): lane holds Q[q][16c + 8*hi + 0..7]
  const int q = q0 + l32;
  const T* qrow = qbase + (int64_t)min(q, Sb - 1) * ss;
  Frag qf[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c) qf[c] = Mfma<T>::load(qrow + min(16 * c + 8 * hi, hd - 8));
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    if (!(q < Sb && 16 * c + 8 * hi < hd)) {
      float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      qf[c] = Mfma<T>::pack(z);
    }
  }
  // K rows and V rows (two keys per item) of keys < kend, zeros past it:
  // every LDS word the math reads is written.
  const int klast = max(kend - 1, 0);
  uint4 rk[KPL], rv0[VPL], rv1[VPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int it = lane + i * 64, key = it / CH, col = (it % CH) * VEC;
    rk[i] = *reinterpret_cast<const uint4*>(kbase + (int64_t)min(key, klast) * ss + min(col, hd - VEC));
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int it = lane + i * 64, p = it % (MAXK / 2), col = min((it / (MAXK / 2)) * VEC, hd - VEC);
    rv0[i] = *reinterpret_cast<const uint4*>(vbase + (int64_t)min(2 * p, klast) * ss + col);
    rv1[i] = *reinterpret_cast<const uint4*>(vbase + (int64_t)min(2 * p + 1, klast) * ss + col);
  }
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int it = lane + i * 64, key = it / CH, col = (it % CH) * VEC;
    if (!(key < kend && col < hd)) rk[i] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int it = lane + i * 64, p = it % (MAXK / 2), col = (it / (MAXK / 2)) * VEC;
    if (!(col < hd && 2 * p < kend)) rv0[i] = make_uint4(0, 0, 0, 0);
    if (!(col < hd && 2 * p + 1 < kend)) rv1[i] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int it = lane + i * 64, key = it / CH, c = it % CH;
    *reinterpret_cast<uint4*>(&sK[key * LDK + c * VEC]) = rk[i];
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int it = lane + i * 64, p = it % (MAXK / 2), c = it / (MAXK / 2);
    PairPack<T>::write(&sV[(c * VEC) * LDV + 2 * p], LDV, rv0[i], rv1[i]);
  }
  __syncthreads();

  // exact softmax over the resident keys (math shared with tjk_attn_block)
  const int lim = causal ? min(q + 1, kend) : kend;
  f32x16 o[HB];
  const float inv = short_attention<T, HDP, MAXK>(
      sK, sV, qf, nkb, lim, scale_log2,
      [&](int key) { return !KEYMASK || key_mask[(int64_t)b * S + min(key, S - 1)] != 0; }, o);
  if (q >= Sb) return;
  T* orow = out + (row0 + q) * ld_out + (int64_t)h * hd;
#pragma unroll
  for (int hb = 0; hb < HB; ++hb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = hb * 32 + 8 * g + 4 * hi;
      if (col < hd) {
        const float4 v = make_float4(o[hb][4 * g] * inv, o[hb][4 * g + 1] * inv, o[hb][4 * g + 2] * inv,
                                     o[hb][4 * g + 3] * inv);
        *reinterpret_cast<typename Quad<T>::raw*>(orow + col) = Quad<T>::from(v);
      }
    }
}

// ------------------------------------------------ software-pipelined variant
//
// Same math and output as flash_fwd_kernel (one 32-query block per wave),
// for 2-byte types, with the per-tile dependency chain
//     S = K Q^T  ->  softmax(S)  ->  O += V P
// broken across tiles: the MFMAs of S for tile t+1 are issued before the
// softmax of tile t, so the matrix cores work while the VALU does the
// softmax.  That needs K of tile t+1 resident while V of tile t is still
// read, so K/V tiles live in a 4-deep LDS ring; the global loads of tile
// t+3 go out at the start of iteration t.  K/V are read through per-tile
// buffer descriptors that end at this head's last key, so keys past S
// arrive as 0 without a bounds branch.  Tiles that need no masking (every
// key below the workgroup's first query and inside the sequence) run a
// loop unrolled over the ring, whose LDS slots are then compile-time
// offsets; the diagonal / tail tiles run a second loop with masks and
// per-wave skips.

// Cache-policy bits of buffer loads / stores (sc0 = 1, sc1 = 16): sc1 makes
// an access device-coherent, sc0 sc1 on a store writes through to memory.
constexpr int kFaSc1 = 16, kFaSc0Sc1 = 17;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kFaSpinLimit = 1 << 20;  // polls of a split item's flag before giving up (>= 0.1 s)

// Buffer descriptor over `bytes` bytes at p (stride 0, raw dword access).
__device__ __forceinline__ u32x4 fa_rsrc(const void* p, int bytes) {
  const uint64_t a = (uint64_t)p;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, (uint32_t)bytes, 0x00020000u};
}
// One LDS DMA: each lane copies 16 bytes at voff of the descriptor's range to
// LDS byte lds_addr + 16 * lane.  Issued as inline asm so that the compiler
// does not track it: for an LDS read it cannot tell apart from a DMA's
// destination (the transposing ds_read_b64_tr_b16 carries no alias
// information) it would otherwise wait for every copy in flight.  The ring's
// own s_waitcnt vmcnt + s_barrier order the copies against the reads.
__device__ __forceinline__ void fa_lds_dma16(u32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds_addr));
}

// NW waves per workgroup own BMQ = 32 NW queries.  NW = 4 (two workgroups
// per CU at head_dim <= 64, one above).  NW = 8 is the head_dim-128 grid
// variant: the LDS ring (143 KB) allows one workgroup per CU, so 8 waves
// put two waves on each SIMD where 4 would leave one -- the second wave's
// MFMAs and softmax fill the first one's stalls, and every K / V tile staged
// into LDS serves 256 queries instead of 128.  Its K and V fragments are
// read just before use (in two halves for S) to stay within the 256
// registers two waves per SIMD leave each wave.
template <typename T, int HDP, bool KEYMASK, bool FULLHD, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(HDP <= 64 || NW == 8 ? 2 : 1, HDP <= 64 || NW == 8 ? 2 : 1))) void flash_pipe_kernel(
    const T* __restrict__ qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh,
    T* __restrict__ out, int64_t ld_out, int B, int S, int H, int hd, float scale_log2,
    int causal, const int32_t* __restrict__ lengths, const uint8_t* __restrict__ key_mask,
    const int32_t* __restrict__ cu_seqlens, int nqb,
    const int4* __restrict__ work, int n_work, float* __restrict__ partials, int* __restrict__ flags, int n_slots,
    int grp) {
  static_assert(sizeof(T) == 2, "2-byte element types only");
  static_assert(NW == 4 || (NW == 8 && HDP == 128), "8 waves for head_dim 128 only");
  constexpr int NT = 64 * NW, BMQ = 32 * NW, BNK = 64, NST = 4, VEC = 8;
  constexpr bool LEAN = NW == 8;  // fragments read just before use
  constexpr int LDK = HDP + VEC, LDV = BNK + VEC;
  constexpr int KC = HDP / 16, HB = HDP / 32, CH = HDP / VEC;
  constexpr int KITEMS = BNK * CH, VITEMS = (BNK / 2) * CH;
  constexpr int KPT = KITEMS / NT, VPT = (VITEMS + NT - 1) / NT;
  static_assert(KITEMS % NT == 0, "K tile must split evenly over the threads");

  // K / V ring.  DMA (head_dim 64 / 128 with the full head dimension, no
  // key mask): tiles are copied straight into LDS by buffer_load ... lds, K
  // and V both key-major with 128- / 256-byte rows whose 16-byte chunks are
  // XOR-swizzled by row, and V^T fragments are gathered with the transposing
  // ds_read_b64_tr_b16.  Otherwise tiles pass through registers, V stored
  // transposed.
  constexpr bool DMA = FULLHD && !KEYMASK && HDP >= 64;
  constexpr int RB = HDP * (int)sizeof(T);  // DMA: bytes per K / V row
  constexpr int CPR = RB / 16, RPI = 64 / CPR, TILE_B = BNK * RB;
  char* smem;  // DMA ring: slot st holds K at st * 2 TILE_B, V TILE_B later
  T (*sK)[BNK * LDK];
  T (*sV)[HDP * LDV];
  int* s_flag;  // the split-item merge's published flag
  if constexpr (DMA) {
    __shared__ __attribute__((aligned(1024))) char ring[NST * 2 * TILE_B + 16];
    smem = ring;
    sK = nullptr;
    sV = nullptr;
    s_flag = reinterpret_cast<int*>(ring + NST * 2 * TILE_B);
  } else {
    __shared__ __attribute__((aligned(16))) T k_ring[NST][BNK * LDK];
    __shared__ __attribute__((aligned(16))) T v_ring[NST][HDP * LDV];
    __shared__ int flag;
    smem = nullptr;
    sK = k_ring;
    sV = v_ring;
    s_flag = &flag;
  }

  const int BH = B * H;
  // One work item: query block qb of (b, h) = bh over key tiles [t_lo,
  // t_hi).  slot -1: a whole item; slot s >= 0: the first half of a
  // key-split item, which publishes its partial in slot s; slot -2 - s: the
  // second half, which merges partial s into its own before the store.
  // bad_slot: the listed slot was outside [0, n_slots) (the rows are written
  // as NaN and counted).
  auto run_item = [&](int bh, int qb, int t_lo, int t_hi, int slot, bool bad_slot) __attribute__((always_inline)) {
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;

  // Sequence b: its tokens are rows row0 .. row0 + Sb - 1 (packed varlen
  // layout when cu_seqlens is given, else b*S .. b*S + S - 1).
  int Sb = S;
  int64_t row0 = (int64_t)b * S, boff = (int64_t)b * sb;
  if (cu_seqlens != nullptr) {
    row0 = max(cu_seqlens[b], 0);
    Sb = min(max(cu_seqlens[b + 1] - cu_seqlens[b], 0), S);  // bounded by the launch's sequence length
    boff = row0 * ss;
  }
  const T* qbase = qkv + boff + (int64_t)h * sh;
  int kv_len = Sb;
  if (lengths != nullptr) kv_len = min(kv_len, max(lengths[b], 0));
  const int q0 = qb * BMQ;
  const int wq0 = q0 + wave * 32;
  if (q0 >= Sb) return;  // the whole workgroup: past this sequence's end
  int kend = causal ? min(q0 + BMQ, Sb) : Sb;
  kend = min(kend, kv_len);
  const int nkt = (kend + BNK - 1) / BNK;
  t_hi = min(t_hi, nkt);

  // Q fragments (B operand of S^T): lane holds Q[q][16c + 8*hi + 0..7]
  typename Mfma<T>::frag qf[KC];
  {
    const int q = wq0 + l32;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int col = 16 * c + 8 * hi;
      if (q < Sb && (FULLHD || col < hd)) {
        qf[c] = Mfma<T>::load(qbase + (int64_t)q * ss + col);
      } else {
        float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        qf[c] = Mfma<T>::pack(z);
      }
    }
  }

  // K / V rows of this (b, h): the span from key 0 to the end of key Sb-1.
  // Tile t is read through a descriptor starting at its first key (scalar
  // work), so the per-lane offsets stay fixed across tiles; a tile past the
  // item's range gets an empty descriptor and reads as zeros.
  const uint32_t row_bytes = (uint32_t)(ss * (int64_t)sizeof(T));
  const int span = (int)(((int64_t)(Sb - 1) * ss + hd) * (int64_t)sizeof(T));
  uint4 rk[KPT], rv0[VPT], rv1[VPT];
  auto load_kv_into = [&](int t, uint4 (&rk)[KPT], uint4 (&rv0)[VPT], uint4 (&rv1)[VPT]) __attribute__((always_inline)) {
    const int64_t t_elems = (int64_t)t * BNK * ss;
    const int nrec = t < t_hi ? span - (int)(t_elems * (int64_t)sizeof(T)) : 0;
    const __amdgpu_buffer_rsrc_t rsk =
        __builtin_amdgcn_make_buffer_rsrc((void*)(qbase + sc + t_elems), (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsv =
        __builtin_amdgcn_make_buffer_rsrc((void*)(qbase + 2 * sc + t_elems), (short)0, nrec, 0x00020000);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int it = tid + i * NT, key = it / CH, c = it % CH;
      const uint32_t off = (uint32_t)key * row_bytes + (uint32_t)(c * 16);
      uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsk, off, 0, 0));
      rk[i] = (FULLHD || c * VEC < hd) ? v : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int it = tid + i * NT;
      const int p = it % (BNK / 2), c = it / (BNK / 2);
      const uint32_t off = (uint32_t)(2 * p) * row_bytes + (uint32_t)(c * 16);
      uint4 v0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsv, off, 0, 0));
      uint4 v1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsv, off + row_bytes, 0, 0));
      const bool ok = FULLHD || c * VEC < hd;
      rv0[i] = ok ? v0 : make_uint4(0, 0, 0, 0);
      rv1[i] = ok ? v1 : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_kv_from = [&](int st, uint4 (&rk)[KPT], uint4 (&rv0)[VPT], uint4 (&rv1)[VPT]) {
    // the loads landed a step ago; pinning the registers here keeps the V
    // transposition (v_perm) from being hoisted into the step that issued
    // the loads, where it would wait for them
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      u32x4 a = __builtin_bit_cast(u32x4, rv0[i]), c = __builtin_bit_cast(u32x4, rv1[i]);
      asm volatile("" : "+v"(a), "+v"(c));
      rv0[i] = __builtin_bit_cast(uint4, a);
      rv1[i] = __builtin_bit_cast(uint4, c);
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int it = tid + i * NT, key = it / CH, c = it % CH;
      *reinterpret_cast<uint4*>(&sK[st][key * LDK + c * VEC]) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int it = tid + i * NT;
      if (VITEMS % NT == 0 || it < VITEMS) {
        const int p = it % (BNK / 2), c = it / (BNK / 2);
        PairPack<T>::write(&sV[st][(c * VEC) * LDV + 2 * p], LDV, rv0[i], rv1[i]);
      }
    }
  };
  auto load_kv = [&](int t) __attribute__((always_inline)) { load_kv_into(t, rk, rv0, rv1); };
  auto store_kv = [&](int st) __attribute__((always_inline)) { store_kv_from(st, rk, rv0, rv1); };

  // DMA path: chunk c of row r sits at physical chunk c ^ swz(r).  With row
  // bits r0..r3, swz = r1 | r3 << 1 | (r1 ^ r2) << 2 at 8 chunks per row and
  // r0 | r1 << 1 | (r0 ^ r2) << 2 | (r1 ^ r3) << 3 at 16.  Both spread
  // the K fragment reads (16 lanes, rows 0..15 of a block, one logical chunk)
  // over all 64 banks.  They also spread each half-wave of a transposing V
  // read (4 consecutive rows, 64 bytes of each): the rows' 64-byte blocks
  // land in distinct bank ranges (the row-major swizzle r & 15 gave 4-way
  // conflicts there, 6 extra cycles per read at 16 chunks, 2 at 8).
  // DMA instruction q of this wave fills the 1 KB block q*NW + wave of a
  // tile: rows (q*NW + wave)*RPI + lane/CPR, lane's chunk landing at byte
  // 16*lane, so it fetches logical chunk (lane % CPR) ^ swz(row).
  constexpr int NDK = DMA ? TILE_B / 1024 / NW : 1;  // DMA instructions per wave per K (or V) tile
  constexpr int NDT = 2 * NDK;                      // ... per K + V tile
  static_assert(!DMA || NDK * 1024 * NW == TILE_B, "K / V tile must split over the waves");
  auto swz = [](int r) __attribute__((always_inline)) {
    const int r0 = r & 1, r1 = (r >> 1) & 1, r2 = (r >> 2) & 1, r3 = (r >> 3) & 1;
    return CPR == 8 ? (r1 | (r3 << 1) | ((r1 ^ r2) << 2)) : (r0 | (r1 << 1) | ((r0 ^ r2) << 2) | ((r1 ^ r3) << 3));
  };
  uint32_t dvoff[NDK];
  const uint32_t lds_ring = (uint32_t)(uintptr_t)(lds_void*)smem;
#pragma unroll
  for (int q = 0; q < NDK; ++q) {
    const int r = (q * NW + wave) * RPI + lane / CPR;
    dvoff[q] = (uint32_t)r * row_bytes + (uint32_t)(((lane % CPR) ^ swz(r)) << 4);
  }
  // K and V of key tile t into ring slot st (a tile past the item's range
  // gets an empty descriptor and moves nothing)
  auto dma_kv = [&](int t, int st) __attribute__((always_inline)) {
    const int64_t t_elems = (int64_t)t * BNK * ss;
    const int nrec = t < t_hi ? span - (int)(t_elems * (int64_t)sizeof(T)) : 0;
    const u32x4 rsk = fa_rsrc(qbase + sc + t_elems, nrec), rsv = fa_rsrc(qbase + 2 * sc + t_elems, nrec);
    const uint32_t kb = lds_ring + (uint32_t)(st * 2 * TILE_B + wave * 1024);
#pragma unroll
    for (int q = 0; q < NDK; ++q) fa_lds_dma16(rsk, dvoff[q], kb + q * NW * 1024);
#pragma unroll
    for (int q = 0; q < NDK; ++q) fa_lds_dma16(rsv, dvoff[q], kb + TILE_B + q * NW * 1024);
  };
  // end of a ring step: this wave's copies of the tile two ahead have landed
  // (only the newest tile's may still be in flight) and its LDS reads are
  // done, then everyone's
  auto step_barrier = [&]() __attribute__((always_inline)) {
    if constexpr (DMA) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(NDT) : "memory");
      asm volatile("s_barrier" ::: "memory");
    } else {
      __syncthreads();
    }
  };
  typedef typename Mfma<T>::frag FragT;
  // K fragment: row `row` of slot st, 16-byte chunk `ch` (8 head-dim elements)
  auto kfrag = [&](int st, int row, int ch) __attribute__((always_inline)) -> FragT {
    if constexpr (DMA)
      return *reinterpret_cast<const FragT*>(smem + st * 2 * TILE_B + row * RB + ((ch ^ swz(row)) << 4));
    else
      return Mfma<T>::load(&sK[st][row * LDK + 8 * ch]);
  };
  // V^T fragment of the PV product: lane (l32, hi) gets V[keys 16 stp + 8 hi
  // + 0..7][head-dim row hb*32 + l32].  DMA: two transposing reads of four
  // keys each; in a group of 16 lanes, source lane s points at key
  // kbase + s/4, head-dim elements c0 + 4 (s%4) .. +3, and lane i receives
  // keys kbase + 0..3 of element c0 + i.  Read rd of step stp in block hb:
  // key 16 stp + 8 hi + 4 rd + g (g = (lane & 15) / 4 = g0 + 2 g1), element
  // hb*32 + 16 b4 + 4 (lane & 3) (b4 = (lane >> 4) & 1), i.e. chunk
  // ch = 4 hb + 2 b4 + b1 (b1 = (lane & 3) >> 1), 8-byte half lane & 1.  In
  // ch ^ swz(key) the bits below 2 depend on the lane only, and the bits from
  // 2 up are c ^ x, c = hb ^ rd for every lane and x a per-lane value, so the
  // address is one of HB per-lane bases (by c) plus a compile-time offset.
  const int vg = (lane & 15) >> 2, g0 = vg & 1, g1 = vg >> 1;
  const int b4 = (lane >> 4) & 1, b1 = (lane & 3) >> 1;
  const int vlow = CPR == 8 ? ((b1 ^ g1) | ((b4 ^ hi) << 1)) : ((b1 ^ g0) | ((b4 ^ g1) << 1));
  const int vx = CPR == 8 ? g1 : (g0 | ((g1 ^ hi) << 1));
  const int vlb = (8 * hi + vg) * RB + 16 * vlow + 8 * (lane & 1);
  int vlane[HB];
#pragma unroll
  for (int c = 0; c < HB; ++c) vlane[c] = vlb + 64 * (c ^ vx);
  auto vfrag = [&](int st, int hb, int stp) __attribute__((always_inline)) -> FragT {
    if constexpr (DMA) {
      typedef short v4s __attribute__((ext_vector_type(4)));
      const char* vb = smem + st * 2 * TILE_B + TILE_B;
      v4s part[2];
#pragma unroll
      for (int rd = 0; rd < 2; ++rd) {
        const int c = hb ^ rd;
        part[rd] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s*)(vb + (16 * stp + 4 * rd) * RB + vlane[c]));
      }
      typedef short v8s __attribute__((ext_vector_type(8)));
      const v8s both = {part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
      return __builtin_bit_cast(FragT, both);
    } else {
      return Mfma<T>::load(&sV[st][(hb * 32 + l32) * LDV + 8 * hi] + 16 * stp);
    }
  };
  // ring slot of key tile tt (slot 0 holds the item's first tile)
  auto slot_of = [&](int tt) { return (tt - t_lo) & (NST - 1); };

  const int krow = swap_bits_2_3(l32);
  auto qk = [&](int st, f32x16 (&sa)[2]) {
    // all K fragment reads of the tile first, then the MFMAs, so the reads'
    // LDS latency overlaps instead of being waited out before every MFMA
    typename Mfma<T>::frag kf[2][KC];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int c = 0; c < KC; ++c) kf[kb][c] = kfrag(st, kb * 32 + krow, 2 * c + hi);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sa[kb][r] = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) Mfma<T>::mma(sa[kb], kf[kb][c], qf[c]);
  };

  f32x16 o[HB];
#pragma unroll
  for (int hb = 0; hb < HB; ++hb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[hb][r] = 0.f;
  // m_off: the exponent offset (log2 units) the running O and l are taken
  // relative to.  It is raised only when a query's scores exceed it by more
  // than kLazyRescale, so most tiles skip the O rescale; p <= 2^kLazyRescale
  // is harmless in fp32 and in the 2-byte P.
  constexpr float kLazyRescale = 8.0f;
  float m_off = -INFINITY, l_run = 0.f;

  // softmax of one tile's scores (already masked) and O += V P
  auto softmax_pv = [&](int st, f32x16 (&sa)[2]) {
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sa[kb][r]);
    {  // both lanes of a query agree (lane l and l^32 swap through v_permlane32_swap)
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale_log2;
    }
    if (__any(mx > m_off + kLazyRescale)) {
      const float m_new = fmaxf(m_off, mx);
      const float alpha = m_off == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_off - m_new);
      l_run *= alpha;
#pragma unroll
      for (int hb = 0; hb < HB; ++hb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[hb][r] *= alpha;
      m_off = m_new;
    }
    const float base = m_off == -INFINITY ? 0.f : m_off;
    float p[2][16];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) p[kb][r] = __builtin_amdgcn_exp2f(fmaf(sa[kb][r], scale_log2, -base));
    typename Mfma<T>::frag pf[4];
#pragma unroll
    for (int stp = 0; stp < 4; ++stp) pf[stp] = Mfma<T>::pack(&p[stp >> 1][8 * (stp & 1)]);
    // row sums of the rounded P (exactly the weights the PV product uses),
    // two per instruction
#pragma unroll
    for (int stp = 0; stp < 4; ++stp) l_run = Mfma<T>::sum8(pf[stp], l_run);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int stp = 0; stp < 4; ++stp) Mfma<T>::mma(o[hb], vfrag(st, hb, stp), pf[stp]);
  };

  // register r of block kb is key k0 + kb*32 + 16*(r/8) + 8*hi + r%8
  auto mask_tile = [&](int t, f32x16 (&sa)[2]) {
    const int k0 = t * BNK, q = wq0 + l32;
    const int lim = causal ? min(q + 1, kend) : kend;
    // mask bytes all loaded before any is used (see flash_fwd_kernel)
    uint8_t km[2][16];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        km[kb][r] = KEYMASK ? key_mask[(int64_t)b * S + min(k0 + kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7), S - 1)]
                            : 1;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7);
        const bool keep = key < lim && km[kb][r] != 0;
        sa[kb][r] = keep ? sa[kb][r] : -INFINITY;
      }
  };

  // ---- interior-tile pipeline (unmasked tiles).  The exponentials of tile
  // t run while the MFMAs of S(t+1) run, so the VALU-heavy stretch of each
  // step has MFMAs to hide behind (and the other wave of the SIMD finds the
  // matrix pipe busy in the opposite phase, the PV product).  No row max is
  // taken: P = 2^(S * scale - m_off) is formed with the running offset, and
  // only when a lane's share of a query's tile sum exceeds kSumLimit (which
  // bounds every P of the tile; a first tile, with m_off = -inf, gives inf)
  // is the tile redone with m_off raised to the row max.  Every P the PV
  // product sees is therefore <= kSumLimit.
  typedef typename Mfma<T>::frag Frag;
  constexpr float kSumLimit = 4096.0f;
  // row max of a tile's scores in log2 units; both lanes of a query agree
  auto rowmax = [&](const f32x16 (&sa)[2]) __attribute__((always_inline)) -> float {
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sa[kb][r]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale_log2;
  };
  // P = 2^(S * scale - m_off) packed to the MFMA type; returns this lane's
  // sum of the rounded P
  auto exp_pack = [&](const f32x16 (&sc)[2], Frag (&pf)[4]) __attribute__((always_inline)) -> float {
    const float nb = -m_off;
    float l0 = 0.f, l1 = 0.f;
#pragma unroll
    for (int stp = 0; stp < 4; ++stp) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        p[e] = __builtin_amdgcn_exp2f(fmaf(sc[stp >> 1][8 * (stp & 1) + e], scale_log2, nb));
      pf[stp] = Mfma<T>::pack(p);
      if (stp & 1) l1 = Mfma<T>::sum8(pf[stp], l1);
      else l0 = Mfma<T>::sum8(pf[stp], l0);
    }
    return l0 + l1;
  };
  // S(next) = K(st) Q^T, interleaved with P of S(cur); returns the lane
  // sum.  The V fragments of the PV product that follows (slot vst) are read
  // here too, so their LDS latency hides behind the exponentials.
  auto qk_exp = [&](int st, f32x16 (&snext)[2], const f32x16 (&scur_)[2], Frag (&pf)[4], int vst,
                    Frag (&vf)[HB][4]) __attribute__((always_inline)) -> float {
    if constexpr (LEAN) {
      // K fragments in two halves of the head dimension, V read in pv
      constexpr int KH = KC / 2;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) snext[kb][r] = 0.f;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        Frag kf[KH][2];
#pragma unroll
        for (int c = 0; c < KH; ++c)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
            kf[c][kb] = kfrag(st, kb * 32 + krow, 2 * (half * KH + c) + hi);
#pragma unroll
        for (int c = 0; c < KH; ++c)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) Mfma<T>::mma(snext[kb], kf[c][kb], qf[half * KH + c]);
      }
      const float lt = exp_pack(scur_, pf);
#pragma unroll
      for (int i = 0; i < 2 * KC; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
      }
      (void)vst;
      (void)vf;
      return lt;
    }
    Frag kf[KC][2];
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) kf[c][kb] = kfrag(st, kb * 32 + krow, 2 * c + hi);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int stp = 0; stp < 4; ++stp) vf[hb][stp] = vfrag(vst, hb, stp);
    // every fragment read issued together, one wait for all of them
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) asm volatile("" : "+v"(kf[c][kb]));
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int stp = 0; stp < 4; ++stp) asm volatile("" : "+v"(vf[hb][stp]));
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) snext[kb][r] = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) Mfma<T>::mma(snext[kb], kf[c][kb], qf[c]);
    const float lt = exp_pack(scur_, pf);
    // order: one MFMA per ~12 VALU (the exponentials of tile t)
#pragma unroll
    for (int i = 0; i < 2 * KC; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
    }
    return lt;
  };
  // accept P of tile `sc` (lane sum lt), or redo it from a raised offset
  auto settle = [&](const f32x16 (&sc)[2], Frag (&pf)[4], float lt) __attribute__((always_inline)) {
    if (__any(!(lt <= kSumLimit))) {
      const float m_new = fmaxf(m_off, rowmax(sc));
      const float alpha = m_off == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_off - m_new);
      l_run *= alpha;
#pragma unroll
      for (int hb = 0; hb < HB; ++hb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[hb][r] *= alpha;
      m_off = m_new;
      lt = exp_pack(sc, pf);
    }
    l_run += lt;
  };
  // O += V^T P^T from the fragments qk_exp read (LEAN: read here, from slot vst)
  auto pv = [&](const Frag (&vf)[HB][4], const Frag (&pf)[4], int vst) __attribute__((always_inline)) {
    if constexpr (LEAN) {
#pragma unroll
      for (int stp = 0; stp < 4; ++stp)
#pragma unroll
        for (int hb = 0; hb < HB; ++hb)
          Mfma<T>::mma(o[hb], vfrag(vst, hb, stp), pf[stp]);
    } else {
#pragma unroll
      for (int stp = 0; stp < 4; ++stp)
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) Mfma<T>::mma(o[hb], vf[hb][stp], pf[stp]);
    }
  };

  // Ring invariant at the top of step t: LDS slots of tiles t and t+1 hold
  // them, and sc holds S(t).  Register path: the staging registers hold tile
  // t+2 (its loads in flight since the previous step); a step first stores
  // tile t+2 into the slot tile t-2 freed, then loads tile t+3.  DMA path:
  // tile t+2's copies are in flight into its slot; a step first issues tile
  // t+3's copies into the slot tile t-1 freed.  Either way every global load
  // has a whole step to land; one barrier per step orders the slot reuse.
  if constexpr (DMA) {
    // the first three tiles in flight at once; the first two have landed
    // at the barrier
    dma_kv(t_lo, 0);
    dma_kv(t_lo + 1, 1);
    dma_kv(t_lo + 2, 2);
    step_barrier();
  } else {
    {
      // both first tiles in flight at once (one global latency, not two)
      uint4 rk1[KPT], rv01[VPT], rv11[VPT];
      load_kv(t_lo);
      load_kv_into(t_lo + 1, rk1, rv01, rv11);
      store_kv(0);
      store_kv_from(1, rk1, rv01, rv11);
    }
    __syncthreads();
    load_kv(t_lo + 2);
  }

  // The compiler does not see the ring's copies (inline asm) and waits for
  // the Q loads before their first use: here, once, not in the interior loop
  // (where its wait would cover every copy in flight on each pass).
  if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  f32x16 scur[2];
  if (t_hi > t_lo) qk(0, scur);
  // Interior tiles: every key below the workgroup's first query and inside
  // the sequence, and a next tile exists in this item's range.
  int n_int = KEYMASK ? 0 : min(causal ? q0 / BNK : nkt, min(kend / BNK, t_hi - 1));
  n_int = max(n_int, t_lo);
  int t = t_lo;
  // an unmasked first tile starts the offset at its row max, so the
  // interior loop does not redo it
  if (t < n_int) m_off = rowmax(scur);
  f32x16 salt[2];
  Frag pf[4];
  // one interior step; j is tile t's ring slot (a constant in the unrolled loop)
  auto istep = [&](int tt, int j, const f32x16 (&sc)[2], f32x16 (&sn)[2]) __attribute__((always_inline)) {
    if constexpr (DMA) {
      dma_kv(tt + 3, (j + 3) & (NST - 1));
    } else {
      store_kv((j + 2) & (NST - 1));
      load_kv(tt + 3);
    }
    Frag vf[HB][4];
    const float lt = qk_exp((j + 1) & (NST - 1), sn, sc, pf, j, vf);
    settle(sc, pf, lt);
    pv(vf, pf, j);
    step_barrier();
  };
  // four tiles per trip (one turn of the ring), scores ping-pong scur <-> salt
  for (; t + 3 < n_int; t += 4) {
    istep(t, 0, scur, salt);
    istep(t + 1, 1, salt, scur);
    istep(t + 2, 2, scur, salt);
    istep(t + 3, 3, salt, scur);
  }
  if (t < n_int) {
    istep(t, slot_of(t), scur, salt);
    ++t;
    if (t < n_int) {
      istep(t, slot_of(t), salt, scur);
      ++t;
      if (t < n_int) {
        istep(t, slot_of(t), scur, salt);
        ++t;
        scur[0] = salt[0];
        scur[1] = salt[1];
      }
    } else {
      scur[0] = salt[0];
      scur[1] = salt[1];
    }
  }
  for (; t < t_hi; ++t) {
    if constexpr (DMA) {
      dma_kv(t + 3, slot_of(t + 3));
    } else {
      store_kv(slot_of(t + 2));
      load_kv(t + 3);
    }
    f32x16 snext[2];
    const bool act_next = t + 1 < t_hi && (!causal || (t + 1) * BNK <= wq0 + 31);
    if (act_next) qk(slot_of(t + 1), snext);
    const bool act = !causal || t * BNK <= wq0 + 31;
    if (act) {
      // a tile below the wave's first query and inside the sequence (the
      // first diagonal tile for the upper waves) needs no mask
      if (KEYMASK || (causal && t * BNK + BNK - 1 > wq0) || t * BNK + BNK > kend) mask_tile(t, scur);
      softmax_pv(slot_of(t), scur);
    }
    step_barrier();
    if (act_next) {
      scur[0] = snext[0];
      scur[1] = snext[1];
    }
  }
  // no copy may still be writing this workgroup's LDS when it ends
  if constexpr (DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // normalise and store: register r of block hb is hd row hb*32 + 8*(r/4) + 4*hi + r%4
  const int q = wq0 + l32;
  const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
  const float l = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
  // Partial slot s: O^T rows [query][HDP] fp32, then m[BMQ], then l[BMQ].
  // The halves of a split item are different workgroups, possibly on
  // different XCDs: the partial is written through to memory (sc0 sc1) and
  // read device-coherently (sc1), with a flag per slot in between.
  // The descriptor covers exactly the n_slots partial slots.
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(partials, (short)0, n_slots * (BMQ * (HDP + 2)) * 4, 0x00020000);
  auto pslot = [&](int sl) { return sl * (BMQ * (HDP + 2)) * 4; };  // byte offset
  const int prow = (wave * 32 + l32) * HDP * 4;
  if (slot >= 0) {
    const int pb = pslot(slot);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = {o[hb][4 * g], o[hb][4 * g + 1], o[hb][4 * g + 2], o[hb][4 * g + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                               pb + prow + (hb * 32 + 8 * g + 4 * hi) * 4, 0, kFaSc0Sc1);
      }
    if (hi == 0) {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, m_off), prs,
                                            pb + (BMQ * HDP + wave * 32 + l32) * 4, 0, kFaSc0Sc1);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, l), prs,
                                            pb + (BMQ * HDP + BMQ + wave * 32 + l32) * 4, 0, kFaSc0Sc1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial is in memory
    __syncthreads();
    if (tid == 0) {
      // 0 -> 1 publishes.  -1 means the second half stopped waiting (its rows
      // are already NaN): the flag is reset for the next launch instead.
      int expected = 0;
      if (!__hip_atomic_compare_exchange_strong(&flags[slot], &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT))
        __hip_atomic_store(&flags[slot], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  float lm = l;
  bool merged = true;
  if (slot <= -2) {
    // Second half: thread 0 waits for the first half's flag (bounded
    // polls).  On a timeout it claims the flag (0 -> -1), counts the timeout
    // in the error word and the item's rows are written as NaN; a first
    // half that publishes later finds -1 and resets the flag, so nothing
    // stale reaches the next launch.  Merged:
    //   O = O_hi a_hi + O_lo a_lo,  l = l_hi a_hi + l_lo a_lo,
    //   a_x = 2^(m_x - max(m_lo, m_hi)),  in this order every time.
    const int ps = -2 - slot;
    int& s_published = *s_flag;
    if (tid == 0) {
      int v = __hip_atomic_load(&flags[ps], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int spins = 0; v != 1 && spins < kFaSpinLimit; ++spins) {
        __builtin_amdgcn_s_sleep(2);
        v = __hip_atomic_load(&flags[ps], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (v != 1) {
        int expected = 0;
        if (__hip_atomic_compare_exchange_strong(&flags[ps], &expected, -1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)) {
          __hip_atomic_fetch_add(&flags[-1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          v = expected;  // published between the last poll and the claim
        }
      }
      s_published = v == 1;
    }
    __syncthreads();
    merged = s_published != 0;
  }
  if (slot <= -2 && merged) {
    const int ps = -2 - slot, pb = pslot(ps);
    const float m_lo = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(prs, pb + (BMQ * HDP + wave * 32 + l32) * 4, 0, kFaSc1));
    const float l_lo = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(prs, pb + (BMQ * HDP + BMQ + wave * 32 + l32) * 4, 0, kFaSc1));
    const float m = fmaxf(m_lo, m_off);
    const float a_lo = m_lo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_lo - m);
    const float a_hi = m_off == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_off - m);
    lm = fmaf(l, a_hi, l_lo * a_lo);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, pb + prow + (hb * 32 + 8 * g + 4 * hi) * 4, 0, kFaSc1));
#pragma unroll
        for (int e = 0; e < 4; ++e) o[hb][4 * g + e] = fmaf(o[hb][4 * g + e], a_hi, v[e] * a_lo);
      }
  }
  float inv = lm > 0.f ? 1.0f / lm : 0.f;
  if (!merged || bad_slot) {
    if (bad_slot && flags != nullptr && tid == 0)
      __hip_atomic_fetch_add(&flags[-1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    inv = __builtin_nanf("");
  }
  // DMA ring: the wave's 32 x HDP block goes through LDS and out as 16-byte
  // pieces of whole rows, 8 lanes per 128 bytes, so a launch that writes 4
  // MiB or more can write them through the L2 (its 8-byte pieces 2 KB apart,
  // stored straight from the accumulator layout, measured 4 us slower per C4
  // launch written through, one by one).  Needs 16-byte aligned rows.
  const bool staged = DMA && ((uintptr_t)out & 15) == 0 && (ld_out % 8) == 0;
  if (staged) {
    // The ring is free once every wave's copies have landed (the copies of
    // tiles past the item write zeros too) and every wave is past its last
    // tile.
    __syncthreads();
    // The GEMM epilogue's staging layout: whole 16-byte pieces per lane (the
    // halves of pieces g = 2k, 2k + 1 trade lanes l32 and l32 + 32), piece p
    // of row r at slot r PPR + (p ^ (r & 7)): no LDS bank conflicts for the
    // 8-lanes-per-cycle writes or the 32-lanes-per-cycle reads.
    constexpr int PPR = HDP * 2 / 16;            // 16-byte pieces per row (8 or 16)
    constexpr int NPASS = 32 * PPR / 64;         // store instructions per wave
    static_assert(!DMA || PPR % 8 == 0, "rows of whole 8-piece XOR groups");
    auto slot = [](int r, int p) __attribute__((always_inline)) { return (r * PPR + (p ^ (r & 7))) * 16; };
    char* stg = smem + wave * 32 * PPR * 16;
    auto scaled = [&](int hb, int g) __attribute__((always_inline)) {
      return Quad<T>::from(make_float4(o[hb][4 * g] * inv, o[hb][4 * g + 1] * inv, o[hb][4 * g + 2] * inv,
                                       o[hb][4 * g + 3] * inv));
    };
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const typename Quad<T>::raw x = scaled(hb, 2 * k), y = scaled(hb, 2 * k + 1);
        const auto s0 = __builtin_amdgcn_permlane32_swap(x.x, y.x, false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(x.y, y.y, false, false);
        *reinterpret_cast<uint4*>(stg + slot(l32, 4 * hb + 2 * k + hi)) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
      }
    const int nrow = min(Sb - wq0, 32);
    const RowOut rows(out + (row0 + wq0) * ld_out + (int64_t)h * hd,
                      nrow > 0 ? ((int64_t)(nrow - 1) * ld_out + HDP) * (int64_t)sizeof(T) : 0,
                      (int64_t)B * S * H * HDP * (int64_t)sizeof(T) >= kWtMinBytes);
    with_wt(rows.wt, [&](auto wt_tag) {
      const auto w = rows.writer<decltype(wt_tag)::value>();
#pragma unroll
      for (int ps = 0; ps < NPASS; ++ps) {
        const int idx = lane + 64 * ps, r = idx / PPR, pc = idx % PPR;
        const uint4 piece = *reinterpret_cast<const uint4*>(stg + slot(r, pc));
        if (r < nrow) w.put((int)(((int64_t)r * ld_out + pc * 8) * (int64_t)sizeof(T)), piece);
      }
    });
  } else if (q < Sb) {
    T* orow = out + (row0 + q) * ld_out + (int64_t)h * hd;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = hb * 32 + 8 * g + 4 * hi;
        if (FULLHD || col < hd) {
          const float4 v = make_float4(o[hb][4 * g] * inv, o[hb][4 * g + 1] * inv, o[hb][4 * g + 2] * inv,
                                       o[hb][4 * g + 3] * inv);
          *reinterpret_cast<typename Quad<T>::raw*>(orow + col) = Quad<T>::from(v);
        }
      }
  }
  if (slot <= -2 && merged) {
    __syncthreads();  // every wave has read the partial
    if (tid == 0) __hip_atomic_store(&flags[-2 - slot], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  };

  // Scheduled (the 4-wave kernel without a key mask; the other
  // instantiations are launched on the grid only and carry one copy of the
  // item code): workgroup w runs items w, w + gridDim.x, w + 2 gridDim.x,
  // ... of the list, in that order.  An item whose (b, h) is -1 is a hole
  // (a shorter list's padding).  An item outside the launch's (b, h) range
  // cannot be placed: it is counted in the error word and dropped.  A slot
  // outside [0, n_slots) (or its second-half image) has no partial to
  // publish or merge: the item's rows are written as NaN and counted.
  if (!KEYMASK && NW == 4 && work != nullptr) {
    for (int j = blockIdx.x; j < n_work; j += gridDim.x) {
      const int4 it = work[j];
      if (it.x == -1) continue;
      const int t_lo = it.z & 0xffff, t_hi = it.z >> 16;
      if (it.x < 0 || it.x >= BH || it.y < 0 || t_lo > t_hi) {
        if (flags != nullptr && threadIdx.x == 0)
          __hip_atomic_fetch_add(&flags[-1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        continue;
      }
      const bool bad_slot = it.w != -1 && (it.w >= n_slots || it.w < -1 - n_slots);
      run_item(it.x, it.y, t_lo, t_hi, bad_slot ? -1 : it.w, bad_slot);
      __syncthreads();  // the next item refills the K / V ring and the LDS flag
    }
  } else {
    // Longest query blocks first within groups of `grp` (b, h) pairs: a
    // group's blocks run together, which bounds the K/V the blocks in
    // flight stream (grp = B*H: one group, longest first over everything).
    const int gi = blockIdx.x / (grp * nqb), r = blockIdx.x % (grp * nqb);
    const int gsize = min(grp, BH - gi * grp);
    const int rank = r / gsize;
    run_item(gi * grp + r % gsize, causal ? nqb - 1 - rank : rank, 0, 1 << 30, -1, false);
  }
}

__global__ __launch_bounds__(256) void clear_words_kernel(int* p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0;
}

template <typename T, int HDP>
static int launch_sched(const void* qkv, int64_t ss, int64_t sc, int64_t sh, void* out, int64_t ld_out,
                        int B, int S, int H, int hd, float scale_log2, int causal, const int32_t* cu_seqlens,
                        const int32_t* work, int n_work, int n_lists, float* partials, int n_slots, bool clear,
                        hipStream_t st) {
  // [n_slots partial slots][error word][n_slots flags]; flags[-1] is the error word
  int* flags = partials != nullptr ? reinterpret_cast<int*>(partials + (size_t)n_slots * 128 * (HDP + 2)) + 1 : nullptr;
  if (clear && flags != nullptr) {
    // a fill kernel, not hipMemsetAsync: the call may be recorded into a graph
    hipLaunchKernelGGL(clear_words_kernel, dim3(1), dim3(256), 0, st, flags - 1, n_slots + 1);
  }
#define TJK_PIPE_SCHED(FULL)                                                                                  \
  hipLaunchKernelGGL((flash_pipe_kernel<T, HDP, false, FULL, 4>), dim3((unsigned)n_lists), dim3(256), 0, st,  \
                     (const T*)qkv, (int64_t)0, ss, sc, sh, (T*)out, ld_out, B, S, H, hd, scale_log2, causal, \
                     (const int32_t*)nullptr, (const uint8_t*)nullptr, cu_seqlens, 0,                         \
                     reinterpret_cast<const int4*>(work), n_work, partials, flags, n_slots, 1)
  if (hd == HDP) TJK_PIPE_SCHED(true); else TJK_PIPE_SCHED(false);
#undef TJK_PIPE_SCHED
  return check_launch("tjk_flash_fwd_sched");
}

template <typename T, int HDP>
static int launch_pipe(const void* qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh, void* out,
                       int64_t ld_out, int B, int S, int H, int hd, float scale_log2, int causal,
                       const int32_t* lengths, const uint8_t* key_mask, const int32_t* cu_seqlens,
                       hipStream_t st) {
  // head_dim 128 without a key mask: 8 waves and 256 queries per workgroup
  // (see flash_pipe_kernel; with a key mask that variant would spill)
  constexpr int NW8 = HDP == 128 ? 8 : 4;
  const int nw = key_mask == nullptr ? NW8 : 4;
  const int nqb = (S + 32 * nw - 1) / (32 * nw);
  const int64_t nblk = (int64_t)nqb * B * H;
  if (nblk > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: grid too large");
  // (b, h) pairs per group: all of them while their K / V fit in about half
  // the 256 MB Infinity Cache, else as many as fit (at least 8).  At the
  // reference's case 14 (B = 32, H = 16, S = 100000) the 512 pairs stream
  // 13 GB of K / V; grouped by 8 the blocks in flight share ~200 MB.
  const int64_t kv_pair = (int64_t)S * hd * 2 * (int64_t)sizeof(T);
  const int64_t fit = (int64_t)128 * 1024 * 1024 / (kv_pair > 0 ? kv_pair : 1);
  const int grp = (int)std::max<int64_t>(std::min<int64_t>(B * H, std::max<int64_t>(fit, 8)), 1);
#define TJK_PIPE(KM, FULL, NWV)                                                                                \
  hipLaunchKernelGGL((flash_pipe_kernel<T, HDP, KM, FULL, NWV>), dim3((unsigned)nblk), dim3(64 * NWV), 0, st,   \
                     (const T*)qkv, sb, ss, sc, sh, (T*)out, ld_out, B, S, H, hd, scale_log2, causal, lengths,  \
                     key_mask, cu_seqlens, nqb, (const int4*)nullptr, 0, (float*)nullptr, (int*)nullptr, 0, grp)
  if (key_mask != nullptr) {
    if (hd == HDP) TJK_PIPE(true, true, 4); else TJK_PIPE(true, false, 4);
  } else {
    if (hd == HDP) TJK_PIPE(false, true, NW8); else TJK_PIPE(false, false, NW8);
  }
#undef TJK_PIPE
  return check_launch("tjk_flash_fwd");
}

template <typename T, int HDP, int NQ, int KS>
static int launch_flash(const void* qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh, void* out,
                        int64_t ld_out, int B, int S, int H, int hd, float scale_log2, int causal,
                        const int32_t* lengths, const uint8_t* key_mask, const int32_t* cu_seqlens,
                       hipStream_t st) {
  constexpr int BMQ = 4 * NQ * 32;
  const int nqb = (S + BMQ - 1) / BMQ;
  const dim3 block(256 * KS);
  const int64_t nblk = (int64_t)nqb * B * H;
  if (nblk > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: grid too large");
  if (key_mask != nullptr)
    hipLaunchKernelGGL((flash_fwd_kernel<T, HDP, NQ, KS, true>), dim3((unsigned)nblk), block, 0, st,
                       (const T*)qkv, sb, ss, sc, sh, (T*)out, ld_out, B, S, H, hd, scale_log2, causal,
                       lengths, key_mask, cu_seqlens, nqb);
  else
    hipLaunchKernelGGL((flash_fwd_kernel<T, HDP, NQ, KS, false>), dim3((unsigned)nblk), block, 0, st,
                       (const T*)qkv, sb, ss, sc, sh, (T*)out, ld_out, B, S, H, hd, scale_log2, causal,
                       lengths, key_mask, cu_seqlens, nqb);
  return check_launch("tjk_flash_fwd");
}

template <typename T, int HDP>
static int launch_short(const void* qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh, void* out,
                        int64_t ld_out, int B, int S, int H, int hd, float scale_log2, int causal,
                        const int32_t* lengths, const uint8_t* key_mask, const int32_t* cu_seqlens,
                        hipStream_t st) {
  const int nqb = (S + 31) / 32;
  const int64_t nblk = (int64_t)nqb * B * H;
  if (nblk > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: grid too large");
  if (key_mask != nullptr)
    hipLaunchKernelGGL((flash_short_kernel<T, HDP, true>), dim3((unsigned)nblk), dim3(64), 0, st, (const T*)qkv,
                       sb, ss, sc, sh, (T*)out, ld_out, B, S, H, hd, scale_log2, causal, lengths, key_mask,
                       cu_seqlens, nqb);
  else
    hipLaunchKernelGGL((flash_short_kernel<T, HDP, false>), dim3((unsigned)nblk), dim3(64), 0, st, (const T*)qkv,
                       sb, ss, sc, sh, (T*)out, ld_out, B, S, H, hd, scale_log2, causal, lengths, key_mask,
                       cu_seqlens, nqb);
  return check_launch("tjk_flash_fwd");
}

template <typename T, int HDP>
static int flash_plan(int plan, const void* qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh, void* out,
                      int64_t ld_out, int B, int S, int H, int hd, float scale_log2, int causal,
                      const int32_t* lengths, const uint8_t* key_mask, const int32_t* cu_seqlens,
                       hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (plan == 0)
      return launch_pipe<T, HDP>(qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                                 key_mask, cu_seqlens, st);
  }
  // plan 4: sequences of at most 128 tokens (checked by the entry point);
  // fp32 at hd 128 would not fit its K / V^T tiles and runs plan 1
  if constexpr (sizeof(T) == 2 || HDP <= 64) {
    if (plan == 4)
      return launch_short<T, HDP>(qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                                  key_mask, cu_seqlens, st);
  }
  if (plan == 2)
    return launch_flash<T, HDP, 2, 1>(qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                                      key_mask, cu_seqlens, st);
  // plan 3: two key splits per query group (8 waves); fp32 at hd 128 would
  // not fit its K/V tiles in LDS and runs plan 1 instead.
  if (plan == 3 && (sizeof(T) == 2 || HDP <= 64))
    return launch_flash<T, HDP, 1, (sizeof(T) == 2 || HDP <= 64) ? 2 : 1>(
        qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths, key_mask, cu_seqlens, st);
  return launch_flash<T, HDP, 1, 1>(qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                                    key_mask, cu_seqlens, st);
}

template <typename T>
static int flash_typed(int plan, const void* qkv, int64_t sb, int64_t ss, int64_t sc, int64_t sh, void* out,
                       int64_t ld_out, int B, int S, int H, int hd, float scale_log2, int causal,
                       const int32_t* lengths, const uint8_t* key_mask, const int32_t* cu_seqlens,
                       hipStream_t st) {
  if (hd <= 32)
    return flash_plan<T, 32>(plan, qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                             key_mask, cu_seqlens, st);
  if (hd <= 64)
    return flash_plan<T, 64>(plan, qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                             key_mask, cu_seqlens, st);
  return flash_plan<T, 128>(plan, qkv, sb, ss, sc, sh, out, ld_out, B, S, H, hd, scale_log2, causal, lengths,
                            key_mask, cu_seqlens, st);
}

}  // namespace tjk

using namespace tjk;

extern "C" int tjk_flash_plan_count(int dtype) {
  if (dtype != TJK_F32 && dtype != TJK_F16 && dtype != TJK_BF16)
    return fail(TJK_EINVAL, "tjk_flash_plan_count: bad dtype %d", dtype);
  return 5;
}

extern "C" int tjk_flash_fwd(const void* qkv, int64_t stride_b, int64_t stride_s,
                             int64_t stride_c, int64_t stride_h,
                             void* out, int64_t ld_out,
                             int batch, int seq, int heads, int head_dim, float scale,
                             int causal, const int32_t* lengths, const uint8_t* key_mask,
                             const int32_t* cu_seqlens, int dtype, int plan_id, void* stream) {
  if (batch < 0 || seq < 0 || heads <= 0 || head_dim <= 0)
    return fail(TJK_EINVAL, "tjk_flash_fwd: bad shape B=%d S=%d H=%d hd=%d", batch, seq, heads, head_dim);
  if (batch == 0 || seq == 0) return TJK_OK;
  if (!qkv || !out) return fail(TJK_EINVAL, "tjk_flash_fwd: null pointer");
  if (dtype != TJK_F32 && dtype != TJK_F16 && dtype != TJK_BF16) return fail(TJK_EINVAL, "tjk_flash_fwd: bad dtype %d", dtype);
  if (head_dim > 128 || head_dim % 8)
    return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: head_dim=%d must be a multiple of 8 and <= 128", head_dim);
  if (plan_id < -1 || plan_id > 4) return fail(TJK_EINVAL, "tjk_flash_fwd: plan %d out of range", plan_id);
  if (plan_id == 4 && seq > 128)
    return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: plan 4 takes sequences of at most 128 tokens, got %d", seq);
  if (cu_seqlens && key_mask)
    return fail(TJK_EINVAL, "tjk_flash_fwd: cu_seqlens (packed sequences) and key_mask are exclusive");
  const int vec = 16 / dtype_size(dtype);
  if (stride_b % vec || stride_s % vec || stride_c % vec || stride_h % vec)
    return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: strides must be multiples of %d elements", vec);
  if (ld_out < (int64_t)heads * head_dim || ld_out % 4) return fail(TJK_EINVAL, "tjk_flash_fwd: bad ld_out");
  if (((uintptr_t)qkv & 15) || ((uintptr_t)out & (4 * dtype_size(dtype) - 1)))
    return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd: misaligned pointer");
  if (!(scale > 0.f)) return fail(TJK_EINVAL, "tjk_flash_fwd: scale must be positive");
  // plan 0: software-pipelined kernel (2-byte types, byte offsets within a
  // head's K/V span must fit 31 bits); plans 1/2: one / two 32-query blocks
  // per wave without cross-tile pipelining (every dtype); plan 3: plan 1
  // with two key splits per query group (8 waves, merged through LDS).
  // Measured on MI355X (bf16): at hd <= 64 plan 0 is fastest at every
  // length (causal 4 x 2048: 54 vs 60 us; S = 32768: 944 vs 790 TFLOP/s);
  // at hd 128 too since its 8-wave workgroups (causal 16 x 512: 50.5 vs
  // 53.0 us, 4 x 2048: 95.1 vs 122.6 us, 2 x 8192: 615 vs 743 us); plans 2
  // and 3 were slower on every BASELINE shape.
  // With a key mask plan 0 runs every tile through its masked
  // (unpipelined) loop: plan 1 from S = 2048 (padded C4 with a per-key
  // mask: 129 vs 168 us).  A sequence of one 128-query block has only
  // diagonal tiles and nothing to pipeline: plan 1 there too (C2's
  // 1 x 128 x 8 heads fp16: 6.2 vs 6.8 us).  Plan 4 (whole sequence in one
  // one-wave workgroup per 32 queries) takes every sequence of at most 128
  // tokens.
  const bool pipe_ok = dtype != TJK_F32 && ((int64_t)seq * stride_s + head_dim) * dtype_size(dtype) < INT32_MAX;
  if (plan_id == -1) {
    if (seq <= 128)
      plan_id = 4;
    else
      plan_id = (pipe_ok && (key_mask == nullptr || seq < 2048)) ? 0 : 1;
  }
  if (plan_id == 0 && !pipe_ok) plan_id = 1;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case TJK_F32:
      return flash_typed<float>(plan_id, qkv, stride_b, stride_s, stride_c, stride_h, out, ld_out, batch, seq,
                                heads, head_dim, scale_log2, causal, lengths, key_mask, cu_seqlens, st);
    case TJK_F16:
      return flash_typed<f16>(plan_id, qkv, stride_b, stride_s, stride_c, stride_h, out, ld_out, batch, seq,
                              heads, head_dim, scale_log2, causal, lengths, key_mask, cu_seqlens, st);
    default:
      return flash_typed<bf16>(plan_id, qkv, stride_b, stride_s, stride_c, stride_h, out, ld_out, batch, seq,
                               heads, head_dim, scale_log2, causal, lengths, key_mask, cu_seqlens, st);
  }
}

extern "C" size_t tjk_flash_partial_bytes(int head_dim, int n_slots) {
  if (head_dim <= 0 || n_slots < 0) return 0;
  const int hdp = head_dim <= 32 ? 32 : head_dim <= 64 ? 64 : 128;
  // partial slots, then the error word and one flag per slot
  return (size_t)n_slots * 128 * (hdp + 2) * sizeof(float) + (size_t)(n_slots + 1) * sizeof(int);
}

static int flash_sched_entry(const char* who, const void* qkv, int64_t stride_s, int64_t stride_c,
                             int64_t stride_h, void* out, int64_t ld_out, int batch, int max_seqlen, int heads,
                             int head_dim, float scale, int causal, const int32_t* cu_seqlens, const int32_t* work,
                             int n_work, int n_lists, float* partials, size_t partials_bytes, int n_slots, int dtype,
                             bool clear, hipStream_t st) {
  if (batch < 0 || max_seqlen < 0 || heads <= 0 || head_dim <= 0 || n_work < 0 || n_slots < 0)
    return fail(TJK_EINVAL, "%s: bad shape or counts", who);
  if (n_work == 0) return TJK_OK;
  if (n_lists <= 0 || n_lists > n_work)
    return fail(TJK_EINVAL, "%s: n_lists=%d must be in [1, n_work=%d]", who, n_lists, n_work);
  if (!qkv || !out || !cu_seqlens || !work) return fail(TJK_EINVAL, "%s: null pointer", who);
  if ((n_slots > 0 || partials) && (!partials || partials_bytes < tjk_flash_partial_bytes(head_dim, n_slots)))
    return fail(TJK_EINVAL, "%s: %d split slots need %zu bytes of partials (got %zu)", who, n_slots,
                tjk_flash_partial_bytes(head_dim, n_slots), partials_bytes);
  if ((int64_t)n_slots * 128 * 130 * 4 >= INT32_MAX) return fail(TJK_EUNSUPPORTED, "%s: too many slots", who);
  if (dtype != TJK_F16 && dtype != TJK_BF16) return fail(TJK_EUNSUPPORTED, "%s: 2-byte dtypes only (got %d)", who, dtype);
  if (head_dim > 128 || head_dim % 8)
    return fail(TJK_EUNSUPPORTED, "%s: head_dim=%d must be a multiple of 8 and <= 128", who, head_dim);
  if (stride_s % 8 || stride_c % 8 || stride_h % 8)
    return fail(TJK_EUNSUPPORTED, "%s: strides must be multiples of 8 elements", who);
  if (((int64_t)max_seqlen * stride_s + head_dim) * 2 >= INT32_MAX)
    return fail(TJK_EUNSUPPORTED, "%s: a sequence's K/V span exceeds 31-bit offsets", who);
  if (ld_out < (int64_t)heads * head_dim || ld_out % 4) return fail(TJK_EINVAL, "%s: bad ld_out", who);
  if (((uintptr_t)qkv & 15) || ((uintptr_t)out & 7) || ((uintptr_t)work & 15) || ((uintptr_t)partials & 15))
    return fail(TJK_EUNSUPPORTED, "%s: misaligned pointer", who);
  if (!(scale > 0.f)) return fail(TJK_EINVAL, "%s: scale must be positive", who);
  const float scale_log2 = scale * 1.4426950408889634f;
#define TJK_SCHED(TT, HDP)                                                                                  \
  return launch_sched<TT, HDP>(qkv, stride_s, stride_c, stride_h, out, ld_out, batch, max_seqlen, heads, \
                               head_dim, scale_log2, causal, cu_seqlens, work, n_work, n_lists, partials, n_slots, \
                               clear, st)
  if (dtype == TJK_F16) {
    if (head_dim <= 32) TJK_SCHED(f16, 32);
    if (head_dim <= 64) TJK_SCHED(f16, 64);
    TJK_SCHED(f16, 128);
  }
  if (head_dim <= 32) TJK_SCHED(bf16, 32);
  if (head_dim <= 64) TJK_SCHED(bf16, 64);
  TJK_SCHED(bf16, 128);
#undef TJK_SCHED
}

extern "C" int tjk_flash_fwd_sched(const void* qkv, int64_t stride_s, int64_t stride_c, int64_t stride_h,
                                   void* out, int64_t ld_out, int batch, int max_seqlen, int heads,
                                   int head_dim, float scale, int causal, const int32_t* cu_seqlens,
                                   const int32_t* work, int n_work, int n_lists, float* partials,
                                   size_t partials_bytes, int n_slots, int dtype, void* stream) {
  return flash_sched_entry("tjk_flash_fwd_sched", qkv, stride_s, stride_c, stride_h, out, ld_out, batch, max_seqlen,
                           heads, head_dim, scale, causal, cu_seqlens, work, n_work, n_lists, partials, partials_bytes,
                           n_slots, dtype, false, reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------- allocation-free variant
//
// The scheduled kernel's workspace (split partials, error word, flags) in a
// file-scope device array instead of a caller's buffer, for callers that
// cannot allocate.  Each device holds its own copy for the life of the
// process; its address is looked up once per device with
// hipGetSymbolAddress (the array's name is only a host-side stand-in) and
// that pointer is what the kernels get.  Every call clears the error word
// and the flags with a fill kernel first (graph-capture safe); calls that
// overlap on one device share the array and race.
constexpr size_t kSchedScratchBytes = size_t(4) << 20;
static __device__ __attribute__((aligned(256))) unsigned char scratch[kSchedScratchBytes];

static std::mutex g_scratch_mu;
static float* g_scratch[64];

static int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(hip_status(e), "tjk_flash_fwd_sched_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd_sched_static: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(e != hipSuccess ? hip_status(e) : TJK_EUNSUPPORTED,
                  "tjk_flash_fwd_sched_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return TJK_OK;
}

extern "C" size_t tjk_flash_sched_static_bytes(void) { return kSchedScratchBytes; }

extern "C" int tjk_flash_fwd_sched_static(const void* qkv, int64_t stride_s, int64_t stride_c, int64_t stride_h,
                                          void* out, int64_t ld_out, int batch, int max_seqlen, int heads,
                                          int head_dim, float scale, int causal, const int32_t* cu_seqlens,
                                          const int32_t* work, int n_work, int n_lists, int n_slots, int dtype,
                                          void* stream) {
  if (head_dim <= 0 || n_slots < 0) return fail(TJK_EINVAL, "tjk_flash_fwd_sched_static: bad shape or counts");
  const size_t need = tjk_flash_partial_bytes(head_dim, n_slots);
  if (need > kSchedScratchBytes)
    return fail(TJK_EUNSUPPORTED, "tjk_flash_fwd_sched_static: %d split slots need %zu bytes, above the %zu-byte "
                "static workspace", n_slots, need, kSchedScratchBytes);
  if (n_work <= 0) return n_work < 0 ? fail(TJK_EINVAL, "tjk_flash_fwd_sched_static: bad shape or counts") : TJK_OK;
  float* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != TJK_OK) return rc;
  return flash_sched_entry("tjk_flash_fwd_sched_static", qkv, stride_s, stride_c, stride_h, out, ld_out, batch,
                           max_seqlen, heads, head_dim, scale, causal, cu_seqlens, work, n_work, n_lists, ws,
                           kSchedScratchBytes, n_slots, dtype, true, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tjk_flash_sched_occupancy(int head_dim, int dtype) {
  // Workgroups of the scheduled kernel resident per CU (LDS / register bound).
  int blocks = 0;
  hipError_t e = hipErrorInvalidValue;
  const bool h16 = dtype == TJK_F16;
#define TJK_OCC(TT, HDP) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, flash_pipe_kernel<TT, HDP, false, true, 4>, 256, 0)
  if (head_dim <= 32) { if (h16) TJK_OCC(f16, 32); else TJK_OCC(bf16, 32); }
  else if (head_dim <= 64) { if (h16) TJK_OCC(f16, 64); else TJK_OCC(bf16, 64); }
  else { if (h16) TJK_OCC(f16, 128); else TJK_OCC(bf16, 128); }
#undef TJK_OCC
  if (e != hipSuccess) return fail(hip_status(e), "tjk_flash_sched_occupancy: %s", hipGetErrorString(e));
  return blocks;
}
