// Attention of one wave's 32 queries over a whole short sequence resident in
// LDS: the math shared by the short-sequence attention kernel (tjk_flash_fwd
// plan 4) and the fused attention block (tjk_attn_block), so that both give
// the same bits for the same Q / K / V.
#pragma once

#include "tjk_common.h"

namespace tjk {

// Key order within a 32-key block in which the S^T registers a lane feeds
// into one 16-key PV step cover 8 consecutive keys (bits 2 and 3 swapped).
__device__ __forceinline__ int swap_bits_2_3(int x) {
  return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1);
}

// Exact (one-pass) softmax attention for the 32 queries of one wave over
// keys 0 .. 32*nkb - 1 (nkb <= MAXK / 32):
//   sK  K rows, key-major, row pitch HDP + VEC elements;
//   sV  V^T, hd-major, row pitch MAXK + VEC elements
//   (VEC = 16 / sizeof(T), one 16-byte chunk of padding per row);
//   qf  the queries as MFMA B fragments: lane (l32, hi) holds
//       Q[query l32][16 c + 8 hi + 0..7] in qf[c].
// A key is admitted when key < lim (per lane, i.e. per query) and
// keep(key); keep is called for every key 0 .. MAXK - 1, so it must be
// safe to evaluate past the sequence end.  Computes S^T = K Q^T per 32-key block, the exact row max
// (lanes l and l ^ 32 hold the two halves of a query's keys), P = 2^(S
// scale_log2 - max) with its fp32 row sum, and O^T = V^T P^T in 16-key
// steps.  o receives O^T unnormalised (block hb, register r = hd row
// hb*32 + 8*(r/4) + 4*hi + r%4 of query l32); the return value is
// 1 / row sum, or 0 for a query with no admitted key.
template <typename T, int HDP, int MAXK, typename Keep>
__device__ __forceinline__ float short_attention(const T* sK, const T* sV,
                                                 const typename Mfma<T>::frag (&qf)[HDP / 16], int nkb,
                                                 int lim, float scale_log2, Keep keep, f32x16 (&o)[HDP / 32]) {
  constexpr int NKB = MAXK / 32, KC = HDP / 16, HB = HDP / 32;
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int LDK = HDP + VEC, LDV = MAXK + VEC;
  typedef typename Mfma<T>::frag Frag;
  const int lane = threadIdx.x & 63, l32 = lane & 31, hi = lane >> 5;

  // S^T per 32-key block: register r of block kb is key
  // kb*32 + 16*(r/8) + 8*hi + r%8 (K rows read with bits 2 and 3 swapped)
  const int krow = swap_bits_2_3(l32);
  f32x16 s[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
    if (kb < nkb) {
      const T* kp = &sK[(kb * 32 + krow) * LDK + 8 * hi];
#pragma unroll
      for (int c = 0; c < KC; ++c) Mfma<T>::mma(s[kb], Mfma<T>::load(kp + 16 * c), qf[c]);
    }
  }
  // masks and the row max; keep() is evaluated for every key first (it may
  // load: loads under the key < lim condition would be waited for one by one)
  bool kp[NKB][16];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) kp[kb][r] = keep(kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7));
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb * 32 + 16 * (r >> 3) + 8 * hi + (r & 7);
      const bool admit = key < lim && kp[kb][r];
      s[kb][r] = admit ? s[kb][r] : -INFINITY;
      mx = fmaxf(mx, s[kb][r]);
    }
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  }
  const float m_use = mx == -INFINITY ? 0.f : mx * scale_log2;
  // P, its fp32 row sum, and O^T = V^T P^T in 16-key steps
#pragma unroll
  for (int hb = 0; hb < HB; ++hb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[hb][r] = 0.f;
  float ls = 0.f;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    if (kb < nkb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(s[kb][r], scale_log2, -m_use));
        ls += p[r];
      }
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const Frag pf = Mfma<T>::pack(&p[8 * st]);
#pragma unroll
        for (int hb = 0; hb < HB; ++hb)
          Mfma<T>::mma(o[hb], Mfma<T>::load(&sV[(hb * 32 + l32) * LDV + 8 * hi] + 16 * (2 * kb + st)), pf);
      }
    }
  }
  const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ls), __float_as_uint(ls), false, false);
  const float l = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
  return l > 0.f ? 1.0f / l : 0.f;
}

}  // namespace tjk
