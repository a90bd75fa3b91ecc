// QKV projection, attention and out-projection of one layer in one launch,
// for sequences of at most 128 tokens.
//
// At such shapes (C2: one 128-token sequence, d = 512, 8 heads) each of the
// three launches this replaces -- the QKV GEMM (tjkernels/engine.py:245),
// attention (tjkernels/kernels/attention.py:189-226) and the out-projection
// GEMM (tjkernels/engine.py:247) -- is a chain of a few dependent memory
// round trips that leaves the GPU nearly idle for 5-8 us; the reference's
// remedy for tiny shapes is fusion (README.md:193-196).
//
// Workgroup (b, h, i), 4 waves: sequence b, head h (head_dim 64), query
// block i (32 queries).  With kend = the end of block i when causal, else
// the sequence length:
//
//   1. K and V of keys 0 .. kend-1 and Q of block i:
//        [Q | K | V] = x[rows] [Wq_h; Wk_h; Wv_h]^T + [bq_h, bk_h, bv_h]
//      with the x rows and the head's 192 weight rows streamed through a
//      three-slot LDS ring of 64-deep K chunks by LDS DMA (the GEMM's
//      direct-to-LDS scheme; rows past kend arrive as zeros), rounded to
//      the compute dtype as the QKV GEMM rounds its output.  Wave (a, c)
//      computes K (c = 0) or V (c = 1) of key blocks 2a and 2a+1 and, when
//      block i is one of them, half of Q.  V is computed with the MFMA
//      operands swapped, so it comes out transposed, as attention reads it.
//   2. ctx_i = softmax(Q K^T scale) V for the 32 queries, by the math of the
//      short-sequence attention kernel (tjk_flash_fwd plan 4; shared code),
//      rounded to the compute dtype.
//   3. P[h][rows of block i] = ctx_i W_out[:, 64h : 64h+64]^T (+ b_out for
//      h = 0), fp32, with the W_out fragments loaded before step 1.
//
// The H per-head partials are summed by the next add+LayerNorm in a fixed
// order (tjk_add_layernorm's delta_splits), like the single-launch FFN's
// f-slices: no workgroup waits for another and the result does not depend
// on timing.  K and V of the earlier query blocks are recomputed by every
// workgroup that needs them (at most 4x the K/V projection of one block);
// that costs less than a second launch or a wait between workgroups.

#include <type_traits>

#include "attn_short.h"
#include "gemm_tiles.h"

namespace tjk {

constexpr int kAbHd = 64;                     // head dim
constexpr int kAbMaxK = 128;                  // tokens per sequence
constexpr int kAbStages = 3;                  // LDS ring slots
constexpr int kAbBkb = 128;                   // bytes of K per ring row (64 elements)
constexpr int kAbARows = 128, kAbWRows = 192; // x rows, weight rows (Q | K | V) per slot
constexpr int kAbStage = (kAbARows + kAbWRows) * kAbBkb;
constexpr int kAbDA = kAbARows / 32, kAbDW = kAbWRows / 32;  // DMA instructions per wave and chunk
constexpr int kAbNdma = kAbDA + kAbDW;
constexpr int kAbMaxD = 512;                  // largest d_model taken

// LDS: the ring during step 1; afterwards the same bytes hold K rows, V^T,
// Q, ctx and the out-projection epilogue's per-wave staging.
template <typename T, int FNW>
struct AbLayout {
  static constexpr int D = 128 * FNW;          // d_model
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int LDK = kAbHd + VEC;       // K / Q / ctx row pitch (elements)
  static constexpr int LDV = kAbMaxK + VEC;     // V^T row pitch (elements)
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + kAbMaxK * LDK * (int)sizeof(T);
  static constexpr int Q_OFF = V_OFF + kAbHd * LDV * (int)sizeof(T);
  static constexpr int C_OFF = Q_OFF + 32 * LDK * (int)sizeof(T);
  static constexpr int E_OFF = C_OFF + 32 * LDK * (int)sizeof(T);
  static constexpr int EBYTES = EpiStage<T, kEpiStoreF32, FNW>::BYTES;
  static constexpr int AFTER = E_OFF + 4 * EBYTES;
  static constexpr int RING = kAbStages * kAbStage;
  // biases, copied in by DMA with the first K chunk: this head's
  // [bq | bk | bv] (3 x 64 elements, one 128-byte row each) and b_out
  static constexpr int BQKV_OFF = RING > AFTER ? RING : AFTER;
  static constexpr int BOUT_OFF = BQKV_OFF + 1024;
  static constexpr int LDS = BOUT_OFF + kAbMaxD * (int)sizeof(T);
  static_assert(V_OFF % 16 == 0 && Q_OFF % 16 == 0 && C_OFF % 16 == 0 && E_OFF % 16 == 0, "LDS alignment");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(D <= kAbMaxD, "zero-bias stand-in size");
};

template <typename T, int FNW>
__global__ __launch_bounds__(256) void attn_block_kernel(
    const T* __restrict__ x, int64_t ldx, const T* __restrict__ wqkv, const T* __restrict__ bqkv,
    const T* __restrict__ wout, const T* __restrict__ bout, float* __restrict__ parts, int64_t ldp,
    int64_t part_stride, T* __restrict__ ctx_out, int64_t ldc, const int32_t* __restrict__ cu_seqlens,
    int B, int S, int causal, float scale_log2, int nqb) {
  typedef AbLayout<T, FNW> Lay;
  typedef typename Mfma<T>::frag Frag;
  constexpr int D = Lay::D, H = D / kAbHd, LDK = Lay::LDK, LDV = Lay::LDV;
  __shared__ __attribute__((aligned(1024))) char smem[Lay::LDS];

  const int BH = B * H;
  const int rank = blockIdx.x / BH, bh = blockIdx.x % BH;
  const int qb = causal ? nqb - 1 - rank : rank;  // causal: most keys first
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so branches on it are scalar
  const int l32 = lane & 31, hi = lane >> 5;
  const int a = wave >> 1, c = wave & 1;          // key blocks 2a, 2a+1; K (c = 0) or V (c = 1)

  int L = S;
  int64_t r0 = (int64_t)b * S;
  if (cu_seqlens != nullptr) {
    r0 = max(cu_seqlens[b], 0);
    L = min(max(cu_seqlens[b + 1] - cu_seqlens[b], 0), S);  // bounded by the launch's sequence length
  }
  L = min(L, kAbMaxK);  // the entry point requires lengths <= 128; this keeps LDS indices in range
  const int q0 = 32 * qb;
  if (q0 >= L) return;  // whole workgroup, before any barrier
  const int kend = causal ? min(q0 + 32, L) : L;
  const int nkb = (kend + 31) / 32;
  const int nq = min(32, L - q0);
  const bool has_q = a == (qb >> 1);  // this wave pair holds block i's rows
  typedef typename Quad<T>::raw Raw;

  // ---- loads that depend on nothing: W_out fragments (B = W_out rows
  // n = nw0 + 32 cb + l32, K columns 64 h + 16 ks + 8 hi ..) and biases
  const int nw0 = wave * FNW * 32;
  Frag wo[FNW][4];
#pragma unroll
  for (int cb = 0; cb < FNW; ++cb)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      wo[cb][ks] = Mfma<T>::load(wout + (int64_t)(nw0 + 32 * cb + l32) * D + kAbHd * h + 16 * ks + 8 * hi);
  // ---- step 1: the projections through the LDS ring
  // x rows past kend fall outside the descriptor's range and arrive as 0.
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(x + r0 * ldx), (short)0, (int)((int64_t)kend * ldx * (int64_t)sizeof(T)), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wqkv, (short)0, (int)((int64_t)3 * D * D * (int64_t)sizeof(T)), 0x00020000);
  // DMA instruction q of this wave fills ring rows (q' * 4 + wave) * 8 + 0..7
  // of the x part (q < kAbDA, q' = q) or of the weight part (q' = q - kAbDA):
  // lane l lands at row + l / 8, physical chunk l % 8, and fetches logical
  // chunk (l % 8) ^ swz(row).  Weight row r of the slot is row
  // (r / 64) * D + 64 h + r % 64 of Wqkv (the Q, K and V rows of head h).
  uint32_t voff[kAbNdma];
#pragma unroll
  for (int q = 0; q < kAbDA; ++q) {
    const int r = (q * 4 + wave) * 8 + lane / 8;
    voff[q] = (uint32_t)((int64_t)r * ldx * (int64_t)sizeof(T)) + (uint32_t)(((lane % 8) ^ swz<kAbBkb>(r)) << 4);
  }
#pragma unroll
  for (int q = 0; q < kAbDW; ++q) {
    const int r = (q * 4 + wave) * 8 + lane / 8;
    const int grow = (r / kAbHd) * D + kAbHd * h + r % kAbHd;
    voff[kAbDA + q] = (uint32_t)(grow * D * (int)sizeof(T)) + (uint32_t)(((lane % 8) ^ swz<kAbBkb>(r)) << 4);
  }
  constexpr int NK = D / 64;  // K chunks
  auto dma = [&](int kt, int q) {
    char* sb = smem + (kt % kAbStages) * kAbStage;
    const uint32_t kb = kt < NK ? (uint32_t)(kt * kAbBkb) : (uint32_t)kPastEnd;
    if (q < kAbDA)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_void*)(sb + (q * 4 + wave) * 1024), 16, voff[q] + kb,
                                               0, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_void*)(sb + kAbARows * kAbBkb + ((q - kAbDA) * 4 + wave) * 1024),
                                               16, voff[q] + kb, 0, 0, 0);
  };

  f32x16 acc[2][2], accq;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc[0][0][r] = 0.f; acc[0][1][r] = 0.f; acc[1][0][r] = 0.f; acc[1][1][r] = 0.f;
    accq[r] = 0.f;
  }
  const int sw = swz<kAbBkb>(l32);
  auto frag = [&](const char* rowbase, int ks) -> Frag {
    return *reinterpret_cast<const Frag*>(rowbase + (((2 * ks + hi) ^ sw) << 4));
  };

  // The biases into LDS, ahead of chunk 0 (so the first wait covers them):
  // wave 0 copies [bq_h | bk_h | bv_h] (lane l: segment l / 8, 16-byte
  // piece l % 8; lanes past the three segments, or every lane without a
  // bias, fall outside the range and write zeros), wave 1 of head 0's
  // workgroups b_out (d elements, one piece per lane).
  if (wave == 0) {
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(bqkv != nullptr ? bqkv : wqkv), (short)0, bqkv != nullptr ? 3 * D * (int)sizeof(T) : 0, 0x00020000);
    const int seg = lane / 8;
    const uint32_t off = seg < 3 ? (uint32_t)((seg * D + kAbHd * h) * (int)sizeof(T) + (lane % 8) * 16)
                                 : (uint32_t)kPastEnd;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_void*)(smem + Lay::BQKV_OFF), 16, off, 0, 0, 0);
  } else if (wave == 1 && h == 0 && bout != nullptr) {
    const __amdgpu_buffer_rsrc_t rso = __builtin_amdgcn_make_buffer_rsrc(
        (void*)bout, (short)0, D * (int)sizeof(T), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rso, (lds_void*)(smem + Lay::BOUT_OFF), 16, (uint32_t)(lane * 16), 0, 0,
                                             0);
  }
#pragma unroll
  for (int t = 0; t < kAbStages - 1; ++t)
#pragma unroll
    for (int q = 0; q < kAbNdma; ++q) dma(t, q);
  // Every wave runs the same branch-free MFMA sequence: key blocks past
  // kend hold zero rows (their results are never read), and the Q product
  // of a wave pair that does not hold block i is discarded.
  auto project = [&](auto v_part) {
    constexpr bool VPART = decltype(v_part)::value;
    for (int kt = 0; kt < NK; ++kt) {
      // chunk kt has landed (chunk kt+1 may still be in flight) and every
      // wave is done reading chunk kt-1, whose slot chunk kt+2 then takes
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((kAbStages - 2) * kAbNdma) : "memory");
      asm volatile("s_barrier" ::: "memory");
#pragma unroll
      for (int q = 0; q < kAbNdma; ++q) dma(kt + kAbStages - 1, q);
      const char* sb = smem + (kt % kAbStages) * kAbStage;
      const char* xa = sb + (64 * a + l32) * kAbBkb;                           // x rows of key block 2a
      const char* wr = sb + kAbARows * kAbBkb + (64 + 64 * c + l32) * kAbBkb;  // K or V weight rows
      const char* wq = sb + kAbARows * kAbBkb + (32 * c + l32) * kAbBkb;       // Q weight rows, half c
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const Frag fa0 = frag(xa, ks), fa1 = frag(xa + 32 * kAbBkb, ks);
        const Frag fw0 = frag(wr, ks), fw1 = frag(wr + 32 * kAbBkb, ks), fq = frag(wq, ks);
        if constexpr (!VPART) {  // K^T blocks: lane = key, registers = head columns
          Mfma<T>::mma(acc[0][0], fw0, fa0); Mfma<T>::mma(acc[0][1], fw1, fa0);
          Mfma<T>::mma(acc[1][0], fw0, fa1); Mfma<T>::mma(acc[1][1], fw1, fa1);
        } else {                 // V blocks: lane = head column, registers = keys
          Mfma<T>::mma(acc[0][0], fa0, fw0); Mfma<T>::mma(acc[0][1], fa0, fw1);
          Mfma<T>::mma(acc[1][0], fa1, fw0); Mfma<T>::mma(acc[1][1], fa1, fw1);
        }
        Mfma<T>::mma(accq, fq, (qb & 1) ? fa1 : fa0);
      }
    }
  };
  if (c == 0)
    project(std::false_type{});
  else
    project(std::true_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the past-the-end DMAs write LDS too
  __syncthreads();

  // ---- step 1 results into LDS in the compute dtype
  T* sK = reinterpret_cast<T*>(smem + Lay::K_OFF);
  T* sV = reinterpret_cast<T*>(smem + Lay::V_OFF);
  T* sQ = reinterpret_cast<T*>(smem + Lay::Q_OFF);
  T* sC = reinterpret_cast<T*>(smem + Lay::C_OFF);
  const T* sB = reinterpret_cast<const T*>(smem + Lay::BQKV_OFF);  // [bq_h | bk_h | bv_h]
  float4 bk[2][4], bq[4];
  float bv[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) bk[cb][g] = Quad<T>::to(*reinterpret_cast<const Raw*>(&sB[64 + 32 * cb + 8 * g + 4 * hi]));
    bv[cb] = to_f32(sB[128 + 32 * cb + l32]);
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) bq[g] = Quad<T>::to(*reinterpret_cast<const Raw*>(&sB[32 * c + 8 * g + 4 * hi]));
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int kb0 = 32 * (2 * a + r);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16& v = acc[r][cb];
        if (c == 0) {  // key kb0 + l32, columns 32 cb + 8 g + 4 hi ..
          const float4 bb = bk[cb][g];
          const float4 o = make_float4(v[4 * g] + bb.x, v[4 * g + 1] + bb.y, v[4 * g + 2] + bb.z, v[4 * g + 3] + bb.w);
          *reinterpret_cast<Raw*>(&sK[(kb0 + l32) * LDK + 32 * cb + 8 * g + 4 * hi]) = Quad<T>::from(o);
        } else {       // column 32 cb + l32, keys kb0 + 8 g + 4 hi ..
          const float bb = bv[cb];
          const float4 o = make_float4(v[4 * g] + bb, v[4 * g + 1] + bb, v[4 * g + 2] + bb, v[4 * g + 3] + bb);
          *reinterpret_cast<Raw*>(&sV[(32 * cb + l32) * LDV + kb0 + 8 * g + 4 * hi]) = Quad<T>::from(o);
        }
      }
  }
  if (has_q) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 o = make_float4(accq[4 * g] + bq[g].x, accq[4 * g + 1] + bq[g].y, accq[4 * g + 2] + bq[g].z,
                                   accq[4 * g + 3] + bq[g].w);
      *reinterpret_cast<Raw*>(&sQ[l32 * LDK + 32 * c + 8 * g + 4 * hi]) = Quad<T>::from(o);
    }
  }
  __syncthreads();

  // ---- step 2: attention of the 32 queries (one wave)
  if (wave == 0) {
    Frag qf[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) qf[k] = Mfma<T>::load(&sQ[l32 * LDK + 16 * k + 8 * hi]);
    const int q = q0 + l32;
    const int lim = causal ? min(q + 1, kend) : kend;
    f32x16 o[2];
    const float inv = short_attention<T, kAbHd, kAbMaxK>(sK, sV, qf, nkb, lim, scale_log2,
                                                         [](int) { return true; }, o);
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = hb * 32 + 8 * g + 4 * hi;
        const Raw pc = Quad<T>::from(make_float4(o[hb][4 * g] * inv, o[hb][4 * g + 1] * inv,
                                                 o[hb][4 * g + 2] * inv, o[hb][4 * g + 3] * inv));
        *reinterpret_cast<Raw*>(&sC[l32 * LDK + col]) = pc;
        if (ctx_out != nullptr && q < L)
          *reinterpret_cast<Raw*>(ctx_out + (r0 + q) * ldc + kAbHd * h + col) = pc;
      }
  }
  __syncthreads();

  // ---- step 3: this head's share of the out-projection
  Frag cf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) cf[ks] = Mfma<T>::load(&sC[l32 * LDK + 16 * ks + 8 * hi]);
  f32x16 acc2[FNW][1];
#pragma unroll
  for (int cb = 0; cb < FNW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc2[cb][0][r] = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int cb = 0; cb < FNW; ++cb) Mfma<T>::mma(acc2[cb][0], wo[cb][ks], cf[ks]);
  const T* sBo = reinterpret_cast<const T*>(smem + Lay::BOUT_OFF);
  epilogue<T, kEpiStoreF32, 1, FNW>(acc2, h == 0 && bout != nullptr ? sBo : nullptr, parts + h * part_stride + (r0 + q0) * ldp, ldp,
                                    nq, D, 0, nw0, lane, smem + Lay::E_OFF + wave * Lay::EBYTES);
}

template <typename T>
static int launch_attn_block(const void* x, int64_t ldx, const void* wqkv, const void* bqkv, const void* wout,
                             const void* bout, float* parts, int64_t ldp, int64_t part_stride, void* ctx_out,
                             int64_t ldc, const int32_t* cu_seqlens, int B, int S, int d, int causal,
                             float scale_log2, hipStream_t st) {
  const int nqb = (S + 31) / 32;
  const int64_t nblk = (int64_t)nqb * B * (d / kAbHd);
  if (nblk > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_attn_block: grid too large");
#define TJK_AB_CASE(F)                                                                                          \
  case F:                                                                                                       \
    hipLaunchKernelGGL((attn_block_kernel<T, F>), dim3((unsigned)nblk), dim3(256), 0, st, (const T*)x, ldx,    \
                       (const T*)wqkv, (const T*)bqkv, (const T*)wout, (const T*)bout, parts, ldp, part_stride, \
                       (T*)ctx_out, ldc, cu_seqlens, B, S, causal, scale_log2, nqb);                            \
    break;
  switch (d / 128) {
    TJK_AB_CASE(1)
    TJK_AB_CASE(2)
    TJK_AB_CASE(3)
    TJK_AB_CASE(4)
    default:
      return fail(TJK_EUNSUPPORTED, "tjk_attn_block: d_model %d", d);
  }
#undef TJK_AB_CASE
  return check_launch("tjk_attn_block");
}

}  // namespace tjk

using namespace tjk;

extern "C" int tjk_attn_block_supported(int64_t d_model, int heads, int head_dim, int64_t max_seqlen, int dtype) {
  return (dtype == TJK_F16 || dtype == TJK_BF16) && head_dim == kAbHd && heads > 0 &&
         (int64_t)heads * head_dim == d_model && d_model % 128 == 0 && d_model <= 512 && max_seqlen >= 0 &&
         max_seqlen <= kAbMaxK;
}

extern "C" int tjk_attn_block(const void* x, int64_t ld_x, const void* w_qkv, const void* b_qkv,
                              const void* w_out, const void* b_out, float* parts, int64_t ld_parts,
                              int64_t part_stride, void* ctx_out, int64_t ld_ctx, const int32_t* cu_seqlens,
                              int batch, int seq, int heads, int head_dim, float scale, int causal, int dtype,
                              void* stream) {
  if (batch < 0 || seq < 0 || heads <= 0 || head_dim <= 0)
    return fail(TJK_EINVAL, "tjk_attn_block: bad shape B=%d S=%d H=%d hd=%d", batch, seq, heads, head_dim);
  const int64_t d = (int64_t)heads * head_dim;
  if (!tjk_attn_block_supported(d, heads, head_dim, seq, dtype))
    return fail(TJK_EUNSUPPORTED,
                "tjk_attn_block: takes bf16 / fp16, head_dim 64, d_model = 64 heads in {128, 256, 384, 512} and "
                "sequences of at most 128 tokens (got dtype %d, H=%d, hd=%d, S=%d)",
                dtype, heads, head_dim, seq);
  if (batch == 0 || seq == 0) return TJK_OK;
  if (!x || !w_qkv || !w_out || !parts) return fail(TJK_EINVAL, "tjk_attn_block: null pointer");
  if (ld_x < d || ld_x % 8 || ld_parts < d || ld_parts % 4 || part_stride % 4)
    return fail(TJK_EINVAL, "tjk_attn_block: bad leading dimension or part stride");
  if (ctx_out != nullptr && (ld_ctx < d || ld_ctx % 4))
    return fail(TJK_EINVAL, "tjk_attn_block: bad ld_ctx");
  if (((uintptr_t)x & 15) || ((uintptr_t)w_qkv & 15) || ((uintptr_t)w_out & 15) || ((uintptr_t)parts & 15) ||
      ((uintptr_t)b_qkv & 7) || ((uintptr_t)b_out & 7) || ((uintptr_t)ctx_out & 7))
    return fail(TJK_EUNSUPPORTED, "tjk_attn_block: misaligned pointer");
  if ((int64_t)kAbMaxK * ld_x * 2 > INT32_MAX) return fail(TJK_EUNSUPPORTED, "tjk_attn_block: ld_x too large");
  if (!(scale > 0.f)) return fail(TJK_EINVAL, "tjk_attn_block: scale must be positive");
  if (cu_seqlens == nullptr && (int64_t)batch * seq * ld_x > INT64_MAX / 4)
    return fail(TJK_EUNSUPPORTED, "tjk_attn_block: shape too large");
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == TJK_F16)
    return launch_attn_block<f16>(x, ld_x, w_qkv, b_qkv, w_out, b_out, parts, ld_parts, part_stride, ctx_out,
                                  ld_ctx, cu_seqlens, batch, seq, (int)d, causal, scale_log2, st);
  return launch_attn_block<bf16>(x, ld_x, w_qkv, b_qkv, w_out, b_out, parts, ld_parts, part_stride, ctx_out,
                                 ld_ctx, cu_seqlens, batch, seq, (int)d, causal, scale_log2, st);
}
