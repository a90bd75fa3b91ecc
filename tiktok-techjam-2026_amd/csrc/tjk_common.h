// Shared definitions for the gfx950 kernels behind the tjk C-ABI.
//
// Element types, 16-byte chunk helpers, MFMA fragment traits and the
// thread-local error string returned by tjk_last_error_string().
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tjk.h"

namespace tjk {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Records a formatted message for tjk_last_error_string() and returns `code`.
int fail(int code, const char* fmt, ...);

// A buffer descriptor over the bytes [base, base + bytes) of a wave-uniform
// address (bytes clamped to [0, 2^31 - 1]).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wave_rsrc(const void* base, int64_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)(bytes < 0 ? 0 : bytes > 0x7fffffff ? 0x7fffffff : bytes));
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, n, 0x00020000);
}

// Output stores of launches that write at least kWtMinBytes go out with the
// sc1 cache policy: written through the L2 to memory as they are issued.  A
// plain store leaves its line dirty in the L2, and the release at the end of
// the kernel writes every dirty line back after the last tile; written
// through, that traffic overlaps the work still running.  Measured on
// MI355X at the packed C4 shapes: each GEMM 0.9-2.7 us and the LayerNorm
// 1.5 us faster per launch.  Below the threshold (launches of a few hundred
// rows) the write-through acknowledgements lengthen the launch instead.
// Only whole-line row segments: scattered pieces of a line are cheaper
// combined in the L2.
constexpr int kStoreWt = 16;
constexpr int64_t kWtMinBytes = 4 << 20;

// Stores of 8- or 16-byte pieces at byte offsets of a row segment: plain,
// or through a descriptor with the write-through policy.
struct PlainRow {
  char* p;
  template <typename Raw>
  __device__ __forceinline__ void put(int off, const Raw& v) const {
    *reinterpret_cast<Raw*>(p + off) = v;
  }
};
struct WtRow {
  __amdgpu_buffer_rsrc_t r;
  template <typename Raw>
  __device__ __forceinline__ void put(int off, const Raw& v) const {
    static_assert(sizeof(Raw) == 8 || sizeof(Raw) == 16, "8- or 16-byte pieces");
    if constexpr (sizeof(Raw) == 16)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kStoreWt);
    else
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, kStoreWt);
  }
};

// A wave's output row segment of `bytes` bytes at a wave-uniform address,
// and the launch's write-through choice.  Callers branch on `wt` once,
// around a whole store loop (with_wt), and store through writer<WT>(), so
// each loop is straight-line code and the plain one builds no descriptor.
struct RowOut {
  char* p;
  int64_t bytes;
  bool wt;
  __device__ __forceinline__ RowOut(void* base, int64_t nbytes, bool write_through)
      : p(static_cast<char*>(base)), bytes(nbytes), wt(write_through) {}
  template <bool WT>
  __device__ __forceinline__ auto writer() const {
    if constexpr (WT)
      return WtRow{wave_rsrc(p, bytes)};
    else
      return PlainRow{p};
  }
};

// Runs f(std::true_type) or f(std::false_type) as `wt` says.
template <typename F>
__device__ __forceinline__ void with_wt(bool wt, F&& f) {
  if (wt)
    f(std::true_type{});
  else
    f(std::false_type{});
}

// Maps a hipError_t to the C-ABI status (positive = HIP error code).
inline int hip_status(hipError_t e) {
  return e == hipSuccess ? TJK_OK : static_cast<int>(e);
}

// Launch-error check shared by every entry point.
int check_launch(const char* what);

inline int dtype_size(int dt) { return dt == TJK_F32 ? 4 : 2; }

// ---------------------------------------------------------------- scalars

template <typename T> __device__ __forceinline__ float to_f32(T v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }

// Four consecutive elements <-> float4 (8 bytes for 2-byte types, 16 for fp32).
template <typename T> struct Quad;
template <> struct Quad<float> {
  typedef float4 raw;
  static __device__ __forceinline__ float4 to(raw r) { return r; }
  static __device__ __forceinline__ raw from(float4 v) { return v; }
};
template <> struct Quad<bf16> {
  typedef uint2 raw;
  static __device__ __forceinline__ float4 to(raw r) {
    float4 v;
    v.x = __uint_as_float(r.x << 16);
    v.y = __uint_as_float(r.x & 0xffff0000u);
    v.z = __uint_as_float(r.y << 16);
    v.w = __uint_as_float(r.y & 0xffff0000u);
    return v;
  }
  static __device__ __forceinline__ raw from(float4 v) {
    bf16 a = static_cast<bf16>(v.x), b = static_cast<bf16>(v.y);
    bf16 c = static_cast<bf16>(v.z), d = static_cast<bf16>(v.w);
    raw r;
    r.x = (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    r.y = (uint32_t)__builtin_bit_cast(uint16_t, c) | ((uint32_t)__builtin_bit_cast(uint16_t, d) << 16);
    return r;
  }
};
template <> struct Quad<f16> {
  typedef uint2 raw;
  static __device__ __forceinline__ float4 to(raw r) {
    f16 a = __builtin_bit_cast(f16, (uint16_t)(r.x & 0xffff));
    f16 b = __builtin_bit_cast(f16, (uint16_t)(r.x >> 16));
    f16 c = __builtin_bit_cast(f16, (uint16_t)(r.y & 0xffff));
    f16 d = __builtin_bit_cast(f16, (uint16_t)(r.y >> 16));
    return make_float4((float)a, (float)b, (float)c, (float)d);
  }
  static __device__ __forceinline__ raw from(float4 v) {
    f16 a = (f16)v.x, b = (f16)v.y, c = (f16)v.z, d = (f16)v.w;
    raw r;
    r.x = (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    r.y = (uint32_t)__builtin_bit_cast(uint16_t, c) | ((uint32_t)__builtin_bit_cast(uint16_t, d) << 16);
    return r;
  }
};

// ------------------------------------------------------------ MFMA traits
//
// A "fragment" is the slice of one 32x32 MFMA operand that one lane owns for
// a 16-deep contraction step: 8 consecutive elements along K.  For 2-byte
// types that is one v_mfma_f32_32x32x16_{bf16,f16}; for fp32 it is eight
// v_mfma_f32_32x32x2_f32, sub-step j contracting element j of every lane.
// Any assignment of K indices to (lane half, element) is valid as long as
// both operands use the same one, which every caller below does.
//
// The 32x32 fp32 accumulator layout (all 32x32 MFMAs): lane l, register r
// holds row 8*(r/4) + 4*(l/32) + (r%4), column l%32.

template <typename T> struct Mfma;

template <> struct Mfma<bf16> {
  typedef bf16x8 frag;
  static constexpr int kVec = 8;  // elements per 16-byte chunk
  static __device__ __forceinline__ void mma(f32x16& acc, const frag& a, const frag& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
  static __device__ __forceinline__ frag load(const bf16* p) {  // 16-byte aligned
    return *reinterpret_cast<const frag*>(p);
  }
  static __device__ __forceinline__ frag pack(const float* v) {
    frag f;
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = static_cast<bf16>(v[i]);
    return f;
  }
  // acc + sum of the 8 elements, two per v_dot2c_f32_bf16
  static __device__ __forceinline__ float sum8(const frag& f, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {static_cast<bf16>(1.0f), static_cast<bf16>(1.0f)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2 pr = {f[2 * i], f[2 * i + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
    }
    return acc;
  }
};

template <> struct Mfma<f16> {
  typedef f16x8 frag;
  static constexpr int kVec = 8;
  static __device__ __forceinline__ void mma(f32x16& acc, const frag& a, const frag& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
  static __device__ __forceinline__ frag load(const f16* p) {
    return *reinterpret_cast<const frag*>(p);
  }
  static __device__ __forceinline__ frag pack(const float* v) {
    frag f;
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = static_cast<f16>(v[i]);
    return f;
  }
  // acc + sum of the 8 elements, two per v_dot2c_f32_f16
  static __device__ __forceinline__ float sum8(const frag& f, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {static_cast<f16>(1.0f), static_cast<f16>(1.0f)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2 pr = {f[2 * i], f[2 * i + 1]};
      acc = __builtin_amdgcn_fdot2(pr, one, acc, false);
    }
    return acc;
  }
};

template <> struct Mfma<float> {
  typedef f32x8 frag;
  static constexpr int kVec = 4;
  static __device__ __forceinline__ void mma(f32x16& acc, const frag& a, const frag& b) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], acc, 0, 0, 0);
  }
  static __device__ __forceinline__ frag load(const float* p) {  // 16-byte aligned
    float4 lo = *reinterpret_cast<const float4*>(p);
    float4 hi = *reinterpret_cast<const float4*>(p + 4);
    frag f;
    f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
    f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
    return f;
  }
  static __device__ __forceinline__ frag pack(const float* v) {
    frag f;
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = v[i];
    return f;
  }
  static __device__ __forceinline__ float sum8(const frag& f, float acc) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += f[i];
    return acc;
  }
};

// Sum over the 64 lanes of a wave (all lanes active), returned in every
// lane.  DPP moves sum
// each 16-lane row (xor 1, xor 2, mirror within 8, mirror within 16), then
// the four row sums are read out as scalars: a few VALU cycles per step,
// where a __shfl_xor butterfly goes through the LDS crossbar (ds_bpermute)
// six times.
__device__ __forceinline__ float wave_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
  const int iv = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return (r0 + r1) + (r2 + r3);
}

// wave_sum of N independent values at once: each value goes through
// exactly wave_sum's operations (same results, bit for bit), with the N
// DPP chains interleaved so their latencies overlap.
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0xB1, 0xF, 0xF, true));
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0x4E, 0xF, 0xF, true));
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0x141, 0xF, 0xF, true));
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0x140, 0xF, 0xF, true));
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int iv = __builtin_bit_cast(int, v[i]);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
    v[i] = (r0 + r1) + (r2 + r3);
  }
}

}  // namespace tjk
