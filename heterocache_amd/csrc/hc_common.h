// Device-side building blocks shared by every libhc kernel (gfx950 / CDNA4).
//
// Ragged per-head KV store ("tiled head-major"):
//   Every (batch, kv-head) row owns a contiguous run of 32-token tiles inside
//   one per-layer K buffer and one per-layer V buffer.  A tile holds
//   32 tokens x 128 channels and is laid out so that one 16-byte load per lane
//   lands directly in the operand register of a 16x16x32 MFMA:
//
//   K tile element (t, d):  h=t/16 m=t%16 s=d/32 g=(d%32)/8 i=d%8
//                           offset = (((h*4 + s)*4 + g)*16 + m)*8 + i
//   V tile element (t, d):  mt=d/16 n=d%16 r=t%16 g=r/4 i=4*(t/16)+r%4
//                           offset = ((mt*4 + g)*16 + n)*8 + i
//
//   For K, MFMA step (h, s) reads lane l = g*16+m at ((h*4+s)*64 + l)*8: one
//   1 KB fully coalesced wave load.  For V, MFMA step mt reads lane
//   l = g*16+n at (mt*64 + l)*8, again 1 KB contiguous.  The V token order
//   inside a lane matches the order in which the Q.K^T MFMA leaves scores in
//   its accumulator, so P never moves between lanes.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define HC_HEAD_DIM 128
#define HC_TILE 32
#define HC_TILE_ELEMS (HC_TILE * HC_HEAD_DIM)

namespace hc {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

enum DType { F32 = 0, F16 = 1, BF16 = 2 };

__host__ __device__ __forceinline__ int64_t k_tile_offset(int t, int d) {
  int h = t >> 4, m = t & 15, s = d >> 5, g = (d >> 3) & 3, i = d & 7;
  return ((((h * 4 + s) * 4 + g) * 16 + m) * 8) + i;
}

__host__ __device__ __forceinline__ int64_t v_tile_offset(int t, int d) {
  int mt = d >> 4, n = d & 15, r = t & 15, g = r >> 2, i = ((t >> 4) << 2) | (r & 3);
  return (((mt * 4 + g) * 16 + n) * 8) + i;
}

// Element traits: storage type, 8-element lane vector and conversions.
template <typename T> struct Elem;

template <> struct Elem<__bf16> {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }
  static __device__ __forceinline__ __bf16 from_f32(float x) { return (__bf16)x; }
};
template <> struct Elem<_Float16> {
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
  static __device__ __forceinline__ _Float16 from_f32(float x) { return (_Float16)x; }
};
template <> struct Elem<float> {
  struct vec8 { f32x4 lo, hi; };
  static __device__ __forceinline__ float to_f32(float x) { return x; }
  static __device__ __forceinline__ float from_f32(float x) { return x; }
};

// Load 8 consecutive elements (16 B for 16-bit types, 32 B for fp32).
template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 load8(const T* p) {
  return *reinterpret_cast<const typename Elem<T>::vec8*>(p);
}
template <>
__device__ __forceinline__ Elem<float>::vec8 load8<float>(const float* p) {
  Elem<float>::vec8 r;
  r.lo = *reinterpret_cast<const f32x4*>(p);
  r.hi = *reinterpret_cast<const f32x4*>(p + 4);
  return r;
}

// Streaming variant of load8 for data read once per launch (KV tiles): the
// nontemporal hint keeps the stream from displacing reusable lines in L2.
template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 load8_stream(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename Elem<T>::vec8*>(p));
}
template <>
__device__ __forceinline__ Elem<float>::vec8 load8_stream<float>(const float* p) {
  Elem<float>::vec8 r;
  r.lo = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  r.hi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
  return r;
}

// load8_stream for a pointer the compiler cannot place in global memory by
// itself (one made from a device address passed as an integer): a generic
// pointer makes a flat load, which counts against both the vector-memory and
// the LDS wait counters, so each wait on it also waits for every LDS access.
// The cast tells the compiler the address is global.
template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 load8_stream_global(const T* p) {
  typedef __attribute__((address_space(1))) const typename Elem<T>::vec8 GV;
  return __builtin_nontemporal_load((GV*)p);
}
template <>
__device__ __forceinline__ Elem<float>::vec8 load8_stream_global<float>(const float* p) {
  typedef __attribute__((address_space(1))) const f32x4 GV;
  Elem<float>::vec8 r;
  r.lo = __builtin_nontemporal_load((GV*)p);
  r.hi = __builtin_nontemporal_load((GV*)(p + 4));
  return r;
}

// acc += A(16x32) * B(32x16) where each lane supplies 8 k-values of its row
// (A) / column (B): lane l owns row/col l%16 and k-slots 8*(l/16)+[0..8).
// For fp32 the same 32-wide contraction is issued as 8 x (16x16x4) MFMAs in
// which step e covers k-slots {8g+e : g=0..3}; the result is identical up to
// summation order.
__device__ __forceinline__ f32x4 mma_16x16x32(bf16x8 a, bf16x8 b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma_16x16x32(f16x8 a, f16x8 b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma_16x16x32(Elem<float>::vec8 a, Elem<float>::vec8 b, f32x4 acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[e], b.lo[e], acc, 0, 0, 0);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[e], b.hi[e], acc, 0, 0, 0);
  return acc;
}

// Pack 8 fp32 values into the lane vector of T (round-to-nearest-even).
template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 pack8(const float (&v)[8]) {
  typename Elem<T>::vec8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = Elem<T>::from_f32(v[e]);
  return r;
}
template <>
__device__ __forceinline__ Elem<float>::vec8 pack8<float>(const float (&v)[8]) {
  Elem<float>::vec8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) { r.lo[e] = v[e]; r.hi[e] = v[e + 4]; }
  return r;
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 zero8() {
  float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  return pack8<T>(z);
}

// Element e of a lane vector as fp32 (e must be a compile-time constant
// after unrolling, so the vector stays in registers).
template <typename T>
__device__ __forceinline__ float vec8_at(const typename Elem<T>::vec8& v, int e) {
  return Elem<T>::to_f32(v[e]);
}
template <>
__device__ __forceinline__ float vec8_at<float>(const Elem<float>::vec8& v, int e) {
  return e < 4 ? v.lo[e] : v.hi[e - 4];
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Rounding of the reference's casts to the model dtype, fixed per kernel
// instance: 0 none, 1 bfloat16, 2 float16.
template <int RM>
__device__ __forceinline__ float round_fixed(float x) {
  if constexpr (RM == 1) return (float)(__bf16)x;
  if constexpr (RM == 2) return (float)(_Float16)x;
  return x;
}

// Sum of a value over the 16 lanes of its row (lanes 16r .. 16r+15), in
// every lane of the row: four DPP adds (rotate the row by 8 and by 4, then
// swap within quads by 2 and by 1), full rate on the VALU, where a
// __shfl_xor butterfly goes through the LDS crossbar once per step.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sums over the 16 lanes of each 16-lane row of a wave, for NR values per
// lane at once (NR = 4, 8 or 16): lane l ends with its row's sum of value
// l % NR.  A reduce-scatter: at each of the first log2(NR) stages a lane
// keeps the half of its values whose index bit equals its own lane bit and
// adds the copy of that half sent by a lane whose bit differs -- l ^ 1 and
// l ^ 2 by quad permutes, then a row rotation by 4 and one by 8 (a rotated
// lane holds the same values as l ^ 4 or l ^ 8, and the later stages
// gather the remaining quads whichever way the rotation turns) -- so the
// values held halve at every stage; rotations by 8 and 4 sum what is left.
// 16 operations at NR = 4 where separate sums of each value take 32.
template <int NR>
__device__ __forceinline__ float row16_sum_scatter(float (&a)[NR], int lane) {
  static_assert(NR == 4 || NR == 8 || NR == 16, "4, 8 or 16 values per lane");
  {
    const bool b = lane & 1;
#pragma unroll
    for (int j = 0; j < NR / 2; ++j) {
      const float keep = b ? a[2 * j + 1] : a[2 * j], send = b ? a[2 * j] : a[2 * j + 1];
      a[j] = keep + dpp_mov<0xB1>(send);  // quad_perm [1,0,3,2]
    }
  }
  {
    const bool b = lane & 2;
#pragma unroll
    for (int j = 0; j < NR / 4; ++j) {
      const float keep = b ? a[2 * j + 1] : a[2 * j], send = b ? a[2 * j] : a[2 * j + 1];
      a[j] = keep + dpp_mov<0x4E>(send);  // quad_perm [2,3,0,1]
    }
  }
  if constexpr (NR >= 8) {
    const bool b = lane & 4;
#pragma unroll
    for (int j = 0; j < NR / 8; ++j) {
      const float keep = b ? a[2 * j + 1] : a[2 * j], send = b ? a[2 * j] : a[2 * j + 1];
      a[j] = keep + dpp_mov<0x124>(send);  // row_ror:4
    }
  }
  if constexpr (NR == 16) {
    const bool b = lane & 8;
    const float keep = b ? a[1] : a[0], send = b ? a[0] : a[1];
    return keep + dpp_mov<0x128>(send);  // row_ror:8
  } else if constexpr (NR == 8) {
    return a[0] + dpp_mov<0x128>(a[0]);
  } else {
    const float v = a[0] + dpp_mov<0x128>(a[0]);
    return v + dpp_mov<0x124>(v);
  }
}

// Combine a value over the four lanes l, l^16, l^32, l^48 of a wave (one
// lane per 16-lane row), as the MFMA layouts need for a per-column max or
// sum.  gfx950's row swaps (v_permlane16_swap / v_permlane32_swap) move the
// data between VGPRs without an LDS round trip.  With both operands equal,
// each swap hands every lane its own value and its partner's (l^16, then
// l^32) as the two results, in a lane-dependent order; max and + are
// commutative, so the result equals that of the xor-shuffle form bit for bit.
// The maximum is IEEE maximum (NaN-propagating; one instruction, where
// fmaxf first canonicalises operands it cannot prove canonical).
__device__ __forceinline__ float rows4_max(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float w = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned uw = __float_as_uint(w);
  const auto b = __builtin_amdgcn_permlane32_swap(uw, uw, false, false);
  return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// Sum over the two lanes l and l^16 (row swap only).
__device__ __forceinline__ float rows2_sum(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float rows4_sum(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float w = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned uw = __float_as_uint(w);
  const auto b = __builtin_amdgcn_permlane32_swap(uw, uw, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Order-preserving uint32 key of a float score (larger float, larger key;
// -0 ranks equal to +0), used by every selection over scores.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Width of the first digit of the drift check's selection: the histogram
// the scorer builds over its scores' top kKeyDigitBits key bits.
constexpr int kKeyDigitBits = 12;
constexpr int kKeyDigitBins = 1 << kKeyDigitBits;
constexpr int kKeyDigitShift = 32 - kKeyDigitBits;

}  // namespace hc
