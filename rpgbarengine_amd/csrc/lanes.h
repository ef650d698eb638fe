// Cross-lane steps of a 64-lane wave on the VALU: DPP row permutes and the
// gfx950 permlane swaps, in place of shuffles through the LDS pipe (which
// cost an LDS round trip and a wait each).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rpg {
namespace lanes {

// DPP controls: quad permutes (lane ^ 1, lane ^ 2), mirrors within 8 and 16
// lanes, rotate by 8 within 16 lanes (lane ^ 8 for lanes 0..7 and 8..15).
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowHalfMirror = 0x141, kRowMirror = 0x140, kRowRor8 = 0x128;

template <int kCtrl>
__device__ __forceinline__ uint32_t Dpp(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ float DppF(float v) {
  return __uint_as_float(Dpp<kCtrl>(__float_as_uint(v)));
}
template <int kCtrl>
__device__ __forceinline__ double DppD(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t r = Dpp<kCtrl>(static_cast<uint32_t>(b)) |
                     (static_cast<uint64_t>(Dpp<kCtrl>(static_cast<uint32_t>(b >> 32))) << 32);
  return __builtin_bit_cast(double, r);
}

__device__ __forceinline__ float ReadLaneF(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double ReadLaneD(double v, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b), lane));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane));
  return __builtin_bit_cast(double, lo | (hi << 32));
}

// v + v of the lane 16 (32) apart: rows r and r ^ 1 (halves) swapped; both
// lanes of a pair add the same two values.
__device__ __forceinline__ float AddXor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float AddXor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float MaxXor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float MaxXor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// A launch argument read into scalar registers at this point: the prologue's
// argument loads then share one round trip instead of trailing the
// branches that first use them.
template <typename T>
__device__ __forceinline__ T Uniform(T v) {
  asm volatile("" : "+s"(v));
  return v;
}

// Pointer arguments read now, kept in the global (or, for a value every lane
// reads, scalar constant) address space: a pinned generic pointer would
// turn its accesses into flat ones, which also hold up every LDS wait.
template <typename T>
using GlobalPtr = __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ GlobalPtr<T> UniformGlobal(T* p) {
  return (GlobalPtr<T>)Uniform(reinterpret_cast<uintptr_t>(p));
}
// *p, uniform over the wave, by a scalar load
template <typename T>
__device__ __forceinline__ T UniformRead(const T* p) {
  return *(const __attribute__((address_space(4))) T*)Uniform(reinterpret_cast<uintptr_t>(p));
}

// DPP / readlane of any 4- or 8-byte type.
template <int kCtrl, typename T>
__device__ __forceinline__ T DppT(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, Dpp<kCtrl>(__builtin_bit_cast(uint32_t, v)));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t r = Dpp<kCtrl>(static_cast<uint32_t>(b)) |
                       (static_cast<uint64_t>(Dpp<kCtrl>(static_cast<uint32_t>(b >> 32))) << 32);
    return __builtin_bit_cast(T, r);
  }
}
template <typename T>
__device__ __forceinline__ T ReadLaneT(T v, int lane) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b), lane));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane));
    return __builtin_bit_cast(T, lo | (hi << 32));
  }
}

// DPP with a row mask; lanes whose source lies outside their row, and rows
// outside the mask, read zero.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t DppZ(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, kRowMask, 0xF, true));
}
template <int kCtrl, int kRowMask, typename T>
__device__ __forceinline__ T DppZT(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, DppZ<kCtrl, kRowMask>(__builtin_bit_cast(uint32_t, v)));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t r = DppZ<kCtrl, kRowMask>(static_cast<uint32_t>(b)) |
                       (static_cast<uint64_t>(DppZ<kCtrl, kRowMask>(static_cast<uint32_t>(b >> 32))) << 32);
    return __builtin_bit_cast(T, r);
  }
}

// Inclusive prefix sum over the wave, lane i getting lanes 0..i (every lane
// active; integer types, so the sums are exact): shifts by 1, 2, 4, 8 within
// 16-lane rows, then row 15's sum into rows 1 and 3 and lane 31's into rows
// 2 and 3.
template <typename T>
__device__ __forceinline__ T WaveInclusiveAdd(T v) {
  v += DppZT<0x111, 0xF>(v);  // row_shr:1
  v += DppZT<0x112, 0xF>(v);  // row_shr:2
  v += DppZT<0x114, 0xF>(v);  // row_shr:4
  v += DppZT<0x118, 0xF>(v);  // row_shr:8
  v += DppZT<0x142, 0xA>(v);  // row_bcast:15
  v += DppZT<0x143, 0xC>(v);  // row_bcast:31
  return v;
}

// op over the wave (every lane active, every lane gets the result), in a
// fixed order: within 16-lane rows by DPP, then the four row values.
template <typename T, typename Op>
__device__ __forceinline__ T WaveReduce(T v, Op op) {
  v = op(v, DppT<kQuadXor1>(v));
  v = op(v, DppT<kQuadXor2>(v));
  v = op(v, DppT<kRowHalfMirror>(v));
  v = op(v, DppT<kRowMirror>(v));
  return op(op(ReadLaneT(v, 0), ReadLaneT(v, 16)), op(ReadLaneT(v, 32), ReadLaneT(v, 48)));
}

// Wave reductions (every lane active, every lane gets the result), in a
// fixed order: within 16-lane rows by DPP, then the four row values.
__device__ __forceinline__ double WaveSumD(double v) {
  v += DppD<kQuadXor1>(v);
  v += DppD<kQuadXor2>(v);
  v += DppD<kRowHalfMirror>(v);
  v += DppD<kRowMirror>(v);
  return (ReadLaneD(v, 0) + ReadLaneD(v, 16)) + (ReadLaneD(v, 32) + ReadLaneD(v, 48));
}
__device__ __forceinline__ float WaveSumF(float v) {
  v += DppF<kQuadXor1>(v);
  v += DppF<kQuadXor2>(v);
  v += DppF<kRowHalfMirror>(v);
  v += DppF<kRowMirror>(v);
  return (ReadLaneF(v, 0) + ReadLaneF(v, 16)) + (ReadLaneF(v, 32) + ReadLaneF(v, 48));
}
__device__ __forceinline__ float WaveMaxF(float v) {
  v = fmaxf(v, DppF<kQuadXor1>(v));
  v = fmaxf(v, DppF<kQuadXor2>(v));
  v = fmaxf(v, DppF<kRowHalfMirror>(v));
  v = fmaxf(v, DppF<kRowMirror>(v));
  return fmaxf(fmaxf(ReadLaneF(v, 0), ReadLaneF(v, 16)), fmaxf(ReadLaneF(v, 32), ReadLaneF(v, 48)));
}

}  // namespace lanes
}  // namespace rpg
