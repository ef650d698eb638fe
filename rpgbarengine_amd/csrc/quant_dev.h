// Device-side GGUF block decoding for gfx950 (Q8_0, Q4_K, Q6_K, F32).
//
// Bit-exactness contract with the reference's scalar DequantizeRow
// (reference src/quant.cc:132-142, :252-279, :321-354), used by the dequant and
// embedding kernels:
//   Q8_0  w = float(q) * d
//   Q4_K  w = (d*sc)*float(nib) - (dmin*m)     product rounded, then difference
//   Q6_K  w = (d*float(sc)) * float(q - 32)
// hipcc contracts a*b-c into an FMA by default, so the exact variants spell the
// roundings out with __fmul_rn / __fsub_rn.
//
// The fused dot kernels use a 32-weight "unit" per lane:
//   Q8_0  unit = one 34-byte block (32 consecutive weights)
//   Q4_K  unit = (block, group g, half h): 16 quant bytes -> 16 low-nibble
//         weights at 64g+16h+[0,16) and 16 high-nibble weights at +32
//   Q6_K  unit = (block, half, j): ql/qh bytes for l = 8j..8j+7 -> weights at
//         128*half + l + {0, 32, 64, 96}
//   F32   unit = 32 consecutive floats
// and form weights as fma(d*sc, nib, -(dmin*m)) for Q4_K (the reference AVX2
// kernel's fmsub, reference src/matmul_avx2.cc:86-89) -- dots are judged by the
// max|d|/sum|a*w| <= 1e-6 bound, not bitwise.

#ifndef RPG_HIP_QUANT_DEV_H_
#define RPG_HIP_QUANT_DEV_H_

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rpg {
namespace dev {

// fp16 bits -> fp32, bit-exact for every input including NaN payloads and
// subnormals (reference src/dtypes.h:21-47 semantics).
__device__ __forceinline__ float HalfBitsToFloat(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      const uint32_t sh = __clz(m) - 21;  // bring the leading 1 to bit 10
      m <<= sh;
      bits = sign | ((113u - sh) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  return __uint_as_float(bits);
}

// Hardware conversion: identical to HalfBitsToFloat for every non-NaN input.
__device__ __forceinline__ float HalfToFloatFast(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

__device__ __forceinline__ uint32_t Byte(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

__device__ __forceinline__ uint32_t LoadU16(const uint8_t* p) {
  return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
}

// 8 bytes from an address that is only 2-byte aligned.
__device__ __forceinline__ uint2 Load8Unaligned(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = static_cast<uint32_t>(a & 3u);
  const uint32_t w0 = base[0], w1 = base[1];
  if (sh == 0) return make_uint2(w0, w1);
  const uint32_t w2 = base[2];
  return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// Q4_K 6-bit scale/min unpack (reference src/quant.cc:159-167) from the 12
// packed bytes held in three dwords s0 = bytes 0..3, s1 = 4..7, s2 = 8..11.
__device__ __forceinline__ void ScaleMinK4(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t* sc,
                                           uint32_t* mn) {
  if (j < 4) {
    *sc = Byte(s0, j) & 63u;
    *mn = Byte(s1, j) & 63u;
  } else {
    const int k = j - 4;
    *sc = (Byte(s2, k) & 0x0Fu) | ((Byte(s0, k) >> 6) << 4);
    *mn = (Byte(s2, k) >> 4) | ((Byte(s1, k) >> 6) << 4);
  }
}

// ---------------------------------------------------------------- bit-exact dequant

// Per-element exact dequant: element e of a row (used by the gather kernels;
// one thread per element keeps them trivially parallel).
__device__ __forceinline__ float DequantQ8_0Exact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 5) * 34;
  const float d = HalfBitsToFloat(LoadU16(blk));
  const int8_t q = static_cast<int8_t>(blk[2 + (e & 31)]);
  return __fmul_rn(static_cast<float>(q), d);
}

__device__ __forceinline__ float DequantQ4_KExact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 8) * 144;
  const int i = static_cast<int>(e & 255);
  const int g = i >> 6;          // 64-element group
  const int hi = (i >> 5) & 1;   // second 32 of the group -> high nibbles
  const int l = i & 31;
  const float d = HalfBitsToFloat(LoadU16(blk));
  const float dmin = HalfBitsToFloat(LoadU16(blk + 2));
  uint32_t s0, s1, s2;
  __builtin_memcpy(&s0, blk + 4, 4);
  __builtin_memcpy(&s1, blk + 8, 4);
  __builtin_memcpy(&s2, blk + 12, 4);
  uint32_t sc, mn;
  ScaleMinK4(2 * g + hi, s0, s1, s2, &sc, &mn);
  const uint32_t qb = blk[16 + 32 * g + l];
  const uint32_t nib = hi ? (qb >> 4) : (qb & 0x0Fu);
  const float d1 = __fmul_rn(d, static_cast<float>(sc));
  const float m1 = __fmul_rn(dmin, static_cast<float>(mn));
  return __fsub_rn(__fmul_rn(d1, static_cast<float>(nib)), m1);
}

__device__ __forceinline__ float DequantQ6_KExact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 8) * 210;
  const int i = static_cast<int>(e & 255);
  const int half = i >> 7;
  const int r = i & 127;
  const int k = r >> 5;   // which of the four 32-strips
  const int l = r & 31;
  const uint8_t* ql = blk + 64 * half;
  const uint8_t* qh = blk + 128 + 32 * half;
  const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192) + 8 * half;
  const float d = HalfBitsToFloat(LoadU16(blk + 208));
  const uint32_t lo = (k & 1) ? ql[l + 32] : ql[l];
  const uint32_t low4 = (k >> 1) ? (lo >> 4) : (lo & 0x0Fu);
  const uint32_t high2 = (qh[l] >> (2 * k)) & 3u;
  const int q = static_cast<int>(low4 | (high2 << 4)) - 32;
  const float s = __fmul_rn(d, static_cast<float>(sc[(l >> 4) + 2 * k]));
  return __fmul_rn(s, static_cast<float>(q));
}

// The other ggml types, element e of a row, with the reference's operation
// order (each product and sum rounded on its own: no contraction).
__device__ __forceinline__ uint32_t LoadU32(const uint8_t* p) {
  return LoadU16(p) | (LoadU16(p + 2) << 16);
}

// 32-element blocks: code = nibble j (j < 16: low nibble of qs[j], else high
// nibble of qs[j - 16]) plus bit j of the 32-bit qh as bit 4 for Q5_0 / Q5_1
// (reference src/quant.cc:66-130); Q8_1 int8 codes (:144-155).
__device__ __forceinline__ uint32_t Nibble32(const uint8_t* qs, int j) {
  return j < 16 ? (qs[j] & 0x0Fu) : (qs[j - 16] >> 4);
}

__device__ __forceinline__ float DequantQ4_0Exact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 5) * 18;
  const int q = static_cast<int>(Nibble32(blk + 2, static_cast<int>(e & 31))) - 8;
  return __fmul_rn(static_cast<float>(q), HalfBitsToFloat(LoadU16(blk)));
}

__device__ __forceinline__ float DequantQ4_1Exact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 5) * 20;
  const uint32_t q = Nibble32(blk + 4, static_cast<int>(e & 31));
  return __fadd_rn(__fmul_rn(static_cast<float>(q), HalfBitsToFloat(LoadU16(blk))), HalfBitsToFloat(LoadU16(blk + 2)));
}

__device__ __forceinline__ float DequantQ5_0Exact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 5) * 22;
  const int j = static_cast<int>(e & 31);
  const uint32_t q = Nibble32(blk + 6, j) | (((LoadU32(blk + 2) >> j) & 1u) << 4);
  return __fmul_rn(static_cast<float>(static_cast<int>(q) - 16), HalfBitsToFloat(LoadU16(blk)));
}

__device__ __forceinline__ float DequantQ5_1Exact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 5) * 24;
  const int j = static_cast<int>(e & 31);
  const uint32_t q = Nibble32(blk + 8, j) | (((LoadU32(blk + 4) >> j) & 1u) << 4);
  return __fadd_rn(__fmul_rn(static_cast<float>(q), HalfBitsToFloat(LoadU16(blk))), HalfBitsToFloat(LoadU16(blk + 2)));
}

__device__ __forceinline__ float DequantQ8_1Exact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 5) * 36;
  const int8_t q = static_cast<int8_t>(blk[4 + (e & 31)]);
  return __fmul_rn(static_cast<float>(q), HalfBitsToFloat(LoadU16(blk)));
}

// Q2_K / Q3_K: element i = 128h + 32j + 16k + l of a super-block reads bits
// 2j of qs[32h + 16k + l] and sub-block scale 8h + 2j + k (reference
// src/quant.cc:169-250). Q3_K's high bit is bit 4h + j of hmask[16k + l], its
// 6-bit scale sits in the 12 packed bytes as the kmask unpack of :231-238
// leaves it: low nibble from byte 4*(s/4 % 2) + s%4 (high nibble when s >= 8),
// top two bits from byte 8 + s%4 at bit 2*(s/4).
__device__ __forceinline__ float DequantQ2_KExact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 8) * 84;
  const int i = static_cast<int>(e & 255), h = i >> 7, j = (i >> 5) & 3, k = (i >> 4) & 1, l = i & 15;
  const uint32_t q = (blk[16 + 32 * h + 16 * k + l] >> (2 * j)) & 3u;
  const uint32_t sb = blk[8 * h + 2 * j + k];
  const float dl = __fmul_rn(HalfBitsToFloat(LoadU16(blk + 80)), static_cast<float>(sb & 0x0Fu));
  const float ml = __fmul_rn(HalfBitsToFloat(LoadU16(blk + 82)), static_cast<float>(sb >> 4));
  return __fsub_rn(__fmul_rn(dl, static_cast<float>(q)), ml);
}

__device__ __forceinline__ float DequantQ3_KExact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 8) * 110;
  const int i = static_cast<int>(e & 255), h = i >> 7, j = (i >> 5) & 3, k = (i >> 4) & 1, l = i & 15;
  const int q = static_cast<int>((blk[32 + 32 * h + 16 * k + l] >> (2 * j)) & 3u);
  const bool hb = (blk[16 * k + l] >> (4 * h + j)) & 1u;
  const int si = 8 * h + 2 * j + k, quarter = si >> 2, r = si & 3;
  const uint32_t lowb = blk[96 + 4 * (quarter & 1) + r];
  const uint32_t sc6 = ((quarter >> 1) ? (lowb >> 4) : (lowb & 0x0Fu)) | (((blk[104 + r] >> (2 * quarter)) & 3u) << 4);
  const float dl = __fmul_rn(HalfBitsToFloat(LoadU16(blk + 108)), static_cast<float>(static_cast<int>(sc6) - 32));
  return __fmul_rn(dl, static_cast<float>(q - (hb ? 0 : 4)));
}

// Q5_K: Q4_K's header and scales; element 64g + 32u + l takes nibble u of
// qs[32g + l] plus 16 * bit (2g + u) of qh[l] (reference src/quant.cc:281-319).
__device__ __forceinline__ float DequantQ5_KExact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 8) * 176;
  const int i = static_cast<int>(e & 255), sb = i >> 5, g = sb >> 1, u = sb & 1, l = i & 31;
  uint32_t sc, mn;
  ScaleMinK4(sb, LoadU32(blk + 4), LoadU32(blk + 8), LoadU32(blk + 12), &sc, &mn);
  const uint32_t qb = blk[48 + 32 * g + l];
  const uint32_t q = (u ? (qb >> 4) : (qb & 0x0Fu)) + (((blk[16 + l] >> (2 * g + u)) & 1u) ? 16u : 0u);
  const float d1 = __fmul_rn(HalfBitsToFloat(LoadU16(blk)), static_cast<float>(sc));
  const float m1 = __fmul_rn(HalfBitsToFloat(LoadU16(blk + 2)), static_cast<float>(mn));
  return __fsub_rn(__fmul_rn(d1, static_cast<float>(q)), m1);
}

// Q8_K: fp32 d, int8 codes (reference src/quant.cc:356-367)
__device__ __forceinline__ float DequantQ8_KExact(const uint8_t* row, int64_t e) {
  const uint8_t* blk = row + (e >> 8) * 292;
  return __fmul_rn(__uint_as_float(LoadU32(blk)), static_cast<float>(static_cast<int8_t>(blk[4 + (e & 255)])));
}

__device__ __forceinline__ float DequantExact(uint32_t type, const uint8_t* row, int64_t e) {
  switch (type) {
    case 8: return DequantQ8_0Exact(row, e);
    case 12: return DequantQ4_KExact(row, e);
    case 14: return DequantQ6_KExact(row, e);
    case 1: return HalfBitsToFloat(LoadU16(row + 2 * e));
    case 30: return __uint_as_float(LoadU16(row + 2 * e) << 16);
    case 2: return DequantQ4_0Exact(row, e);
    case 3: return DequantQ4_1Exact(row, e);
    case 6: return DequantQ5_0Exact(row, e);
    case 7: return DequantQ5_1Exact(row, e);
    case 9: return DequantQ8_1Exact(row, e);
    case 10: return DequantQ2_KExact(row, e);
    case 11: return DequantQ3_KExact(row, e);
    case 13: return DequantQ5_KExact(row, e);
    case 15: return DequantQ8_KExact(row, e);
    default: {
      float v;
      __builtin_memcpy(&v, row + 4 * e, 4);
      return v;
    }
  }
}

// Elements 32u .. 32u + 31 of a row of any type, exactly as above (the
// generic kernels' unit: natural element order).
__device__ __forceinline__ void DequantUnit(uint32_t type, const uint8_t* row, int u, float* w) {
#pragma unroll 4
  for (int i = 0; i < 32; ++i) w[i] = DequantExact(type, row, 32 * static_cast<int64_t>(u) + i);
}

// ---------------------------------------------------------------- fused units

// Unit<T>::Decode(row, u, w) fills w[32]; w[i] multiplies activation element
// Unit<T>::Elem(u, i) of the row. Reads may touch up to 3 bytes past a block
// (aligned dword windows), so weight arenas carry tail padding.
template <uint32_t T>
struct Unit;

template <>
struct Unit<8> {  // Q8_0
  static constexpr int kPerBlock = 1;
  __device__ static __forceinline__ int Elem(int u, int i) { return 32 * u + i; }
  __device__ static __forceinline__ void Decode(const uint8_t* row, int u, float* w) {
    const uint8_t* blk = row + 34 * u;
    const float d = HalfToFloatFast(LoadU16(blk));
    // quant bytes start 2 bytes into the block: 2-byte aligned
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint2 q = Load8Unaligned(blk + 2 + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[8 * c + i] = static_cast<float>(static_cast<int8_t>(Byte(q.x, i))) * d;
        w[8 * c + 4 + i] = static_cast<float>(static_cast<int8_t>(Byte(q.y, i))) * d;
      }
    }
  }
};

template <>
struct Unit<12> {  // Q4_K
  static constexpr int kPerBlock = 8;
  __device__ static __forceinline__ int Elem(int u, int i) {
    const int b = u >> 3, g = (u >> 1) & 3, h = u & 1;
    return 256 * b + 64 * g + 16 * h + (i < 16 ? i : 16 + i);
  }
  __device__ static __forceinline__ void Decode(const uint8_t* row, int u, float* w) {
    const int b = u >> 3, g = (u >> 1) & 3, h = u & 1;
    const uint8_t* blk = row + 144 * b;
    const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
    const uint4 q = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g + 16 * h);
    const float d = HalfToFloatFast(hdr.x & 0xFFFFu);
    const float dmin = HalfToFloatFast(hdr.x >> 16);
    uint32_t sc, mn;
    ScaleMinK4(2 * g, hdr.y, hdr.z, hdr.w, &sc, &mn);
    const float dl = d * static_cast<float>(sc), ml = dmin * static_cast<float>(mn);
    ScaleMinK4(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc, &mn);
    const float dh = d * static_cast<float>(sc), mh = dmin * static_cast<float>(mn);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t byte = Byte(qw[c], i);
        w[4 * c + i] = __builtin_fmaf(dl, static_cast<float>(byte & 0x0Fu), -ml);
        w[16 + 4 * c + i] = __builtin_fmaf(dh, static_cast<float>(byte >> 4), -mh);
      }
    }
  }
};

template <>
struct Unit<14> {  // Q6_K
  static constexpr int kPerBlock = 8;
  __device__ static __forceinline__ int Elem(int u, int i) {
    const int b = u >> 3, half = (u >> 2) & 1, j = u & 3;
    return 256 * b + 128 * half + 8 * j + 32 * (i >> 3) + (i & 7);
  }
  __device__ static __forceinline__ void Decode(const uint8_t* row, int u, float* w) {
    const int b = u >> 3, half = (u >> 2) & 1, j = u & 3;
    const uint8_t* blk = row + 210 * b;
    const uint2 l0 = Load8Unaligned(blk + 64 * half + 8 * j);
    const uint2 l1 = Load8Unaligned(blk + 64 * half + 32 + 8 * j);
    const uint2 hh = Load8Unaligned(blk + 128 + 32 * half + 8 * j);
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192) + 8 * half + (j >> 1);
    const float d = HalfToFloatFast(LoadU16(blk + 208));
    const float s0 = d * static_cast<float>(sc[0]);
    const float s1 = d * static_cast<float>(sc[2]);
    const float s2 = d * static_cast<float>(sc[4]);
    const float s3 = d * static_cast<float>(sc[6]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t a = Byte(i < 4 ? l0.x : l0.y, i & 3);
      const uint32_t c = Byte(i < 4 ? l1.x : l1.y, i & 3);
      const uint32_t h = Byte(i < 4 ? hh.x : hh.y, i & 3);
      w[i] = s0 * static_cast<float>(static_cast<int>((a & 15u) | ((h & 3u) << 4)) - 32);
      w[8 + i] = s1 * static_cast<float>(static_cast<int>((c & 15u) | (((h >> 2) & 3u) << 4)) - 32);
      w[16 + i] = s2 * static_cast<float>(static_cast<int>((a >> 4) | (((h >> 4) & 3u) << 4)) - 32);
      w[24 + i] = s3 * static_cast<float>(static_cast<int>((c >> 4) | (((h >> 6) & 3u) << 4)) - 32);
    }
  }
};

template <>
struct Unit<0> {  // F32
  static constexpr int kPerBlock = 1;
  __device__ static __forceinline__ int Elem(int u, int i) { return 32 * u + i; }
  __device__ static __forceinline__ void Decode(const uint8_t* row, int u, float* w) {
    const float4* p = reinterpret_cast<const float4*>(row + 128 * u);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float4 v = p[c];
      w[4 * c + 0] = v.x;
      w[4 * c + 1] = v.y;
      w[4 * c + 2] = v.z;
      w[4 * c + 3] = v.w;
    }
  }
};

}  // namespace dev
}  // namespace rpg

#endif  // RPG_HIP_QUANT_DEV_H_
