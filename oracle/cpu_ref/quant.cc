// Scalar dequantisation -- restates reference src/quant.cc. Compiled without
// -mfma (oracle/Makefile), like the reference TU, so `d1 * q - m1` rounds twice.

#include <cstdarg>
#include <cstdio>

#include "oracle.h"

namespace orc {

void Fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw std::runtime_error(buf);
}

// Block geometry (reference src/quant.cc:29-45).
int64_t BlockElems(uint32_t type) {
  switch (type) {
    case kF32: case kF16: case kBF16: return 1;
    case kQ4_0: case kQ4_1: case kQ5_0: case kQ5_1: case kQ8_0: case kQ8_1: return 32;
    case kQ2_K: case kQ3_K: case kQ4_K: case kQ5_K: case kQ6_K: case kQ8_K: return 256;
    default: return -1;
  }
}

int64_t BlockBytes(uint32_t type) {
  switch (type) {
    case kF32: return 4;
    case kF16: case kBF16: return 2;
    case kQ4_0: return 18;
    case kQ4_1: return 20;
    case kQ5_0: return 22;
    case kQ5_1: return 24;
    case kQ8_0: return 34;
    case kQ8_1: return 36;
    case kQ2_K: return 84;
    case kQ3_K: return 110;
    case kQ4_K: return 144;
    case kQ5_K: return 176;
    case kQ6_K: return 210;
    case kQ8_K: return 292;
    default: return -1;
  }
}

// reference src/quant.cc:406-414
int64_t RowBytes(uint32_t type, int64_t n) {
  const int64_t be = BlockElems(type);
  ORC_CHECK(be > 0, "unsupported ggml type %u", type);
  ORC_CHECK(n % be == 0, "%lld elements is not a multiple of block %lld", (long long)n, (long long)be);
  return n / be * BlockBytes(type);
}

// reference src/quant.cc:159-167
void ScaleMinK4(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn) {
  if (j < 4) {
    *sc = static_cast<uint8_t>(q[j] & 63);
    *mn = static_cast<uint8_t>(q[j + 4] & 63);
  } else {
    *sc = static_cast<uint8_t>((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *mn = static_cast<uint8_t>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

namespace {

// reference src/quant.cc:132-142: value = float(q) * d
void DeqQ8_0(const uint8_t* src, int64_t n, float* dst) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = src + b * 34;
    const float d = HalfToFloat(Load16(blk));
    for (int j = 0; j < 32; ++j) {
      dst[b * 32 + j] = static_cast<float>(static_cast<int8_t>(blk[2 + j])) * d;
    }
  }
}

// reference src/quant.cc:252-279: per 64-group, d1 = d*sc, m1 = dmin*m,
// y = d1*float(nibble) - m1 (product rounded, then difference rounded).
void DeqQ4_K(const uint8_t* src, int64_t n, float* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = src + b * 144;
    const float d = HalfToFloat(Load16(blk));
    const float dmin = HalfToFloat(Load16(blk + 2));
    const uint8_t* packed = blk + 4;
    const uint8_t* qs = blk + 16;
    float* y = dst + b * 256;
    for (int g = 0; g < 4; ++g) {
      uint8_t sc, mn;
      ScaleMinK4(2 * g, packed, &sc, &mn);
      const float d_lo = d * static_cast<float>(sc);
      const float m_lo = dmin * static_cast<float>(mn);
      ScaleMinK4(2 * g + 1, packed, &sc, &mn);
      const float d_hi = d * static_cast<float>(sc);
      const float m_hi = dmin * static_cast<float>(mn);
      const uint8_t* qg = qs + 32 * g;
      for (int l = 0; l < 32; ++l) y[64 * g + l] = d_lo * static_cast<float>(qg[l] & 0x0F) - m_lo;
      for (int l = 0; l < 32; ++l) y[64 * g + 32 + l] = d_hi * static_cast<float>(qg[l] >> 4) - m_hi;
    }
  }
}

// reference src/quant.cc:321-354: y = (d * float(sc)) * float(q - 32)
void DeqQ6_K(const uint8_t* src, int64_t n, float* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = src + b * 210;
    const float d = HalfToFloat(Load16(blk + 208));
    for (int half = 0; half < 2; ++half) {
      const uint8_t* ql = blk + 64 * half;
      const uint8_t* qh = blk + 128 + 32 * half;
      const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192) + 8 * half;
      float* y = dst + b * 256 + 128 * half;
      for (int l = 0; l < 32; ++l) {
        const int s = l / 16;
        const int v0 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
        const int v1 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int v2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int v3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        y[l] = d * static_cast<float>(sc[s]) * static_cast<float>(v0);
        y[l + 32] = d * static_cast<float>(sc[s + 2]) * static_cast<float>(v1);
        y[l + 64] = d * static_cast<float>(sc[s + 4]) * static_cast<float>(v2);
        y[l + 96] = d * static_cast<float>(sc[s + 6]) * static_cast<float>(v3);
      }
    }
  }
}

// The 32-element blocks, element j of a block: code = nibble (j < 16: low
// nibble of qs[j], else high nibble of qs[j - 16]) plus, for the 5-bit types,
// bit j of the little-endian 32-bit qh as bit 4.
//   Q4_0 float(code - 8) * d        reference src/quant.cc:66-78
//   Q4_1 float(code) * d + m        :80-93
//   Q5_0 float(code - 16) * d       :95-113 (integer difference first)
//   Q5_1 float(code) * d + m        :115-130
//   Q8_1 float(int8 q) * d          :144-155 (the s field unused)
int LegacyCode(const uint8_t* qs, const uint8_t* qh, int j) {
  const int nib = j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4);
  if (qh == nullptr) return nib;
  uint32_t h;
  std::memcpy(&h, qh, 4);
  return nib | static_cast<int>(((h >> j) & 1u) << 4);
}

void DeqLegacy(uint32_t type, const uint8_t* src, int64_t n, float* dst) {
  const int64_t bb = BlockBytes(type);
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = src + b * bb;
    const float d = HalfToFloat(Load16(blk));
    float* y = dst + b * 32;
    switch (type) {
      case kQ4_0:
        for (int j = 0; j < 32; ++j) y[j] = static_cast<float>(LegacyCode(blk + 2, nullptr, j) - 8) * d;
        break;
      case kQ4_1: {
        const float m = HalfToFloat(Load16(blk + 2));
        for (int j = 0; j < 32; ++j) y[j] = static_cast<float>(LegacyCode(blk + 4, nullptr, j)) * d + m;
        break;
      }
      case kQ5_0:
        for (int j = 0; j < 32; ++j) y[j] = static_cast<float>(LegacyCode(blk + 6, blk + 2, j) - 16) * d;
        break;
      case kQ5_1: {
        const float m = HalfToFloat(Load16(blk + 2));
        for (int j = 0; j < 32; ++j) y[j] = static_cast<float>(LegacyCode(blk + 8, blk + 4, j)) * d + m;
        break;
      }
      default:  // Q8_1
        for (int j = 0; j < 32; ++j) y[j] = static_cast<float>(static_cast<int8_t>(blk[4 + j])) * d;
        break;
    }
  }
}

// Q2_K / Q3_K: element e = 128h + 32j + 16k + l of a super-block reads bits
// 2j..2j+1 of qs[32h + 16k + l] and sub-block scale 8h + 2j + k
// (reference src/quant.cc:169-201 and :203-250).
//   Q2_K: scale byte = sc | m << 4; y = (d * float(sc)) * float(q) - dmin * float(m)
//   Q3_K: 6-bit scale s (12 packed bytes, below), high bit 4h + j of
//         hmask[16k + l]; y = (d * float(s - 32)) * float(q - (bit ? 0 : 4))
int Q3Scale(const uint8_t* packed, int i) {
  const int quarter = i >> 2, r = i & 3;
  const uint8_t lowb = packed[4 * (quarter & 1) + r];
  const int low4 = (quarter >> 1) ? (lowb >> 4) : (lowb & 0x0F);
  const int high2 = (packed[8 + r] >> (2 * quarter)) & 3;
  return low4 | (high2 << 4);
}

void DeqQ2Q3(uint32_t type, const uint8_t* src, int64_t n, float* dst) {
  const bool q3 = type == kQ3_K;
  const int64_t bb = q3 ? 110 : 84;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = src + b * bb;
    const uint8_t* qs = blk + (q3 ? 32 : 16);
    float* y = dst + b * 256;
    for (int e = 0; e < 256; ++e) {
      const int h = e >> 7, j = (e >> 5) & 3, k = (e >> 4) & 1, l = e & 15;
      const int q = (qs[32 * h + 16 * k + l] >> (2 * j)) & 3;
      const int si = 8 * h + 2 * j + k;
      if (q3) {
        const float d = HalfToFloat(Load16(blk + 108));
        const bool hb = (blk[16 * k + l] >> (4 * h + j)) & 1;
        const float dl = d * static_cast<float>(Q3Scale(blk + 96, si) - 32);
        y[e] = dl * static_cast<float>(q - (hb ? 0 : 4));
      } else {
        const float d = HalfToFloat(Load16(blk + 80));
        const float dmin = HalfToFloat(Load16(blk + 82));
        const float dl = d * static_cast<float>(blk[si] & 0x0F);
        const float ml = dmin * static_cast<float>(blk[si] >> 4);
        y[e] = dl * static_cast<float>(q) - ml;
      }
    }
  }
}

// reference src/quant.cc:281-319: Q4_K's scales; element 64g + 32u + l takes
// nibble u of qs[32g + l] plus 16 * bit (2g + u) of qh[l];
// y = (d * float(sc)) * float(q) - dmin * float(m).
void DeqQ5_K(const uint8_t* src, int64_t n, float* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = src + b * 176;
    const float d = HalfToFloat(Load16(blk));
    const float dmin = HalfToFloat(Load16(blk + 2));
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    float* y = dst + b * 256;
    for (int sb = 0; sb < 8; ++sb) {
      uint8_t sc, mn;
      ScaleMinK4(sb, blk + 4, &sc, &mn);
      const float d1 = d * static_cast<float>(sc);
      const float m1 = dmin * static_cast<float>(mn);
      const int g = sb >> 1, u = sb & 1;
      for (int l = 0; l < 32; ++l) {
        const int q = (u ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 0x0F)) + (((qh[l] >> (2 * g + u)) & 1) ? 16 : 0);
        y[32 * sb + l] = d1 * static_cast<float>(q) - m1;
      }
    }
  }
}

// reference src/quant.cc:356-367: fp32 d, y = d * float(int8 q)
void DeqQ8_K(const uint8_t* src, int64_t n, float* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = src + b * 292;
    float d;
    std::memcpy(&d, blk, 4);
    for (int j = 0; j < 256; ++j) dst[b * 256 + j] = d * static_cast<float>(static_cast<int8_t>(blk[4 + j]));
  }
}

}  // namespace

// reference src/quant.cc:416-436
void DequantizeRow(uint32_t type, const uint8_t* src, int64_t n, float* dst) {
  switch (type) {
    case kF32: std::memcpy(dst, src, static_cast<size_t>(n) * 4); return;
    case kF16:
      for (int64_t i = 0; i < n; ++i) dst[i] = HalfToFloat(Load16(src + 2 * i));
      return;
    case kBF16:
      for (int64_t i = 0; i < n; ++i) {
        const uint32_t bits = static_cast<uint32_t>(Load16(src + 2 * i)) << 16;
        std::memcpy(dst + i, &bits, 4);
      }
      return;
    case kQ4_0: case kQ4_1: case kQ5_0: case kQ5_1: case kQ8_1: DeqLegacy(type, src, n, dst); return;
    case kQ8_0: DeqQ8_0(src, n, dst); return;
    case kQ2_K: case kQ3_K: DeqQ2Q3(type, src, n, dst); return;
    case kQ4_K: DeqQ4_K(src, n, dst); return;
    case kQ5_K: DeqQ5_K(src, n, dst); return;
    case kQ6_K: DeqQ6_K(src, n, dst); return;
    case kQ8_K: DeqQ8_K(src, n, dst); return;
    default: Fail("unsupported ggml type id=%u", type);
  }
}

}  // namespace orc
