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
    case kQ8_0: return 32;
    case kQ4_K: case kQ6_K: return 256;
    default: return -1;
  }
}

int64_t BlockBytes(uint32_t type) {
  switch (type) {
    case kF32: return 4;
    case kF16: case kBF16: return 2;
    case kQ8_0: return 34;
    case kQ4_K: return 144;
    case kQ6_K: return 210;
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

}  // namespace

// reference src/quant.cc:416-436 (the types this build's models use)
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
    case kQ8_0: DeqQ8_0(src, n, dst); return;
    case kQ4_K: DeqQ4_K(src, n, dst); return;
    case kQ6_K: DeqQ6_K(src, n, dst); return;
    default: Fail("unsupported ggml type id=%u", type);
  }
}

}  // namespace orc
