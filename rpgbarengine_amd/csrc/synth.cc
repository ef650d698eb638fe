// Synthetic qwen3 GGUF writer and block quantizers (see include/rpg_synth.h).
//
// The quantizers are this project's own simple min/max schemes. Their only
// contract is to emit structurally valid blocks in the ggml layouts that the
// reference dequantises (reference src/quant.cc:66-145 Q4_0 .. Q8_1, :159-167
// the 6-bit scale packing of Q4_K / Q5_K, :169-369 the K-quants, dtypes.h
// F16 / BF16): the CPU oracle and the GPU engine then read the same bytes, so
// any valid encoding is a fair input. Codes are rounded to nearest so a dequantised tensor stays close to
// the N(0, std) source (checked by tests/test_synth.py).

#include "rpg_synth.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;

// ------------------------------------------------------------ random source

inline uint64_t Mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

inline uint64_t StreamKey(uint64_t seed, uint64_t stream) {
  return Mix64(seed ^ Mix64(stream + 0x632BE59BD9B4E019ull));
}

// Pair i of the stream -> two N(0,1) samples (Box-Muller in double).
inline void GaussPair(uint64_t key, uint64_t i, double* z0, double* z1) {
  const uint64_t a = Mix64(key + 2 * i);
  const uint64_t b = Mix64(key + 2 * i + 1);
  const double u1 = (static_cast<double>(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
  const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
  const double r = std::sqrt(-2.0 * std::log(u1));
  const double t = 6.283185307179586476925 * u2;
  *z0 = r * std::cos(t);
  *z1 = r * std::sin(t);
}

void Gaussian(uint64_t seed, uint64_t stream, int64_t n, float std_dev, float* out) {
  const uint64_t key = StreamKey(seed, stream);
  for (int64_t i = 0; i < n; i += 2) {
    double z0, z1;
    GaussPair(key, static_cast<uint64_t>(i / 2), &z0, &z1);
    out[i] = static_cast<float>(z0 * std_dev);
    if (i + 1 < n) out[i + 1] = static_cast<float>(z1 * std_dev);
  }
}

uint64_t NameHash(const std::string& s) {
  uint64_t h = 0xCBF29CE484222325ull;  // FNV-1a
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001B3ull;
  }
  return h;
}

// ------------------------------------------------------------ fp16

// float -> IEEE half, round to nearest even (own implementation).
uint16_t ToHalf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t absu = u & 0x7FFFFFFFu;
  if (absu >= 0x7F800000u) return static_cast<uint16_t>(sign | 0x7C00u | (absu > 0x7F800000u ? 0x200u : 0u));
  if (absu >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // rounds to inf
  if (absu < 0x38800000u) {
    // subnormal half (or zero): value = m * 2^-24
    if (absu < 0x33000000u) return static_cast<uint16_t>(sign);  // < 2^-25 -> 0
    const uint32_t e = absu >> 23;
    const uint32_t mant = (absu & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126 - e;  // 14 - (e - 127) + 13 - 1 ... shift of mant to 2^-24 units
    const uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
    return static_cast<uint16_t>(sign | r);
  }
  const uint32_t e = ((absu >> 23) - 112) << 10;
  const uint32_t m = (absu >> 13) & 0x3FFu;
  uint32_t h = e | m;
  const uint32_t rem = absu & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
  return static_cast<uint16_t>(sign | h);
}

float FromHalf(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1F;
  const uint32_t m = h & 0x3FF;
  float v;
  if (e == 0) {
    v = std::ldexp(static_cast<float>(m), -24);
  } else if (e == 31) {
    uint32_t u = 0x7F800000u | (m << 13);
    std::memcpy(&v, &u, 4);
  } else {
    uint32_t u = ((e + 112) << 23) | (m << 13);
    std::memcpy(&v, &u, 4);
  }
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

inline void PutHalf(uint8_t* p, float v) {
  const uint16_t h = ToHalf(v);
  p[0] = static_cast<uint8_t>(h & 0xFF);
  p[1] = static_cast<uint8_t>(h >> 8);
}

inline float GetHalf(const uint8_t* p) {
  return FromHalf(static_cast<uint16_t>(p[0] | (p[1] << 8)));
}

inline int RoundClamp(float v, int lo, int hi) {
  int q = static_cast<int>(std::lround(v));
  return q < lo ? lo : (q > hi ? hi : q);
}

// ------------------------------------------------------------ quantizers

// Q8_0: 32 elements -> fp16 d | int8 q[32]; value = q * d.
void QuantQ8_0(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const float* xb = x + b * 32;
    uint8_t* p = dst + b * 34;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(xb[j]));
    PutHalf(p, amax / 127.0f);
    const float d = GetHalf(p);
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    for (int j = 0; j < 32; ++j) {
      p[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(RoundClamp(xb[j] * id, -127, 127)));
    }
  }
}

// Q4_K: 256 elements = 8 sub-blocks of 32. fp16 d | fp16 dmin | 12 bytes of
// 6-bit (scale, min) pairs | 128 bytes of nibbles. value = d*sc*q - dmin*m.
void QuantQ4_K(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const float* xb = x + b * 256;
    uint8_t* p = dst + b * 144;
    float scale[8], minv[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 8; ++s) {
      float lo = 0.0f, hi = 0.0f;
      for (int j = 0; j < 32; ++j) {
        lo = std::min(lo, xb[32 * s + j]);
        hi = std::max(hi, xb[32 * s + j]);
      }
      scale[s] = (hi - lo) / 15.0f;
      minv[s] = -lo;
      max_scale = std::max(max_scale, scale[s]);
      max_min = std::max(max_min, minv[s]);
    }
    PutHalf(p + 0, max_scale / 63.0f);
    PutHalf(p + 2, max_min / 63.0f);
    const float d = GetHalf(p + 0);
    const float dmin = GetHalf(p + 2);
    int sc[8], mn[8];
    for (int s = 0; s < 8; ++s) {
      sc[s] = d > 0.0f ? RoundClamp(scale[s] / d, 0, 63) : 0;
      mn[s] = dmin > 0.0f ? RoundClamp(minv[s] / dmin, 0, 63) : 0;
    }
    uint8_t* q = p + 4;
    for (int j = 0; j < 4; ++j) {
      q[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      q[j + 4] = static_cast<uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
      q[j + 8] = static_cast<uint8_t>((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
    int code[256];
    for (int s = 0; s < 8; ++s) {
      const float es = d * static_cast<float>(sc[s]);
      const float em = dmin * static_cast<float>(mn[s]);
      for (int j = 0; j < 32; ++j) {
        code[32 * s + j] = es > 0.0f ? RoundClamp((xb[32 * s + j] + em) / es, 0, 15) : 0;
      }
    }
    uint8_t* qs = p + 16;
    for (int g = 0; g < 4; ++g) {
      for (int l = 0; l < 32; ++l) {
        qs[32 * g + l] = static_cast<uint8_t>(code[64 * g + l] | (code[64 * g + 32 + l] << 4));
      }
    }
  }
}

// Q6_K: 256 elements = 16 sub-blocks of 16. ql[128] | qh[64] | int8 sc[16] |
// fp16 d. value = d*sc*(q - 32), q in 0..63.
void QuantQ6_K(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const float* xb = x + b * 256;
    uint8_t* p = dst + b * 210;
    float scale[16];
    float max_scale = 0.0f;
    for (int s = 0; s < 16; ++s) {
      float amax = 0.0f;
      for (int j = 0; j < 16; ++j) amax = std::max(amax, std::fabs(xb[16 * s + j]));
      scale[s] = amax / 31.0f;
      max_scale = std::max(max_scale, scale[s]);
    }
    PutHalf(p + 208, max_scale / 127.0f);
    const float d = GetHalf(p + 208);
    int8_t* scb = reinterpret_cast<int8_t*>(p + 192);
    int u[256];
    for (int s = 0; s < 16; ++s) {
      const int sc = d > 0.0f ? RoundClamp(scale[s] / d, -128, 127) : 0;
      scb[s] = static_cast<int8_t>(sc);
      const float es = d * static_cast<float>(sc);
      for (int j = 0; j < 16; ++j) {
        const int q = es > 0.0f ? RoundClamp(xb[16 * s + j] / es, -32, 31) : 0;
        u[16 * s + j] = q + 32;
      }
    }
    uint8_t* ql = p;
    uint8_t* qh = p + 128;
    for (int h = 0; h < 2; ++h) {
      const int* uh = u + 128 * h;
      uint8_t* qlh = ql + 64 * h;
      uint8_t* qhh = qh + 32 * h;
      for (int l = 0; l < 32; ++l) {
        const int u1 = uh[l], u2 = uh[l + 32], u3 = uh[l + 64], u4 = uh[l + 96];
        qlh[l] = static_cast<uint8_t>((u1 & 15) | ((u3 & 15) << 4));
        qlh[l + 32] = static_cast<uint8_t>((u2 & 15) | ((u4 & 15) << 4));
        qhh[l] = static_cast<uint8_t>((u1 >> 4) | ((u2 >> 4) << 2) | ((u3 >> 4) << 4) | ((u4 >> 4) << 6));
      }
    }
  }
}

// The 32-element legacy blocks: amax or min/max of the block, codes rounded
// to nearest. Q4_0 / Q5_0 value = (q - 8 | 16) * d; Q4_1 / Q5_1 value =
// q * d + m; the fifth bit of element j sits in bit j of the 32-bit qh.
void QuantLegacy(uint32_t type, const float* x, int64_t n, uint8_t* dst) {
  const bool with_min = type == RPG_GGML_Q4_1 || type == RPG_GGML_Q5_1;
  const bool five = type == RPG_GGML_Q5_0 || type == RPG_GGML_Q5_1;
  const int levels = five ? 31 : 15;
  const int64_t bb = (with_min ? 4 : 2) + (five ? 4 : 0) + 16;
  for (int64_t b = 0; b < n / 32; ++b) {
    const float* xb = x + b * 32;
    uint8_t* p = dst + b * bb;
    float lo = xb[0], hi = xb[0], amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
      lo = std::min(lo, xb[j]);
      hi = std::max(hi, xb[j]);
      amax = std::max(amax, std::fabs(xb[j]));
    }
    int code[32];
    if (with_min) {
      PutHalf(p, (hi - lo) / static_cast<float>(levels));
      PutHalf(p + 2, lo);
      const float d = GetHalf(p), m = GetHalf(p + 2);
      for (int j = 0; j < 32; ++j) code[j] = d > 0.0f ? RoundClamp((xb[j] - m) / d, 0, levels) : 0;
    } else {
      const int half = (levels + 1) / 2;  // 8 or 16
      PutHalf(p, amax / static_cast<float>(half - 1));
      const float d = GetHalf(p);
      for (int j = 0; j < 32; ++j) code[j] = d > 0.0f ? RoundClamp(xb[j] / d, -half, half - 1) + half : half;
    }
    uint8_t* qs = p + (with_min ? 4 : 2) + (five ? 4 : 0);
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
      qs[j] = static_cast<uint8_t>((code[j] & 15) | ((code[j + 16] & 15) << 4));
      qh |= static_cast<uint32_t>((code[j] >> 4) & 1) << j;
      qh |= static_cast<uint32_t>((code[j + 16] >> 4) & 1) << (j + 16);
    }
    if (five) std::memcpy(p + (with_min ? 4 : 2), &qh, 4);
  }
}

// Q8_1: fp16 d | fp16 s (d * sum q, unused by the dequantisation) | int8 q[32].
void QuantQ8_1(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const float* xb = x + b * 32;
    uint8_t* p = dst + b * 36;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(xb[j]));
    PutHalf(p, amax / 127.0f);
    const float d = GetHalf(p);
    int sum = 0;
    for (int j = 0; j < 32; ++j) {
      const int q = d > 0.0f ? RoundClamp(xb[j] / d, -127, 127) : 0;
      p[4 + j] = static_cast<uint8_t>(static_cast<int8_t>(q));
      sum += q;
    }
    PutHalf(p + 2, d * static_cast<float>(sum));
  }
}

// Q2_K: 256 elements = 16 sub-blocks of 16. scales[16] (scale low nibble, min
// high nibble) | qs[64] (2-bit codes, four per byte) | fp16 d | fp16 dmin.
// value = d*sc*q - dmin*m; element 128h + 32j + 16k + l takes bits 2j of
// qs[32h + 16k + l] and scale byte 8h + 2j + k.
void QuantQ2_K(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const float* xb = x + b * 256;
    uint8_t* p = dst + b * 84;
    float scale[16], minv[16], max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 16; ++s) {
      float lo = 0.0f, hi = 0.0f;
      for (int j = 0; j < 16; ++j) {
        lo = std::min(lo, xb[16 * s + j]);
        hi = std::max(hi, xb[16 * s + j]);
      }
      scale[s] = (hi - lo) / 3.0f;
      minv[s] = -lo;
      max_scale = std::max(max_scale, scale[s]);
      max_min = std::max(max_min, minv[s]);
    }
    PutHalf(p + 80, max_scale / 15.0f);
    PutHalf(p + 82, max_min / 15.0f);
    const float d = GetHalf(p + 80), dmin = GetHalf(p + 82);
    int code[256];
    for (int s = 0; s < 16; ++s) {
      const int sc = d > 0.0f ? RoundClamp(scale[s] / d, 0, 15) : 0;
      const int mn = dmin > 0.0f ? RoundClamp(minv[s] / dmin, 0, 15) : 0;
      p[s] = static_cast<uint8_t>(sc | (mn << 4));
      const float es = d * static_cast<float>(sc), em = dmin * static_cast<float>(mn);
      for (int j = 0; j < 16; ++j) code[16 * s + j] = es > 0.0f ? RoundClamp((xb[16 * s + j] + em) / es, 0, 3) : 0;
    }
    uint8_t* qs = p + 16;
    for (int h = 0; h < 2; ++h)
      for (int k = 0; k < 2; ++k)
        for (int l = 0; l < 16; ++l) {
          uint8_t v = 0;
          for (int j = 0; j < 4; ++j) v |= static_cast<uint8_t>(code[128 * h + 32 * j + 16 * k + l] << (2 * j));
          qs[32 * h + 16 * k + l] = v;
        }
  }
}

// Q3_K: 256 elements = 16 sub-blocks of 16. hmask[32] | qs[64] | 12 bytes of
// 6-bit scales (stored + 32) | fp16 d. value = d*(sc - 32)*(q - 4*!hbit),
// q2 the 2-bit code; element 128h + 32j + 16k + l takes bits 2j of
// qs[32h + 16k + l], bit 4h + j of hmask[16k + l], scale 8h + 2j + k.
void QuantQ3_K(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const float* xb = x + b * 256;
    uint8_t* p = dst + b * 110;
    float scale[16], max_scale = 0.0f;
    for (int s = 0; s < 16; ++s) {
      float amax = 0.0f;
      for (int j = 0; j < 16; ++j) amax = std::max(amax, std::fabs(xb[16 * s + j]));
      scale[s] = amax / 4.0f;
      max_scale = std::max(max_scale, scale[s]);
    }
    PutHalf(p + 108, max_scale / 31.0f);
    const float d = GetHalf(p + 108);
    int sc6[16], code[256];
    for (int s = 0; s < 16; ++s) {
      const int sc = d > 0.0f ? RoundClamp(scale[s] / d, 0, 31) : 0;
      sc6[s] = sc + 32;
      const float es = d * static_cast<float>(sc);
      for (int j = 0; j < 16; ++j) code[16 * s + j] = es > 0.0f ? RoundClamp(xb[16 * s + j] / es, -4, 3) : 0;
    }
    // the inverse of the kmask unpack (reference src/quant.cc:231-238)
    uint8_t* sp = p + 96;
    for (int j = 0; j < 4; ++j) {
      sp[j] = static_cast<uint8_t>((sc6[j] & 15) | ((sc6[8 + j] & 15) << 4));
      sp[4 + j] = static_cast<uint8_t>((sc6[4 + j] & 15) | ((sc6[12 + j] & 15) << 4));
      sp[8 + j] = static_cast<uint8_t>((sc6[j] >> 4) | ((sc6[4 + j] >> 4) << 2) | ((sc6[8 + j] >> 4) << 4) |
                                       ((sc6[12 + j] >> 4) << 6));
    }
    uint8_t* hm = p;
    uint8_t* qs = p + 32;
    std::memset(hm, 0, 32);
    for (int h = 0; h < 2; ++h)
      for (int k = 0; k < 2; ++k)
        for (int l = 0; l < 16; ++l) {
          uint8_t v = 0;
          for (int j = 0; j < 4; ++j) {
            const int q = code[128 * h + 32 * j + 16 * k + l];  // -4 .. 3
            const bool high = q >= 0;
            v |= static_cast<uint8_t>((high ? q : q + 4) << (2 * j));
            if (high) hm[16 * k + l] |= static_cast<uint8_t>(1u << (4 * h + j));
          }
          qs[32 * h + 16 * k + l] = v;
        }
  }
}

// Q5_K: Q4_K's header and 6-bit (scale, min) packing, qh[32] | qs[128];
// element 64i + 32u + l: nibble u of qs[32i + l], bit 2i + u of qh[l].
void QuantQ5_K(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const float* xb = x + b * 256;
    uint8_t* p = dst + b * 176;
    float scale[8], minv[8], max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 8; ++s) {
      float lo = 0.0f, hi = 0.0f;
      for (int j = 0; j < 32; ++j) {
        lo = std::min(lo, xb[32 * s + j]);
        hi = std::max(hi, xb[32 * s + j]);
      }
      scale[s] = (hi - lo) / 31.0f;
      minv[s] = -lo;
      max_scale = std::max(max_scale, scale[s]);
      max_min = std::max(max_min, minv[s]);
    }
    PutHalf(p + 0, max_scale / 63.0f);
    PutHalf(p + 2, max_min / 63.0f);
    const float d = GetHalf(p + 0), dmin = GetHalf(p + 2);
    int sc[8], mn[8];
    for (int s = 0; s < 8; ++s) {
      sc[s] = d > 0.0f ? RoundClamp(scale[s] / d, 0, 63) : 0;
      mn[s] = dmin > 0.0f ? RoundClamp(minv[s] / dmin, 0, 63) : 0;
    }
    uint8_t* q = p + 4;
    for (int j = 0; j < 4; ++j) {
      q[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      q[j + 4] = static_cast<uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
      q[j + 8] = static_cast<uint8_t>((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
    int code[256];
    for (int s = 0; s < 8; ++s) {
      const float es = d * static_cast<float>(sc[s]), em = dmin * static_cast<float>(mn[s]);
      for (int j = 0; j < 32; ++j) code[32 * s + j] = es > 0.0f ? RoundClamp((xb[32 * s + j] + em) / es, 0, 31) : 0;
    }
    uint8_t* qh = p + 16;
    uint8_t* qs = p + 48;
    std::memset(qh, 0, 32);
    for (int i = 0; i < 4; ++i)
      for (int l = 0; l < 32; ++l) {
        const int c0 = code[64 * i + l], c1 = code[64 * i + 32 + l];
        qs[32 * i + l] = static_cast<uint8_t>((c0 & 15) | ((c1 & 15) << 4));
        qh[l] |= static_cast<uint8_t>(((c0 >> 4) << (2 * i)) | ((c1 >> 4) << (2 * i + 1)));
      }
  }
}

// Q8_K: fp32 d | int8 q[256] | int16 sums of each 16 codes.
void QuantQ8_K(const float* x, int64_t n, uint8_t* dst) {
  for (int64_t b = 0; b < n / 256; ++b) {
    const float* xb = x + b * 256;
    uint8_t* p = dst + b * 292;
    float amax = 0.0f;
    for (int j = 0; j < 256; ++j) amax = std::max(amax, std::fabs(xb[j]));
    const float d = amax / 127.0f;
    std::memcpy(p, &d, 4);
    for (int g = 0; g < 16; ++g) {
      int16_t sum = 0;
      for (int j = 0; j < 16; ++j) {
        const int q = d > 0.0f ? RoundClamp(xb[16 * g + j] / d, -127, 127) : 0;
        p[4 + 16 * g + j] = static_cast<uint8_t>(static_cast<int8_t>(q));
        sum = static_cast<int16_t>(sum + q);
      }
      std::memcpy(p + 260 + 2 * g, &sum, 2);
    }
  }
}

// bf16 with round-to-nearest-even (NaN kept quiet)
inline uint16_t ToBf16(float v) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

int64_t BlockElems(uint32_t type) {
  switch (type) {
    case RPG_GGML_F32: case RPG_GGML_F16: case RPG_GGML_BF16: return 1;
    case RPG_GGML_Q4_0: case RPG_GGML_Q4_1: case RPG_GGML_Q5_0: case RPG_GGML_Q5_1:
    case RPG_GGML_Q8_0: case RPG_GGML_Q8_1: return 32;
    case RPG_GGML_Q2_K: case RPG_GGML_Q3_K: case RPG_GGML_Q4_K: case RPG_GGML_Q5_K:
    case RPG_GGML_Q6_K: case RPG_GGML_Q8_K: return 256;
    default: return -1;
  }
}

int64_t BlockBytes(uint32_t type) {
  switch (type) {
    case RPG_GGML_F32: return 4;
    case RPG_GGML_F16: case RPG_GGML_BF16: return 2;
    case RPG_GGML_Q4_0: return 18;
    case RPG_GGML_Q4_1: return 20;
    case RPG_GGML_Q5_0: return 22;
    case RPG_GGML_Q5_1: return 24;
    case RPG_GGML_Q8_0: return 34;
    case RPG_GGML_Q8_1: return 36;
    case RPG_GGML_Q2_K: return 84;
    case RPG_GGML_Q3_K: return 110;
    case RPG_GGML_Q4_K: return 144;
    case RPG_GGML_Q5_K: return 176;
    case RPG_GGML_Q6_K: return 210;
    case RPG_GGML_Q8_K: return 292;
    default: return -1;
  }
}

int64_t RowBytes(uint32_t type, int64_t n) {
  const int64_t be = BlockElems(type);
  if (be <= 0 || n % be != 0) return -1;
  return n / be * BlockBytes(type);
}

int64_t Quantize(uint32_t type, const float* src, int64_t n, uint8_t* dst) {
  const int64_t rb = RowBytes(type, n);
  if (rb < 0) return -1;
  switch (type) {
    case RPG_GGML_F32: std::memcpy(dst, src, static_cast<size_t>(n) * 4); break;
    case RPG_GGML_F16:
      for (int64_t i = 0; i < n; ++i) PutHalf(dst + 2 * i, src[i]);
      break;
    case RPG_GGML_BF16:
      for (int64_t i = 0; i < n; ++i) {
        const uint16_t h = ToBf16(src[i]);
        dst[2 * i] = static_cast<uint8_t>(h & 0xFF);
        dst[2 * i + 1] = static_cast<uint8_t>(h >> 8);
      }
      break;
    case RPG_GGML_Q4_0: case RPG_GGML_Q4_1: case RPG_GGML_Q5_0: case RPG_GGML_Q5_1:
      QuantLegacy(type, src, n, dst);
      break;
    case RPG_GGML_Q8_0: QuantQ8_0(src, n, dst); break;
    case RPG_GGML_Q8_1: QuantQ8_1(src, n, dst); break;
    case RPG_GGML_Q2_K: QuantQ2_K(src, n, dst); break;
    case RPG_GGML_Q3_K: QuantQ3_K(src, n, dst); break;
    case RPG_GGML_Q4_K: QuantQ4_K(src, n, dst); break;
    case RPG_GGML_Q5_K: QuantQ5_K(src, n, dst); break;
    case RPG_GGML_Q6_K: QuantQ6_K(src, n, dst); break;
    case RPG_GGML_Q8_K: QuantQ8_K(src, n, dst); break;
    default: return -1;
  }
  return rb;
}

// ------------------------------------------------------------ BBPE vocabulary

// GPT-2's byte characters: printable Latin-1 bytes stand for themselves, the
// other 68 take U+0100.. in byte order.
std::string ByteChar(uint8_t b) {
  const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || b >= 0xAE;
  uint32_t cp = b;
  if (!printable) cp = b <= 0x20 ? 0x100u + b : (b < 0xAD ? 0x121u + (b - 0x7F) : 0x143u);
  std::string s;
  if (cp < 0x80) {
    s.push_back(static_cast<char>(cp));
  } else {
    s.push_back(static_cast<char>(0xC0 | (cp >> 6)));
    s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
  }
  return s;
}

// Training text of the synthetic merges: a little of everything a chat
// engine sees (prose with contractions, ChatML, tool calls, CJK, Hangul,
// Greek, Cyrillic, code, numbers).
const char kCorpus[] = R"CORPUS(The innkeeper of the Drunken Cat wipes the counter and glances at the door. "You're late," she says. "The caravan left at dawn, and they'll not wait for anyone." The ranger shrugs: "I've walked these roads for 12 years; I'd rather be late than dead." Rain drums on the roof. Three travellers argue about the price of 40 silver coins, and a bard tunes a lute in the corner. "Don't touch that map," says the old man. "It's the only one that shows the ruins north of the river." The party checks the scene, rolls for perception (DC 15), and moves toward the temple hall where torchlight flickers on the walls.
<|im_start|>system
You are the game master of a tabletop role-playing game. Call the tools when the players ask to look around, roll a check or move.<|im_end|>
<|im_start|>user
I raise my torch and look around the temple hall.<|im_end|>
<|im_start|>assistant
<think>
The player wants to inspect the scene, so I should call read_scene.
</think>

<tool_call>
{"name": "read_scene", "arguments": {"scene": "temple_hall"}}
</tool_call><|im_end|>
{"type": "function", "function": {"name": "roll_check", "description": "Roll a skill check", "parameters": {"type": "object", "properties": {"skill": {"type": "string"}, "dc": {"type": "integer"}}, "required": ["skill", "dc"]}}}
玩家的角色是一名叫李明的游侠。他正在醉猫酒馆里向老板打听北方废墟的传言。老板压低声音说：那座神庙已经荒废了三百年，进去的人很少有回来的。你是一位文字跑团的主持人（DM）。当玩家要求你查看场景、检定或移动时，必须调用相应工具，不要凭记忆作答。我举起火把，仔细查看神庙大厅里有什么。
旅人は酒場の扉を開けた。「北の遺跡について何か知っているか？」と彼女は尋ねた。
여행자는 주점의 문을 열었다. 북쪽 폐허에 대해 아는 것이 있습니까?
Ο ταξιδιώτης άνοιξε την πόρτα της ταβέρνας. Путешественник открыл дверь таверны и спросил о руинах на севере.
def roll(dice, sides=20):
    return sum(random.randint(1, sides) for _ in range(dice))  # 3d6 -> 3..18
for (int i = 0; i < n; ++i) { total += weights[i] * values[i]; }
Numbers: 0 1 2 3 4 5 6 7 8 9 10 100 1000 3.14 2026-12-02 42% ① ② Ⅻ ４２
)CORPUS";

// Qwen's 26 added tokens; type 3 = control, 4 = user-defined
const std::pair<const char*, int32_t> kAddedTokens[] = {
    {"<|endoftext|>", 3}, {"<|im_start|>", 3}, {"<|im_end|>", 3}, {"<|object_ref_start|>", 3},
    {"<|object_ref_end|>", 3}, {"<|box_start|>", 3}, {"<|box_end|>", 3}, {"<|quad_start|>", 3},
    {"<|quad_end|>", 3}, {"<|vision_start|>", 3}, {"<|vision_end|>", 3}, {"<|vision_pad|>", 3},
    {"<|image_pad|>", 3}, {"<|video_pad|>", 3}, {"<tool_call>", 4}, {"</tool_call>", 4},
    {"<|fim_prefix|>", 3}, {"<|fim_middle|>", 3}, {"<|fim_suffix|>", 3}, {"<|fim_pad|>", 3},
    {"<|repo_name|>", 3}, {"<|file_sep|>", 3}, {"<tool_response>", 4}, {"</tool_response>", 4},
    {"<think>", 4}, {"</think>", 4},
};

struct BbpeVocab {
  std::vector<std::string> tokens, merges;
  std::vector<int32_t> types;
  int32_t bos = -1, eos = -1;
};

// Greedy byte-pair training: words are the corpus split before each space
// and around line breaks; each round merges the most frequent adjacent pair
// (the smallest pair of strings among equals) while any pair is left and the
// vocabulary has room.
BbpeVocab BuildBbpe(int32_t vocab) {
  const int32_t n_added = static_cast<int32_t>(sizeof(kAddedTokens) / sizeof(kAddedTokens[0]));
  if (vocab < 256 + n_added) throw std::runtime_error("a BPE vocabulary needs at least 282 entries");
  BbpeVocab v;
  std::map<std::string, int32_t> known;
  for (int b = 0; b < 256; ++b) {
    v.tokens.push_back(ByteChar(static_cast<uint8_t>(b)));
    v.types.push_back(1);
    known.emplace(v.tokens.back(), b);
  }
  std::map<std::string, int64_t> word_count;
  {
    const std::string text = kCorpus;
    size_t i = 0;
    while (i < text.size()) {
      size_t j = i + 1;
      if (text[i] != '\n')
        while (j < text.size() && text[j] != ' ' && text[j] != '\n') ++j;
      ++word_count[text.substr(i, j - i)];
      i = j;
    }
  }
  std::vector<std::pair<std::vector<std::string>, int64_t>> words;
  for (const auto& wc : word_count) {
    std::vector<std::string> sym;
    for (unsigned char b : wc.first) sym.push_back(ByteChar(b));
    words.emplace_back(std::move(sym), wc.second);
  }
  const int32_t budget = vocab - n_added;
  while (static_cast<int32_t>(v.tokens.size()) < budget) {
    std::map<std::pair<std::string, std::string>, int64_t> pairs;
    for (const auto& w : words)
      for (size_t k = 0; k + 1 < w.first.size(); ++k) pairs[{w.first[k], w.first[k + 1]}] += w.second;
    const std::pair<std::string, std::string>* best = nullptr;
    int64_t best_n = 0;
    for (const auto& p : pairs)
      if (p.second > best_n) best_n = p.second, best = &p.first;  // ordered map: the smallest pair among equals
    if (best == nullptr) break;
    const std::string left = best->first, right = best->second, joined = left + right;
    v.merges.push_back(left + " " + right);
    if (!known.count(joined)) {
      known.emplace(joined, static_cast<int32_t>(v.tokens.size()));
      v.tokens.push_back(joined);
      v.types.push_back(1);
    }
    for (auto& w : words) {
      std::vector<std::string> out;
      for (size_t k = 0; k < w.first.size(); ++k) {
        if (k + 1 < w.first.size() && w.first[k] == left && w.first[k + 1] == right) {
          out.push_back(joined);
          ++k;
        } else {
          out.push_back(w.first[k]);
        }
      }
      w.first.swap(out);
    }
  }
  for (const auto& a : kAddedTokens) {
    if (std::string(a.first) == "<|endoftext|>") v.bos = static_cast<int32_t>(v.tokens.size());
    if (std::string(a.first) == "<|im_end|>") v.eos = static_cast<int32_t>(v.tokens.size());
    v.tokens.push_back(a.first);
    v.types.push_back(a.second);
  }
  while (static_cast<int32_t>(v.tokens.size()) < vocab) {
    v.tokens.push_back("[PAD" + std::to_string(v.tokens.size()) + "]");
    v.types.push_back(5);
  }
  return v;
}

// ------------------------------------------------------------ GGUF writer

enum : uint32_t {
  kMetaU32 = 4, kMetaI32 = 5, kMetaF32 = 6, kMetaBool = 7, kMetaString = 8,
  kMetaArray = 9, kMetaU64 = 10,
};

struct Buf {
  std::vector<uint8_t> b;
  void Raw(const void* p, size_t n) {
    const uint8_t* c = static_cast<const uint8_t*>(p);
    b.insert(b.end(), c, c + n);
  }
  void U32(uint32_t v) { Raw(&v, 4); }
  void U64(uint64_t v) { Raw(&v, 8); }
  void F32(float v) { Raw(&v, 4); }
  void Str(const std::string& s) {
    U64(s.size());
    Raw(s.data(), s.size());
  }
};

struct TensorPlan {
  std::string name;
  std::vector<int64_t> dims;  // dims[0] fastest (cols)
  uint32_t type;
  bool is_norm;               // 1 + N(0, norm_std) instead of N(0, weight_std)
  uint64_t offset = 0;
  uint64_t bytes = 0;
};

uint32_t MatrixType(int mix, const std::string& name, int layer) {
  switch (mix) {
    case RPG_MIX_Q8_0: return RPG_GGML_Q8_0;
    case RPG_MIX_F32: return RPG_GGML_F32;
    case RPG_MIX_Q4_K: return RPG_GGML_Q4_K;
    case RPG_MIX_Q6_K: return RPG_GGML_Q6_K;
    case RPG_MIX_Q4_K_M:
      if (name == "token_embd.weight") return RPG_GGML_Q6_K;
      if (name.find("attn_v.weight") != std::string::npos) return RPG_GGML_Q6_K;
      if (name.find("ffn_down.weight") != std::string::npos && layer % 2 == 0) return RPG_GGML_Q6_K;
      return RPG_GGML_Q4_K;
    case RPG_MIX_OTHER: {
      static const uint32_t kCycle[11] = {RPG_GGML_Q4_0, RPG_GGML_Q4_1, RPG_GGML_Q5_0, RPG_GGML_Q5_1,
                                          RPG_GGML_Q8_1, RPG_GGML_Q2_K, RPG_GGML_Q3_K, RPG_GGML_Q5_K,
                                          RPG_GGML_Q8_K, RPG_GGML_F16,  RPG_GGML_BF16};
      static const char* kMats[7] = {"attn_q.", "attn_k.", "attn_v.", "attn_output.", "ffn_gate.", "ffn_up.",
                                     "ffn_down."};
      if (name == "token_embd.weight") return RPG_GGML_Q5_K;
      int m = 0;
      while (m < 7 && name.find(kMats[m]) == std::string::npos) ++m;
      return kCycle[(7 * layer + m) % 11];
    }
    default: throw std::runtime_error("unknown mix");
  }
}

// Norm gains stay F32 except in the mix that exercises the other types.
uint32_t NormType(int mix, const std::string& name) {
  if (mix != RPG_MIX_OTHER) return RPG_GGML_F32;
  if (name.find("attn_norm.") != std::string::npos) return RPG_GGML_F16;
  if (name.find("ffn_norm.") != std::string::npos) return RPG_GGML_BF16;
  return RPG_GGML_F32;
}

const char* MixName(int mix) {
  switch (mix) {
    case RPG_MIX_Q8_0: return "Q8_0";
    case RPG_MIX_Q4_K_M: return "Q4_K_M";
    case RPG_MIX_F32: return "F32";
    case RPG_MIX_Q4_K: return "Q4_K";
    case RPG_MIX_Q6_K: return "Q6_K";
    case RPG_MIX_OTHER: return "OTHER";
    default: return "?";
  }
}

void ParallelFor(int64_t n, int threads, const std::function<void(int64_t)>& body);

void WriteGguf(const char* path, const rpg_synth_spec& s, int n_threads) {
  if (s.n_layers <= 0 || s.hidden <= 0 || s.n_heads <= 0 || s.n_kv_heads <= 0 ||
      s.head_dim <= 0 || s.ffn <= 0 || s.vocab <= 0)
    throw std::runtime_error("spec has a non-positive shape field");
  if (s.n_heads % s.n_kv_heads != 0) throw std::runtime_error("n_heads % n_kv_heads != 0");
  const int64_t qd = static_cast<int64_t>(s.n_heads) * s.head_dim;
  const int64_t kvd = static_cast<int64_t>(s.n_kv_heads) * s.head_dim;

  std::vector<TensorPlan> plan;
  auto mat = [&](const std::string& name, int layer, int64_t rows, int64_t cols) {
    TensorPlan t;
    t.name = name;
    t.dims = {cols, rows};
    t.type = MatrixType(s.mix, name, layer);
    t.is_norm = false;
    if (RowBytes(t.type, cols) < 0)
      throw std::runtime_error("tensor " + name + ": cols not a multiple of the block size");
    plan.push_back(t);
  };
  auto norm = [&](const std::string& name, int64_t n) {
    TensorPlan t;
    t.name = name;
    t.dims = {n};
    t.type = NormType(s.mix, name);
    t.is_norm = true;
    plan.push_back(t);
  };
  mat("token_embd.weight", -1, s.vocab, s.hidden);
  norm("output_norm.weight", s.hidden);
  for (int l = 0; l < s.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    norm(p + "attn_norm.weight", s.hidden);
    norm(p + "ffn_norm.weight", s.hidden);
    norm(p + "attn_q_norm.weight", s.head_dim);
    norm(p + "attn_k_norm.weight", s.head_dim);
    mat(p + "attn_q.weight", l, qd, s.hidden);
    mat(p + "attn_k.weight", l, kvd, s.hidden);
    mat(p + "attn_v.weight", l, kvd, s.hidden);
    mat(p + "attn_output.weight", l, s.hidden, qd);
    mat(p + "ffn_gate.weight", l, s.ffn, s.hidden);
    mat(p + "ffn_up.weight", l, s.ffn, s.hidden);
    mat(p + "ffn_down.weight", l, s.hidden, s.ffn);
  }

  const uint64_t align = 32;
  uint64_t off = 0;
  for (TensorPlan& t : plan) {
    int64_t elems = 1;
    for (int64_t d : t.dims) elems *= d;
    t.bytes = static_cast<uint64_t>(RowBytes(t.type, elems));
    t.offset = off;
    off += t.bytes;
    off = (off + align - 1) / align * align;
  }
  const uint64_t data_bytes = off;

  // ---- header + metadata + tensor infos
  Buf h;
  h.U32(0x46554747u);  // "GGUF"
  h.U32(3);
  h.U64(plan.size());
  const uint64_t n_kv_pos = h.b.size();
  h.U64(0);  // patched below
  uint64_t n_kv = 0;
  auto key = [&](const std::string& k, uint32_t type) {
    h.Str(k);
    h.U32(type);
    ++n_kv;
  };
  key("general.architecture", kMetaString); h.Str("qwen3");
  key("general.name", kMetaString);
  h.Str(std::string("synthetic-qwen3-") + MixName(s.mix));
  key("general.alignment", kMetaU32); h.U32(static_cast<uint32_t>(align));
  key("qwen3.block_count", kMetaU32); h.U32(static_cast<uint32_t>(s.n_layers));
  key("qwen3.embedding_length", kMetaU32); h.U32(static_cast<uint32_t>(s.hidden));
  key("qwen3.feed_forward_length", kMetaU32); h.U32(static_cast<uint32_t>(s.ffn));
  key("qwen3.attention.head_count", kMetaU32); h.U32(static_cast<uint32_t>(s.n_heads));
  key("qwen3.attention.head_count_kv", kMetaU32); h.U32(static_cast<uint32_t>(s.n_kv_heads));
  key("qwen3.attention.key_length", kMetaU32); h.U32(static_cast<uint32_t>(s.head_dim));
  key("qwen3.attention.value_length", kMetaU32); h.U32(static_cast<uint32_t>(s.head_dim));
  key("qwen3.context_length", kMetaU32); h.U32(static_cast<uint32_t>(s.context_length));
  key("qwen3.rope.freq_base", kMetaF32); h.F32(s.rope_theta);
  key("qwen3.attention.layer_norm_rms_epsilon", kMetaF32); h.F32(s.rms_eps);
  key("tokenizer.ggml.model", kMetaString); h.Str("gpt2");
  if (s.tokenizer == 1) {
    const BbpeVocab v = BuildBbpe(s.vocab);
    key("tokenizer.ggml.pre", kMetaString); h.Str("qwen2");
    key("tokenizer.ggml.tokens", kMetaArray);
    h.U32(kMetaString);
    h.U64(v.tokens.size());
    for (const std::string& t : v.tokens) h.Str(t);
    key("tokenizer.ggml.token_type", kMetaArray);
    h.U32(kMetaI32);
    h.U64(v.types.size());
    for (int32_t t : v.types) h.Raw(&t, 4);
    key("tokenizer.ggml.merges", kMetaArray);
    h.U32(kMetaString);
    h.U64(v.merges.size());
    for (const std::string& m : v.merges) h.Str(m);
    key("tokenizer.ggml.bos_token_id", kMetaU32); h.U32(static_cast<uint32_t>(v.bos));
    key("tokenizer.ggml.eos_token_id", kMetaU32); h.U32(static_cast<uint32_t>(v.eos));
    key("tokenizer.ggml.padding_token_id", kMetaU32); h.U32(static_cast<uint32_t>(v.bos));
    key("tokenizer.ggml.add_bos_token", kMetaBool); h.b.push_back(0);
  } else {
    key("tokenizer.ggml.tokens", kMetaArray);
    h.U32(kMetaString);
    h.U64(static_cast<uint64_t>(s.vocab));
    for (int32_t i = 0; i < s.vocab; ++i) h.Str("<t" + std::to_string(i) + ">");
    key("tokenizer.ggml.merges", kMetaArray);
    h.U32(kMetaString);
    h.U64(1);
    h.Str("a b");
    key("tokenizer.ggml.eos_token_id", kMetaU32); h.U32(static_cast<uint32_t>(s.vocab - 1));
  }
  key("rpg.synth.seed", kMetaU64); h.U64(s.seed);
  key("rpg.synth.mix", kMetaString); h.Str(MixName(s.mix));
  std::memcpy(h.b.data() + n_kv_pos, &n_kv, 8);
  for (const TensorPlan& t : plan) {
    h.Str(t.name);
    h.U32(static_cast<uint32_t>(t.dims.size()));
    for (int64_t d : t.dims) h.U64(static_cast<uint64_t>(d));
    h.U32(t.type);
    h.U64(t.offset);
  }
  while (h.b.size() % align) h.b.push_back(0);

  std::FILE* f = std::fopen(path, "wb");
  if (!f) throw std::runtime_error(std::string("cannot open ") + path + " for writing");
  struct Closer {
    std::FILE* f;
    ~Closer() { if (f) std::fclose(f); }
  } closer{f};
  if (std::fwrite(h.b.data(), 1, h.b.size(), f) != h.b.size())
    throw std::runtime_error("short write (header)");

  // ---- tensor data, one tensor at a time, rows in parallel
  std::vector<uint8_t> tbuf;
  for (const TensorPlan& t : plan) {
    tbuf.assign(t.bytes, 0);
    const int64_t cols = t.dims[0];
    const int64_t rows = t.dims.size() >= 2 ? t.dims[1] : 1;
    const int64_t rb = RowBytes(t.type, cols);
    const uint64_t tkey = NameHash(t.name);
    const float sd = t.is_norm ? s.norm_std : s.weight_std;
    ParallelFor(rows, n_threads, [&](int64_t r) {
      std::vector<float> row(static_cast<size_t>(cols));
      Gaussian(s.seed, tkey + static_cast<uint64_t>(r) * 0x9E3779B97F4A7C15ull, cols, sd, row.data());
      if (t.is_norm)
        for (float& v : row) v += 1.0f;
      Quantize(t.type, row.data(), cols, tbuf.data() + r * rb);
    });
    if (std::fwrite(tbuf.data(), 1, tbuf.size(), f) != tbuf.size())
      throw std::runtime_error("short write (tensor " + t.name + ")");
    const uint64_t pad = (t.bytes + align - 1) / align * align - t.bytes;
    static const uint8_t zeros[64] = {0};
    if (pad && std::fwrite(zeros, 1, pad, f) != pad) throw std::runtime_error("short write (pad)");
  }
  (void)data_bytes;
  if (std::fflush(f) != 0) throw std::runtime_error("flush failed");
}

void ParallelFor(int64_t n, int threads, const std::function<void(int64_t)>& body) {
  if (threads <= 0) {
    const unsigned hw = std::thread::hardware_concurrency();
    threads = hw ? static_cast<int>(std::min(hw, 64u)) : 1;
  }
  if (threads == 1 || n < 64) {
    for (int64_t i = 0; i < n; ++i) body(i);
    return;
  }
  std::atomic<int64_t> next{0};
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t) {
    pool.emplace_back([&]() {
      for (;;) {
        const int64_t i0 = next.fetch_add(64);
        if (i0 >= n) return;
        const int64_t i1 = std::min(n, i0 + 64);
        for (int64_t i = i0; i < i1; ++i) body(i);
      }
    });
  }
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

void rpg_synth_default_spec(rpg_synth_spec* spec) {
  std::memset(spec, 0, sizeof(*spec));
  spec->context_length = 4096;
  spec->rope_theta = 1e6f;
  spec->rms_eps = 1e-6f;
  spec->mix = RPG_MIX_Q8_0;
  spec->seed = 1;
  spec->weight_std = 0.02f;
  spec->norm_std = 0.01f;
}

int32_t rpg_synth_write_gguf(const char* path, const rpg_synth_spec* spec, int32_t n_threads) {
  try {
    if (!path || !spec) throw std::runtime_error("null argument");
    WriteGguf(path, *spec, n_threads);
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

int64_t rpg_synth_quantize(uint32_t type, const float* src, int64_t n, uint8_t* dst) {
  const int64_t r = Quantize(type, src, n, dst);
  if (r < 0) g_err = "unsupported type or length not a block multiple";
  return r;
}

int64_t rpg_synth_row_bytes(uint32_t type, int64_t n) { return RowBytes(type, n); }

void rpg_synth_gaussian(uint64_t seed, uint64_t stream, int64_t n, float std_dev, float* out) {
  Gaussian(seed, stream, n, std_dev, out);
}

void rpg_synth_token_ids(uint64_t seed, int64_t n, int32_t vocab, int32_t* out) {
  const uint64_t key = StreamKey(seed, 0x746F6B656E73ull);  // "tokens"
  for (int64_t i = 0; i < n; ++i) {
    // 64-bit multiply-high: uniform in [0, vocab) without modulo bias worth noting
    const unsigned __int128 m = static_cast<unsigned __int128>(Mix64(key + static_cast<uint64_t>(i))) *
                                static_cast<uint64_t>(vocab);
    out[i] = static_cast<int32_t>(m >> 64);
  }
}

const char* rpg_synth_last_error(void) { return g_err.c_str(); }

}  // extern "C"
