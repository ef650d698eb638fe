// AVX2+FMA fused dequant dots -- restates reference src/matmul_avx2.cc.
//
// Bitwise parity with the reference needs the same vector operation order:
// four 8-lane accumulators per dot (one per 8-element slice of each 32-element
// step), the Q4_K weight formed as fmsub(d*sc, nibble, dmin*m), Q6_K/Q8_0
// weights as (d*sc)*q, and the same horizontal sum. The blocked kernel keeps
// one accumulator per token over 8 tokens. This TU alone gets -mavx2 -mfma.

#include <immintrin.h>

#include "oracle.h"

namespace orc {

bool Avx2Available() {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

namespace {

// reference src/matmul_avx2.cc:41-50: ((l0+h0)+(l1+h1)) + ((l2+h2)+(l3+h3))
inline float HorizontalSum(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v);
  const __m128 hi = _mm256_extractf128_ps(v, 1);
  lo = _mm_add_ps(lo, hi);
  __m128 odd = _mm_movehdup_ps(lo);
  __m128 pair = _mm_add_ps(lo, odd);
  odd = _mm_movehl_ps(odd, pair);
  pair = _mm_add_ss(pair, odd);
  return _mm_cvtss_f32(pair);
}

inline __m256 U8ToF32(__m128i x) { return _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(x)); }
inline __m256 I8ToF32(__m128i x) { return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(x)); }
inline __m128i Hi8(__m128i x) { return _mm_srli_si128(x, 8); }

inline float HalfAt(const uint8_t* p) { return HalfToFloat(Load16(p)); }

// Q4_K group g of a block: 32 quant bytes -> low nibbles (sub-block 2g) and
// high nibbles (sub-block 2g+1) as four 8-byte halves each.
struct Q4Group {
  __m128i lo0, lo1, hi0, hi1;
  float d_lo, m_lo, d_hi, m_hi;
};

inline Q4Group LoadQ4Group(const uint8_t* blk, int g) {
  const float d = HalfAt(blk);
  const float dmin = HalfAt(blk + 2);
  Q4Group r;
  uint8_t sc, mn;
  ScaleMinK4(2 * g, blk + 4, &sc, &mn);
  r.d_lo = d * static_cast<float>(sc);
  r.m_lo = dmin * static_cast<float>(mn);
  ScaleMinK4(2 * g + 1, blk + 4, &sc, &mn);
  r.d_hi = d * static_cast<float>(sc);
  r.m_hi = dmin * static_cast<float>(mn);
  const __m256i mask = _mm256_set1_epi8(0x0F);
  const __m256i q = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(blk + 16 + 32 * g));
  const __m256i lo = _mm256_and_si256(q, mask);
  const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), mask);
  r.lo0 = _mm256_castsi256_si128(lo);
  r.lo1 = _mm256_extracti128_si256(lo, 1);
  r.hi0 = _mm256_castsi256_si128(hi);
  r.hi1 = _mm256_extracti128_si256(hi, 1);
  return r;
}

// Q6_K: 8 positions l0..l0+7 of one half -> the four 6-bit codes minus 32
// (reference src/matmul_avx2.cc:218-244).
inline void Q6Codes(const uint8_t* ql, const uint8_t* qh, int l0, __m256* c0, __m256* c1,
                    __m256* c2, __m256* c3) {
  const __m256i m4 = _mm256_set1_epi32(0x0F);
  const __m256i m2 = _mm256_set1_epi32(0x03);
  const __m256i off = _mm256_set1_epi32(32);
  const __m256i a = _mm256_cvtepu8_epi32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(ql + l0)));
  const __m256i b = _mm256_cvtepu8_epi32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(ql + l0 + 32)));
  const __m256i h = _mm256_cvtepu8_epi32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(qh + l0)));
  const __m256i v0 = _mm256_or_si256(_mm256_and_si256(a, m4), _mm256_slli_epi32(_mm256_and_si256(h, m2), 4));
  const __m256i v1 = _mm256_or_si256(_mm256_and_si256(b, m4),
                                     _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 2), m2), 4));
  const __m256i v2 = _mm256_or_si256(_mm256_srli_epi32(a, 4),
                                     _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 4), m2), 4));
  const __m256i v3 = _mm256_or_si256(_mm256_srli_epi32(b, 4),
                                     _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 6), m2), 4));
  *c0 = _mm256_cvtepi32_ps(_mm256_sub_epi32(v0, off));
  *c1 = _mm256_cvtepi32_ps(_mm256_sub_epi32(v1, off));
  *c2 = _mm256_cvtepi32_ps(_mm256_sub_epi32(v2, off));
  *c3 = _mm256_cvtepi32_ps(_mm256_sub_epi32(v3, off));
}

// ---------------------------------------------------------------- M = 1

// reference src/matmul_avx2.cc:95-115
float DotF32(const float* a, const uint8_t* w, int64_t k) {
  const float* wf = reinterpret_cast<const float*>(w);
  __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
  __m256 s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
  int64_t i = 0;
  for (; i + 32 <= k; i += 32) {
    s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(wf + i), s0);
    s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(wf + i + 8), s1);
    s2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(wf + i + 16), s2);
    s3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(wf + i + 24), s3);
  }
  for (; i + 8 <= k; i += 8) s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(wf + i), s0);
  float s = HorizontalSum(_mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3)));
  for (; i < k; ++i) s += a[i] * wf[i];
  return s;
}

// reference src/matmul_avx2.cc:121-149
float DotQ8_0(const float* a, const uint8_t* w, int64_t k) {
  __m256 s[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  for (int64_t b = 0; b < k / 32; ++b) {
    const uint8_t* blk = w + b * 34;
    const __m256 d = _mm256_set1_ps(HalfAt(blk));
    for (int j = 0; j < 4; ++j) {
      const __m256 q = I8ToF32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(blk + 2 + 8 * j)));
      s[j] = _mm256_fmadd_ps(_mm256_loadu_ps(a + b * 32 + 8 * j), _mm256_mul_ps(d, q), s[j]);
    }
  }
  return HorizontalSum(_mm256_add_ps(_mm256_add_ps(s[0], s[1]), _mm256_add_ps(s[2], s[3])));
}

// reference src/matmul_avx2.cc:160-205: acc += a * fmsub(d*sc, nibble, dmin*m)
float DotQ4_K(const float* a, const uint8_t* w, int64_t k) {
  __m256 s[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  for (int64_t b = 0; b < k / 256; ++b) {
    const uint8_t* blk = w + b * 144;
    const float* ab = a + b * 256;
    for (int g = 0; g < 4; ++g) {
      const Q4Group q = LoadQ4Group(blk, g);
      const __m256 dl = _mm256_set1_ps(q.d_lo), ml = _mm256_set1_ps(q.m_lo);
      const __m256 dh = _mm256_set1_ps(q.d_hi), mh = _mm256_set1_ps(q.m_hi);
      const __m128i parts_lo[4] = {q.lo0, Hi8(q.lo0), q.lo1, Hi8(q.lo1)};
      const __m128i parts_hi[4] = {q.hi0, Hi8(q.hi0), q.hi1, Hi8(q.hi1)};
      for (int j = 0; j < 4; ++j)
        s[j] = _mm256_fmadd_ps(_mm256_loadu_ps(ab + 64 * g + 8 * j),
                               _mm256_fmsub_ps(dl, U8ToF32(parts_lo[j]), ml), s[j]);
      for (int j = 0; j < 4; ++j)
        s[j] = _mm256_fmadd_ps(_mm256_loadu_ps(ab + 64 * g + 32 + 8 * j),
                               _mm256_fmsub_ps(dh, U8ToF32(parts_hi[j]), mh), s[j]);
    }
  }
  return HorizontalSum(_mm256_add_ps(_mm256_add_ps(s[0], s[1]), _mm256_add_ps(s[2], s[3])));
}

// reference src/matmul_avx2.cc:246-289
float DotQ6_K(const float* a, const uint8_t* w, int64_t k) {
  __m256 s[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  for (int64_t b = 0; b < k / 256; ++b) {
    const uint8_t* blk = w + b * 210;
    const float d = HalfAt(blk + 208);
    const int8_t* scales = reinterpret_cast<const int8_t*>(blk + 192);
    for (int half = 0; half < 2; ++half) {
      const uint8_t* ql = blk + 64 * half;
      const uint8_t* qh = blk + 128 + 32 * half;
      const int8_t* sc = scales + 8 * half;
      const float* ab = a + b * 256 + 128 * half;
      for (int l0 = 0; l0 < 32; l0 += 8) {
        __m256 c[4];
        Q6Codes(ql, qh, l0, &c[0], &c[1], &c[2], &c[3]);
        const int si = l0 >> 4;
        for (int j = 0; j < 4; ++j) {
          const __m256 scale = _mm256_set1_ps(d * static_cast<float>(sc[si + 2 * j]));
          s[j] = _mm256_fmadd_ps(_mm256_loadu_ps(ab + 32 * j + l0), _mm256_mul_ps(scale, c[j]), s[j]);
        }
      }
    }
  }
  return HorizontalSum(_mm256_add_ps(_mm256_add_ps(s[0], s[1]), _mm256_add_ps(s[2], s[3])));
}

// ---------------------------------------------------------------- 8 tokens x 1 row

// acc[t] += X[t][off .. off+8) * wv for t = 0..7 (reference :309-320)
inline void Acc8(__m256* acc, const float* xbase, int64_t ld, int64_t off, __m256 wv) {
  for (int t = 0; t < 8; ++t) acc[t] = _mm256_fmadd_ps(_mm256_loadu_ps(xbase + t * ld + off), wv, acc[t]);
}

// reference :335-383
void Row8Q4K(const uint8_t* w, int64_t cols, const float* xbase, int64_t ld, __m256* acc) {
  for (int64_t b = 0; b < cols / 256; ++b) {
    const uint8_t* blk = w + b * 144;
    for (int g = 0; g < 4; ++g) {
      const Q4Group q = LoadQ4Group(blk, g);
      const __m256 dl = _mm256_set1_ps(q.d_lo), ml = _mm256_set1_ps(q.m_lo);
      const __m256 dh = _mm256_set1_ps(q.d_hi), mh = _mm256_set1_ps(q.m_hi);
      const __m128i parts_lo[4] = {q.lo0, Hi8(q.lo0), q.lo1, Hi8(q.lo1)};
      const __m128i parts_hi[4] = {q.hi0, Hi8(q.hi0), q.hi1, Hi8(q.hi1)};
      const int64_t base = b * 256 + 64 * g;
      for (int j = 0; j < 4; ++j) Acc8(acc, xbase, ld, base + 8 * j, _mm256_fmsub_ps(dl, U8ToF32(parts_lo[j]), ml));
      for (int j = 0; j < 4; ++j) Acc8(acc, xbase, ld, base + 32 + 8 * j, _mm256_fmsub_ps(dh, U8ToF32(parts_hi[j]), mh));
    }
  }
}

// reference :386-426
void Row8Q6K(const uint8_t* w, int64_t cols, const float* xbase, int64_t ld, __m256* acc) {
  for (int64_t b = 0; b < cols / 256; ++b) {
    const uint8_t* blk = w + b * 210;
    const float d = HalfAt(blk + 208);
    const int8_t* scales = reinterpret_cast<const int8_t*>(blk + 192);
    for (int half = 0; half < 2; ++half) {
      const uint8_t* ql = blk + 64 * half;
      const uint8_t* qh = blk + 128 + 32 * half;
      const int8_t* sc = scales + 8 * half;
      for (int l0 = 0; l0 < 32; l0 += 8) {
        __m256 c[4];
        Q6Codes(ql, qh, l0, &c[0], &c[1], &c[2], &c[3]);
        const int si = l0 >> 4;
        __m256 s[4];
        for (int j = 0; j < 4; ++j) s[j] = _mm256_set1_ps(d * static_cast<float>(sc[si + 2 * j]));
        const int64_t base = b * 256 + 128 * half + l0;
        for (int j = 0; j < 4; ++j) Acc8(acc, xbase, ld, base + 32 * j, _mm256_mul_ps(s[j], c[j]));
      }
    }
  }
}

// reference :429-448
void Row8Q8_0(const uint8_t* w, int64_t cols, const float* xbase, int64_t ld, __m256* acc) {
  for (int64_t b = 0; b < cols / 32; ++b) {
    const uint8_t* blk = w + b * 34;
    const __m256 d = _mm256_set1_ps(HalfAt(blk));
    for (int i = 0; i < 4; ++i) {
      const __m256 wv = _mm256_mul_ps(d, I8ToF32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(blk + 2 + 8 * i))));
      Acc8(acc, xbase, ld, b * 32 + 8 * i, wv);
    }
  }
}

// reference :451-463 (a tail of cols % 8 is not visited, as in the reference)
void Row8F32(const uint8_t* w, int64_t cols, const float* xbase, int64_t ld, __m256* acc) {
  const float* wf = reinterpret_cast<const float*>(w);
  for (int64_t i = 0; i < cols / 8; ++i) Acc8(acc, xbase, ld, 8 * i, _mm256_loadu_ps(wf + 8 * i));
}

bool HasBlocked(uint32_t type) {
  return type == kQ4_K || type == kQ6_K || type == kQ8_0 || type == kF32;
}

}  // namespace

// reference src/matmul_avx2.cc:511-531
float DotRowAvx2(uint32_t type, const float* a, const uint8_t* w, int64_t k) {
  switch (type) {
    case kQ4_K:
      ORC_CHECK(k % 256 == 0, "Q4_K dot length %lld", (long long)k);
      return DotQ4_K(a, w, k);
    case kQ6_K:
      ORC_CHECK(k % 256 == 0, "Q6_K dot length %lld", (long long)k);
      return DotQ6_K(a, w, k);
    case kQ8_0:
      ORC_CHECK(k % 32 == 0, "Q8_0 dot length %lld", (long long)k);
      return DotQ8_0(a, w, k);
    case kF32: return DotF32(a, w, k);
    default: return DotRowScalar(type, a, w, k);
  }
}

// reference src/matmul_avx2.cc:482-507: rows in parallel; per row, groups of
// 8 tokens share one weight read; the < 8 token tail uses the per-token dot.
bool MatMulBlockedAvx2(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols,
                       const float* X, int64_t n_tokens, float* OUT, Pool* pool) {
  if (!HasBlocked(type) || n_tokens < 8) return false;
  const int64_t rb = RowBytes(type, cols);
  auto body = [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      const uint8_t* wr = w + r * rb;
      int64_t t = 0;
      for (; t + 8 <= n_tokens; t += 8) {
        __m256 acc[8];
        for (int i = 0; i < 8; ++i) acc[i] = _mm256_setzero_ps();
        const float* xb = X + t * cols;
        switch (type) {
          case kQ4_K: Row8Q4K(wr, cols, xb, cols, acc); break;
          case kQ6_K: Row8Q6K(wr, cols, xb, cols, acc); break;
          case kQ8_0: Row8Q8_0(wr, cols, xb, cols, acc); break;
          default: Row8F32(wr, cols, xb, cols, acc); break;
        }
        for (int i = 0; i < 8; ++i) OUT[(t + i) * rows + r] = HorizontalSum(acc[i]);
      }
      for (; t < n_tokens; ++t) OUT[t * rows + r] = DotRowAvx2(type, X + t * cols, wr, cols);
    }
  };
  if (pool != nullptr) {
    pool->ParallelForRange(rows, body);
  } else {
    body(0, rows);
  }
  return true;
}

}  // namespace orc
