// Scalar reference dot and kernel dispatch -- restates reference
// src/matmul.cc:28-124. Non-AVX translation unit (no contraction).

#include <cstdlib>

#include "oracle.h"

namespace orc {

// reference src/matmul.cc:73-102: dequantise one block to a stack buffer,
// four lane accumulators s[j % 4], tail into s0, return (s0+s1)+(s2+s3).
float DotRowScalar(uint32_t type, const float* a, const uint8_t* w, int64_t k) {
  float tmp[256];
  const int64_t be = BlockElems(type);
  const int64_t bb = BlockBytes(type);
  ORC_CHECK(be > 0, "unsupported ggml type %u", type);
  ORC_CHECK(k % be == 0, "dot length %lld is not a multiple of %lld", (long long)k, (long long)be);
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  for (int64_t b = 0; b < k / be; ++b) {
    DequantizeRow(type, w + b * bb, be, tmp);
    const float* ab = a + b * be;
    int64_t j = 0;
    for (; j < be - 3; j += 4) {
      s0 += ab[j] * tmp[j];
      s1 += ab[j + 1] * tmp[j + 1];
      s2 += ab[j + 2] * tmp[j + 2];
      s3 += ab[j + 3] * tmp[j + 3];
    }
    for (; j < be; ++j) s0 += ab[j] * tmp[j];
  }
  return (s0 + s1) + (s2 + s3);
}

namespace {

// reference src/matmul.cc:41-54: RPGBAR_NO_SIMD=1 or no AVX2+FMA -> scalar.
bool UseSimd() {
  const char* v = std::getenv("RPGBAR_NO_SIMD");
  if (v != nullptr && v[0] != '\0' && v[0] != '0') return false;
  return Avx2Available();
}

const bool g_simd = UseSimd();

}  // namespace

// reference src/matmul.cc:106-108
float DotRowQuant(uint32_t type, const float* a, const uint8_t* w, int64_t k) {
  return g_simd ? DotRowAvx2(type, a, w, k) : DotRowScalar(type, a, w, k);
}

// reference src/model.cc:32-37
void Matrix::Row(int64_t r, float* out) const {
  ORC_CHECK(r >= 0 && r < rows, "row %lld out of range (%lld rows)", (long long)r, (long long)rows);
  DequantizeRow(type, data + r * RowBytes(type, cols), cols, out);
}

// reference src/model.cc:39-69: n >= 8 -> blocked kernel; otherwise every
// (token, row) dot independently, flattened i = t*rows + r, pooled if > 256.
void Matrix::MatMulBatch(const float* X, int64_t n, float* OUT, Pool* pool) const {
  const int64_t rb = RowBytes(type, cols);
  if (n >= 8 && g_simd && MatMulBlockedAvx2(type, data, rows, cols, X, n, OUT, pool)) return;
  auto body = [&](int64_t begin, int64_t end) {
    for (int64_t i = begin; i < end; ++i) {
      const int64_t t = i / rows;
      const int64_t r = i - t * rows;
      OUT[t * rows + r] = DotRowQuant(type, X + t * cols, data + r * rb, cols);
    }
  };
  const int64_t total = n * rows;
  if (pool && total > 256) {
    pool->ParallelForRange(total, body);
  } else {
    body(0, total);
  }
}

}  // namespace orc
