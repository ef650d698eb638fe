// Counter-based uniform + temperature/top-k/top-p filter + inverse-CDF draw --
// restates reference src/sampler.cc:16-112. Non-AVX TU; std::exp(float) is
// glibc expf, as in the reference.

#include <algorithm>
#include <cmath>
#include <limits>

#include "oracle.h"

namespace orc {

// reference src/sampler.cc:16-22 (the SplitMix64 finaliser constants)
uint64_t SplitMix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// reference src/sampler.cc:24-28
uint64_t CounterRng(uint64_t seed, uint64_t counter) {
  return SplitMix64(seed + 0x9E3779B97F4A7C15ull * counter);
}

// reference src/sampler.cc:30-34: top 24 bits / 2^24
float CounterUniform(uint64_t seed, uint64_t counter) {
  const uint32_t bits = static_cast<uint32_t>(CounterRng(seed, counter) >> 40);
  return static_cast<float>(bits) * (1.0f / 16777216.0f);
}

// reference src/sampler.cc:36-94
void FilterToProbs(const float* logits, int64_t n, const SampleOptions& opt,
                   std::vector<float>* probs) {
  probs->assign(logits, logits + n);
  float* s = probs->data();
  if (!(opt.temperature > 0.0f)) {  // greedy: one-hot at the first maximum
    const int32_t best = ArgMax(s, n);
    std::fill(s, s + n, 0.0f);
    s[best] = 1.0f;
    return;
  }
  if (opt.temperature != 1.0f) {
    const float inv = 1.0f / opt.temperature;
    for (int64_t i = 0; i < n; ++i) s[i] *= inv;
  }
  if (opt.top_k > 1 && opt.top_k < n) {
    // k-th largest value as threshold; strictly smaller values drop out
    std::vector<float> tmp(s, s + n);
    std::nth_element(tmp.begin(), tmp.begin() + (opt.top_k - 1), tmp.end(), std::greater<float>());
    const float kth = tmp[opt.top_k - 1];
    for (int64_t i = 0; i < n; ++i)
      if (s[i] < kth) s[i] = -std::numeric_limits<float>::infinity();
  }
  SoftmaxInPlace(s, n);
  if (opt.top_p > 0.0f && opt.top_p < 1.0f) {
    // ascending order; zero the tail while the double cumulative <= 1 - p;
    // always keep the largest; renormalise with a double sum.
    std::vector<int32_t> order(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) order[i] = static_cast<int32_t>(i);
    std::sort(order.begin(), order.end(), [s](int32_t a, int32_t b) { return s[a] < s[b]; });
    const double limit = 1.0 - static_cast<double>(opt.top_p);
    double cum = 0.0;
    for (int64_t j = 0; j < n; ++j) {
      cum += static_cast<double>(s[order[j]]);
      if (cum <= limit) s[order[j]] = 0.0f;
    }
    if (n > 0 && s[order[n - 1]] == 0.0f) s[order[n - 1]] = 1.0f;
    double total = 0.0;
    for (int64_t i = 0; i < n; ++i) total += static_cast<double>(s[i]);
    if (total > 0.0) {
      const float inv = static_cast<float>(1.0 / total);
      for (int64_t i = 0; i < n; ++i) s[i] *= inv;
    }
  }
}

// reference src/sampler.cc:96-112: first index whose double cumulative > u.
int32_t SampleToken(const float* logits, int64_t n, const SampleOptions& opt, float u) {
  if (!(opt.temperature > 0.0f)) return ArgMax(logits, n);
  std::vector<float> probs;
  FilterToProbs(logits, n, opt, &probs);
  double cum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    cum += static_cast<double>(probs[i]);
    if (cum > static_cast<double>(u)) return static_cast<int32_t>(i);
  }
  return ArgMax(probs.data(), n);
}

}  // namespace orc
