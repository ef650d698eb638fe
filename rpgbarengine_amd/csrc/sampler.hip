// Exact on-GPU sampler (reference src/sampler.cc:16-112).
//
// Reference steps and how each is reproduced bit for bit:
//  1. s = logits * (1/T)                      float multiply, same
//  2. top-k (1 < k < n): kth = k-th largest,  radix select on order-preserving
//     s < kth -> -inf                         keys: exact; survivors compacted
//                                             in index order
//  3. softmax: float max, e = expf(s - max),  glibc-exact expf (expf_glibc.h);
//     double sum in index order,              the double sum is computed in
//     inv = float(1/sum), p = e * inv         parallel with a rigorous bound
//                                             |seq - par| <= 2 n u S; when
//                                             float(1/(S+-B)) agree the answer
//                                             is exact, else one thread redoes
//                                             the sequential sum
//  4. top-p: ascending std::sort, double      the zeroed set is {p < v*} plus
//     cumulative, zero while cum <= 1 - p,    J ties at v*, where v* and J come
//     renormalise (double sum, float inv)     from a radix select with exact
//                                             fixed-point mass (multiples of
//                                             2^-57); the J ties are the lowest
//                                             indices (std::sort leaves their
//                                             order unspecified); renormalise
//                                             as in step 3
//  5. first i with double cum > u, else       exact uint64 prefix sums when all
//     ArgMax(probs)                           nonzero probs are >= 2^-29
//                                             (then every partial sum is exact
//                                             in double), else sequential
//  u = float(SplitMix64(seed + 0x9E3779B97F4A7C15 * pos) >> 40) / 2^24.

#include <hip/hip_runtime.h>

#include "common.h"
#include "expf_glibc.h"
#include "sampler.h"

namespace rpg {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ uint64_t Mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ float CounterUniform(uint64_t seed, uint64_t counter) {
  const uint32_t bits = static_cast<uint32_t>(Mix64(seed + 0x9E3779B97F4A7C15ull * counter) >> 40);
  return static_cast<float>(bits) * (1.0f / 16777216.0f);
}

// Larger float -> larger key.
__device__ __forceinline__ uint32_t OrderKey(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float FromOrderKey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct Shared {
  double d[kWaves];
  float f[kWaves];
  unsigned long long u[kWaves];
  int32_t i[kWaves];
  uint32_t cnt[256];
  unsigned long long mass[256];
  uint32_t prefix, mask, krem;
  int32_t sel;
  int32_t n_surv;
  int32_t scan[kThreads];
  int32_t flag;
  float inv;
  int32_t answer;
};

template <typename T, typename Op>
__device__ __forceinline__ T WaveReduce(T v, Op op) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ double BlockSumD(double v, Shared& sh) {
  v = WaveReduce(v, [](double a, double b) { return a + b; });
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.d[threadIdx.x >> 6] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kWaves; ++w) t += sh.d[w];
  return t;
}

__device__ float BlockMaxF(float v, Shared& sh) {
  v = WaveReduce(v, [](float a, float b) { return fmaxf(a, b); });
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = sh.f[0];
  for (int w = 1; w < kWaves; ++w) t = fmaxf(t, sh.f[w]);
  return t;
}

__device__ int BlockMinI(int v, Shared& sh) {
  v = WaveReduce(v, [](int a, int b) { return a < b ? a : b; });
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.i[threadIdx.x >> 6] = v;
  __syncthreads();
  int t = sh.i[0];
  for (int w = 1; w < kWaves; ++w) t = t < sh.i[w] ? t : sh.i[w];
  return t;
}

__device__ int BlockOrI(int v, Shared& sh) {
  v = WaveReduce(v, [](int a, int b) { return a | b; });
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.i[threadIdx.x >> 6] = v;
  __syncthreads();
  int t = 0;
  for (int w = 0; w < kWaves; ++w) t |= sh.i[w];
  return t;
}

// Exclusive prefix over threads of one int per thread; returns the total.
__device__ int BlockExclusiveScan(int v, int* excl, Shared& sh) {
  __syncthreads();
  sh.scan[threadIdx.x] = v;
  __syncthreads();
  // Hillis-Steele over 1024 entries
  for (int off = 1; off < kThreads; off <<= 1) {
    const int add = threadIdx.x >= off ? sh.scan[threadIdx.x - off] : 0;
    __syncthreads();
    sh.scan[threadIdx.x] += add;
    __syncthreads();
  }
  const int incl = sh.scan[threadIdx.x];
  const int total = sh.scan[kThreads - 1];
  *excl = incl - v;
  __syncthreads();
  return total;
}

// Exact double-sum emulation: parallel sum + bound, sequential on ambiguity.
// vals(j) gives the j-th addend in index order, j < n; all addends >= 0.
template <typename Vals>
__device__ float InvOfSequentialSum(int n, Vals vals, Shared& sh, unsigned long long* fallbacks) {
  double part = 0.0;
  const int chunk = (n + kThreads - 1) / kThreads;
  const int b = threadIdx.x * chunk, e = min(n, b + chunk);
  for (int j = b; j < e; ++j) part += static_cast<double>(vals(j));
  const double S = BlockSumD(part, sh);
  const double B = 2.0 * static_cast<double>(n) * S * 0x1p-52;
  const float lo = static_cast<float>(1.0 / (S + B));
  const float hi = static_cast<float>(1.0 / (S - B));
  if (lo == hi && S - B > 0.0) return lo;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int j = 0; j < n; ++j) s += static_cast<double>(vals(j));
    sh.inv = static_cast<float>(1.0 / s);
    atomicAdd(fallbacks, 1ull);
  }
  __syncthreads();
  return sh.inv;
}

__global__ __launch_bounds__(kThreads) void SampleKernel(const float* __restrict__ logits_all, int64_t ld, int n,
                                                         const SamplerParamsDev* __restrict__ params,
                                                         const int32_t* __restrict__ counter_dev,
                                                         int64_t counter_host, int32_t* __restrict__ token_out,
                                                         float* __restrict__ work_all, int32_t* __restrict__ idx_all,
                                                         float* __restrict__ probs_out,
                                                         unsigned long long* __restrict__ fallbacks) {
  __shared__ Shared sh;
  const int row = blockIdx.x;
  const float* logits = logits_all + row * ld;
  float* work = work_all + static_cast<int64_t>(row) * n;
  int32_t* idx = idx_all + static_cast<int64_t>(row) * n;
  const SamplerParamsDev P = params[row];
  const int tid = threadIdx.x;
  const bool write_probs = probs_out != nullptr && row == 0;

  if (!(P.temperature > 0.0f)) {  // greedy: first index of the maximum
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int i = tid; i < n; i += kThreads) {
      const float v = logits[i];
      if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
      }
    }
    const float m = BlockMaxF(bv, sh);
    int cand = (bv == m) ? bi : 0x7fffffff;
    cand = BlockMinI(cand, sh);
    if (tid == 0) token_out[row] = (cand == 0x7fffffff || logits[0] != logits[0]) ? 0 : cand;
    if (write_probs) {
      for (int i = tid; i < n; i += kThreads) probs_out[i] = (i == cand) ? 1.0f : 0.0f;
    }
    return;
  }

  const bool scale_t = P.temperature != 1.0f;
  const float invT = 1.0f / P.temperature;
  auto S = [&](int i) { return scale_t ? logits[i] * invT : logits[i]; };
  const uint64_t pos = counter_dev ? static_cast<uint64_t>(counter_dev[row]) : static_cast<uint64_t>(counter_host);
  const float u = CounterUniform(P.seed, pos);
  const int chunk = (n + kThreads - 1) / kThreads;
  const int c0 = tid * chunk, c1 = min(n, c0 + chunk);

  // ---- 2. top-k threshold
  const bool use_topk = P.top_k > 1 && P.top_k < n;
  float kth = -__builtin_inff();
  if (use_topk) {
    if (tid == 0) {
      sh.prefix = 0;
      sh.mask = 0;
      sh.krem = static_cast<uint32_t>(P.top_k);
    }
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int b = tid; b < 256; b += kThreads) sh.cnt[b] = 0;
      __syncthreads();
      const uint32_t prefix = sh.prefix, mask = sh.mask;
      for (int i = tid; i < n; i += kThreads) {
        const uint32_t key = OrderKey(S(i));
        if ((key & mask) == prefix) atomicAdd(&sh.cnt[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t cum = 0;
        int sel = 0;
        for (int b = 255; b >= 0; --b) {
          if (cum + sh.cnt[b] >= sh.krem) {
            sel = b;
            break;
          }
          cum += sh.cnt[b];
        }
        sh.krem -= cum;
        sh.prefix |= static_cast<uint32_t>(sel) << shift;
        sh.mask |= 0xFFu << shift;
      }
      __syncthreads();
    }
    kth = FromOrderKey(sh.prefix);
  }

  // ---- compaction of the survivors (s >= kth), in index order
  int my = 0;
  for (int i = c0; i < c1; ++i) my += (!use_topk || S(i) >= kth) ? 1 : 0;
  int base;
  const int n_surv = BlockExclusiveScan(my, &base, sh);
  {
    int j = base;
    for (int i = c0; i < c1; ++i) {
      if (!use_topk || S(i) >= kth) idx[j++] = i;
    }
  }
  __syncthreads();
  const int schunk = (n_surv + kThreads - 1) / kThreads;
  const int s0 = tid * schunk, s1 = min(n_surv, s0 + schunk);

  // ---- 3. softmax over the survivors (masked entries are exactly 0)
  float mx = -__builtin_inff();
  for (int j = s0; j < s1; ++j) mx = fmaxf(mx, S(idx[j]));
  mx = BlockMaxF(mx, sh);
  for (int j = s0; j < s1; ++j) work[j] = GlibcExpf(S(idx[j]) - mx);
  __syncthreads();
  const float inv = InvOfSequentialSum(n_surv, [&](int j) { return work[j]; }, sh, fallbacks);
  for (int j = s0; j < s1; ++j) work[j] = work[j] * inv;
  __syncthreads();

  // ---- 4. top-p
  const bool use_topp = P.top_p > 0.0f && P.top_p < 1.0f;
  if (use_topp) {
    const double thr = 1.0 - static_cast<double>(P.top_p);
    const unsigned long long THR = static_cast<unsigned long long>(thr * 0x1p57);
    unsigned long long cum_below = 0;
    if (tid == 0) {
      sh.prefix = 0;
      sh.mask = 0;
      sh.sel = 0;
      sh.flag = 0;
    }
    __syncthreads();
    int all_zero = 0;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int b = tid; b < 256; b += kThreads) {
        sh.cnt[b] = 0;
        sh.mass[b] = 0;
      }
      __syncthreads();
      const uint32_t prefix = sh.prefix, mask = sh.mask;
      for (int j = tid; j < n_surv; j += kThreads) {
        const float p = work[j];
        const uint32_t key = __float_as_uint(p);
        if ((key & mask) == prefix) {
          const uint32_t b = (key >> shift) & 255u;
          atomicAdd(&sh.cnt[b], 1u);
          atomicAdd(&sh.mass[b], static_cast<unsigned long long>(static_cast<double>(p) * 0x1p57));
        }
      }
      __syncthreads();
      if (tid == 0) {
        int sel = -1;
        unsigned long long cum = cum_below;
        for (int b = 0; b < 256; ++b) {
          if (cum + sh.mass[b] > THR) {
            sel = b;
            break;
          }
          cum += sh.mass[b];
        }
        if (sel < 0) {
          sh.flag = 1;  // everything fits under the threshold
          sel = 255;
        }
        sh.sel = sel;
        sh.u[0] = cum;
        sh.prefix |= static_cast<uint32_t>(sel) << shift;
        sh.mask |= 0xFFu << shift;
      }
      __syncthreads();
      cum_below = sh.u[0];
      all_zero = sh.flag;
      __syncthreads();
      if (all_zero) break;
    }
    if (all_zero) {
      // Every cumulative stays <= 1 - p: the reference zeroes all and keeps
      // the largest (its sorted last); then renormalises a single 1.0.
      float bv = -1.0f;
      int bi = 0x7fffffff;
      for (int j = s0; j < s1; ++j) {
        if (work[j] > bv) {
          bv = work[j];
          bi = j;
        }
      }
      const float m = BlockMaxF(bv, sh);
      int cand = (bv == m) ? bi : 0x7fffffff;
      cand = BlockMinI(cand, sh);
      for (int j = s0; j < s1; ++j) work[j] = (j == cand) ? 1.0f : 0.0f;
      __syncthreads();
    } else {
      const float vstar = __uint_as_float(sh.prefix);
      const unsigned long long V = static_cast<unsigned long long>(static_cast<double>(vstar) * 0x1p57);
      const unsigned long long room = THR - cum_below;
      const long long J = V > 0 ? static_cast<long long>(room / V) : 0;
      // rank the ties at v* by index
      int ties = 0;
      for (int j = s0; j < s1; ++j) ties += work[j] == vstar ? 1 : 0;
      int tie_base;
      (void)BlockExclusiveScan(ties, &tie_base, sh);
      int r = tie_base;
      for (int j = s0; j < s1; ++j) {
        const float p = work[j];
        if (p < vstar) {
          work[j] = 0.0f;
        } else if (p == vstar) {
          if (r < J) work[j] = 0.0f;
          ++r;
        }
      }
      __syncthreads();
      const float inv2 = InvOfSequentialSum(n_surv, [&](int j) { return work[j]; }, sh, fallbacks);
      for (int j = s0; j < s1; ++j) work[j] = work[j] * inv2;
      __syncthreads();
    }
  }

  // ---- 5. inverse CDF: first j with cum > u
  // exact in uint64 fixed point (2^-52 units) when every nonzero p >= 2^-29
  int tiny = 0;
  for (int j = s0; j < s1; ++j) {
    const float p = work[j];
    tiny |= (p != 0.0f && p < 0x1p-29f) ? 1 : 0;
  }
  tiny = BlockOrI(tiny, sh);
  if (tid == 0) sh.answer = -1;
  __syncthreads();
  if (!tiny) {
    unsigned long long mine = 0;
    for (int j = s0; j < s1; ++j) mine += static_cast<unsigned long long>(static_cast<double>(work[j]) * 0x1p52);
    // exclusive scan of the 64-bit partials (two 32-bit halves would lose
    // carries; reuse the double slots as u64 via a serial pass over waves)
    __syncthreads();
    unsigned long long incl = mine;
    for (int off = 1; off < 64; off <<= 1) {
      const unsigned long long o = __shfl_up(incl, off, 64);
      if ((tid & 63) >= off) incl += o;
    }
    if ((tid & 63) == 63) sh.u[tid >> 6] = incl;
    __syncthreads();
    unsigned long long wave_base = 0;
    for (int w = 0; w < (tid >> 6); ++w) wave_base += sh.u[w];
    unsigned long long cum = wave_base + incl - mine;
    const unsigned long long U = static_cast<unsigned long long>(static_cast<double>(u) * 0x1p52);
    int found = 0x7fffffff;
    for (int j = s0; j < s1; ++j) {
      cum += static_cast<unsigned long long>(static_cast<double>(work[j]) * 0x1p52);
      if (cum > U) {
        found = j;
        break;
      }
    }
    found = BlockMinI(found, sh);
    if (tid == 0 && found != 0x7fffffff) sh.answer = found;
  } else {
    if (tid == 0) {
      double cum = 0.0;
      for (int j = 0; j < n_surv; ++j) {
        cum += static_cast<double>(work[j]);
        if (cum > static_cast<double>(u)) {
          sh.answer = j;
          break;
        }
      }
      atomicAdd(fallbacks, 1ull);
    }
  }
  __syncthreads();
  int ans = sh.answer;
  if (ans < 0) {
    // ArgMax(probs) over the full vocabulary: masked entries are 0, so the
    // first maximum among survivors (in index order) unless all are 0.
    float bv = -1.0f;
    int bi = 0x7fffffff;
    for (int j = s0; j < s1; ++j) {
      if (work[j] > bv) {
        bv = work[j];
        bi = j;
      }
    }
    const float m = BlockMaxF(bv, sh);
    int cand = (bv == m) ? bi : 0x7fffffff;
    cand = BlockMinI(cand, sh);
    ans = cand;
    if (m <= 0.0f) ans = -2;  // all probabilities 0: argmax is index 0
  }
  if (tid == 0) token_out[row] = ans == -2 ? 0 : idx[ans];
  if (write_probs) {
    for (int i = tid; i < n; i += kThreads) probs_out[i] = 0.0f;
    __syncthreads();
    for (int j = s0; j < s1; ++j) probs_out[idx[j]] = work[j];
  }
}

}  // namespace

Sampler::Sampler(int rows, int vocab) : rows_(rows), vocab_(vocab) {
  HIP_CHECK(hipMalloc(&params_, sizeof(SamplerParamsDev) * rows));
  HIP_CHECK(hipMalloc(&work_, sizeof(float) * static_cast<size_t>(rows) * vocab));
  HIP_CHECK(hipMalloc(&idx_, sizeof(int32_t) * static_cast<size_t>(rows) * vocab));
  HIP_CHECK(hipMalloc(&fallbacks_, sizeof(unsigned long long)));
  HIP_CHECK(hipMemset(fallbacks_, 0, sizeof(unsigned long long)));
  HIP_CHECK(hipMemset(params_, 0, sizeof(SamplerParamsDev) * rows));
}

Sampler::~Sampler() {
  (void)hipFree(params_);
  (void)hipFree(work_);
  (void)hipFree(idx_);
  (void)hipFree(fallbacks_);
}

void Sampler::SetParams(const SamplerParamsDev* p, int rows, hipStream_t s) {
  RPG_CHECK(rows <= rows_, "sampler: %d rows > capacity %d", rows, rows_);
  HIP_CHECK(hipMemcpyAsync(params_, p, sizeof(SamplerParamsDev) * rows, hipMemcpyHostToDevice, s));
}

void Sampler::Enqueue(const float* logits, int64_t ld, const int32_t* counter, int64_t counter_host, int32_t* token,
                      float* probs_out, hipStream_t s) {
  hipLaunchKernelGGL(SampleKernel, dim3(static_cast<unsigned>(rows_)), dim3(kThreads), 0, s, logits, ld, vocab_,
                     params_, counter, counter_host, token, work_, idx_, probs_out, fallbacks_);
  HIP_CHECK(hipGetLastError());
}

int64_t Sampler::FallbackCount(hipStream_t s) const {
  unsigned long long v = 0;
  HIP_CHECK(hipMemcpyAsync(&v, fallbacks_, sizeof(v), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  return static_cast<int64_t>(v);
}

}  // namespace rpg
