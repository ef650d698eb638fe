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
//
// Launch shapes. With top-k: 256-thread workgroups each take a 4096-logit
// slice and radix-select their local top-k candidates in LDS (written in
// index order); one 1024-thread workgroup per row gathers them, selects the
// global k-th value, and one wave of it finishes on the survivors. Every
// survivor is a candidate: a slice cannot hold k values strictly above the
// global k-th, so its local k-th value is <= the global one. Without top-k
// one 1024-thread workgroup per row finishes over the whole vocabulary.
// Radix selections find their bin with one wave's prefix sums.

#include <hip/hip_runtime.h>

#include "common.h"
#include "expf_glibc.h"
#include "lanes.h"
#include "sampler.h"

namespace rpg {

namespace {

constexpr int kThreads = 1024;
constexpr int kSlice = 4096;       // logits per selection workgroup
constexpr int kSelThreads = 256;
constexpr int kWaveFinish = 2048;  // survivors finished by a single wave

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

using lanes::WaveReduce;

// Histogram add: the lanes that share the first active lane's bin (most of
// them, for the high digits of float keys) add through one aggregated LDS
// atomic; the rest add with one atomic each, issued together. Every lane of
// the wave must call it (uniform control flow); `active` selects
// contributors.
__device__ __forceinline__ void AggAdd(uint32_t* cnt, unsigned long long* mass, bool active, uint32_t bin,
                                       unsigned long long m) {
  const int lane = threadIdx.x & 63;
  const unsigned long long pending = __ballot(active);
  if (pending == 0) return;
  const int leader = __ffsll(static_cast<long long>(pending)) - 1;
  const uint32_t lbin = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bin), leader));
  const bool mine = active && bin == lbin;
  const unsigned long long group = __ballot(mine);
  if (mass) {
    const unsigned long long v =
        WaveReduce(mine ? m : 0ull, [](unsigned long long a, unsigned long long b) { return a + b; });
    if (lane == leader) atomicAdd(&mass[lbin], v);
  }
  if (lane == leader) atomicAdd(&cnt[lbin], static_cast<uint32_t>(__popcll(group)));
  if (active && !mine) {
    atomicAdd(&cnt[bin], 1u);
    if (mass) atomicAdd(&mass[bin], m);
  }
}

// Block-shared scratch, templated on the block size. A one-wave instance
// (NT == 64) serves the survivors' finish, run by wave 0 of a bigger
// workgroup.
template <int NT>
struct Shared {
  static constexpr int kW = NT / 64;
  double d[kW];
  float f[kW];
  unsigned long long u[kW];
  int32_t i[kW];
  alignas(16) uint32_t cnt[256];
  alignas(16) unsigned long long mass[256];
  uint32_t sel, above;
  int32_t scan[NT];
  int32_t flag;
  float inv;
  int32_t answer;
};

// Synchronisation of the helpers below (they share LDS and the global work
// arrays between threads): a workgroup barrier, or for the one-wave
// instance release / acquire fences only.
template <int NT>
__device__ __forceinline__ void BlockSync() {
  if constexpr (NT == 64) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  } else {
    __syncthreads();
  }
}

template <int NT>
__device__ double BlockSumD(double v, Shared<NT>& sh) {
  v = WaveReduce(v, [](double a, double b) { return a + b; });
  if constexpr (NT == 64) return v;
  BlockSync<NT>();
  if ((threadIdx.x & 63) == 0) sh.d[threadIdx.x >> 6] = v;
  BlockSync<NT>();
  double t = 0.0;
  for (int w = 0; w < Shared<NT>::kW; ++w) t += sh.d[w];
  return t;
}

template <int NT>
__device__ float BlockMaxF(float v, Shared<NT>& sh) {
  v = WaveReduce(v, [](float a, float b) { return fmaxf(a, b); });
  if constexpr (NT == 64) return v;
  BlockSync<NT>();
  if ((threadIdx.x & 63) == 0) sh.f[threadIdx.x >> 6] = v;
  BlockSync<NT>();
  float t = sh.f[0];
  for (int w = 1; w < Shared<NT>::kW; ++w) t = fmaxf(t, sh.f[w]);
  return t;
}

template <int NT>
__device__ int BlockMinI(int v, Shared<NT>& sh) {
  v = WaveReduce(v, [](int a, int b) { return a < b ? a : b; });
  if constexpr (NT == 64) return v;
  BlockSync<NT>();
  if ((threadIdx.x & 63) == 0) sh.i[threadIdx.x >> 6] = v;
  BlockSync<NT>();
  int t = sh.i[0];
  for (int w = 1; w < Shared<NT>::kW; ++w) t = t < sh.i[w] ? t : sh.i[w];
  return t;
}

template <int NT>
__device__ int BlockOrI(int v, Shared<NT>& sh) {
  v = WaveReduce(v, [](int a, int b) { return a | b; });
  if constexpr (NT == 64) return v;
  BlockSync<NT>();
  if ((threadIdx.x & 63) == 0) sh.i[threadIdx.x >> 6] = v;
  BlockSync<NT>();
  int t = 0;
  for (int w = 0; w < Shared<NT>::kW; ++w) t |= sh.i[w];
  return t;
}

// Exclusive prefix over threads of one int per thread; returns the total
// and leaves each thread's inclusive prefix in sh.scan[thread].
template <int NT>
__device__ int BlockExclusiveScan(int v, int* excl, Shared<NT>& sh) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int incl = lanes::WaveInclusiveAdd(v);
  int base = 0, total;
  if constexpr (NT == 64) {
    total = lanes::ReadLaneT(incl, 63);
  } else {
    BlockSync<NT>();
    if (lane == 63) sh.i[w] = incl;
    BlockSync<NT>();
    total = 0;
    for (int q = 0; q < Shared<NT>::kW; ++q) {
      base += q < w ? sh.i[q] : 0;
      total += sh.i[q];
    }
  }
  *excl = base + incl - v;
  sh.scan[tid] = base + incl;
  BlockSync<NT>();
  return total;
}

// One wave (lanes 0..63; lane l owns bins 4l..4l+3): the bin of the
// krem-th largest key -- the highest b with sum_{b' >= b} cnt[b'] >= krem --
// and the count strictly above it, as a scan from bin 255 down would find
// them (bin 0 and the total when krem exceeds the total).
__device__ __forceinline__ void SelectBinDesc(const uint32_t* cnt, uint32_t krem, uint32_t* sel_out,
                                              uint32_t* above_out) {
  const int lane = threadIdx.x & 63;
  const uint4 c4 = reinterpret_cast<const uint4*>(cnt)[lane];
  const uint32_t cb[4] = {c4.x, c4.y, c4.z, c4.w};
  const uint32_t s = (cb[0] + cb[1]) + (cb[2] + cb[3]);
  const uint32_t incl = lanes::WaveInclusiveAdd(s);
  const uint32_t suf = lanes::ReadLaneT(incl, 63) - incl + s;  // count of bins >= 4 * lane
  const unsigned long long m = __ballot(suf >= krem);
  const int L = m ? 63 - __clzll(static_cast<long long>(m)) : 0;
  if (lane == L) {
    uint32_t cum = suf - s;
    uint32_t sel = 4u * static_cast<uint32_t>(L);
#pragma unroll
    for (int b = 3; b >= 0; --b) {
      if (cum + cb[b] >= krem) {
        sel = 4u * static_cast<uint32_t>(L) + static_cast<uint32_t>(b);
        break;
      }
      cum += cb[b];
    }
    *sel_out = sel;
    *above_out = cum;
  }
}

// One wave: the first bin b (from 0) with below + sum_{b' <= b} mass[b'] >
// thr, and the mass below it; flag = 1 (bin 255, mass below it all) when no
// bin gets there -- as a scan from bin 0 up would find them.
__device__ __forceinline__ void SelectBinAsc(const unsigned long long* mass, unsigned long long below,
                                             unsigned long long thr, uint32_t* sel_out,
                                             unsigned long long* below_out, int32_t* flag_out) {
  const int lane = threadIdx.x & 63;
  const unsigned long long mb[4] = {mass[4 * lane], mass[4 * lane + 1], mass[4 * lane + 2], mass[4 * lane + 3]};
  const unsigned long long s = (mb[0] + mb[1]) + (mb[2] + mb[3]);
  const unsigned long long pre = lanes::WaveInclusiveAdd(s);  // mass of bins <= 4 * lane + 3
  const unsigned long long m = __ballot(below + pre > thr);
  if (m == 0) {
    if (lane == 63) {
      *sel_out = 255u;
      *below_out = below + pre;
      *flag_out = 1;
    }
    return;
  }
  const int L = __ffsll(static_cast<long long>(m)) - 1;
  if (lane == L) {
    unsigned long long cum = below + pre - s;
    uint32_t sel = 4u * static_cast<uint32_t>(L) + 3u;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (cum + mb[b] > thr) {
        sel = 4u * static_cast<uint32_t>(L) + static_cast<uint32_t>(b);
        break;
      }
      cum += mb[b];
    }
    *sel_out = sel;
    *below_out = cum;
    *flag_out = 0;
  }
}

// Key of the k-th largest of n keys (key(i), i < n), by four 8-bit radix
// passes from the top (counting duplicates, as nth_element does).
template <int NT, typename Key>
__device__ uint32_t RadixKth(int n, int k, Key key, Shared<NT>& sh) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0, krem = static_cast<uint32_t>(k);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int b = tid; b < 256; b += NT) sh.cnt[b] = 0;
    BlockSync<NT>();
    for (int base = 0; base < n; base += NT) {
      const int i = base + tid;
      bool act = false;
      uint32_t bin = 0;
      if (i < n) {
        const uint32_t kk = key(i);
        act = (kk & mask) == prefix;
        bin = (kk >> shift) & 255u;
      }
      AggAdd(sh.cnt, nullptr, act, bin, 0ull);
    }
    BlockSync<NT>();
    if (tid < 64) SelectBinDesc(sh.cnt, krem, &sh.sel, &sh.above);
    BlockSync<NT>();
    krem -= sh.above;
    prefix |= sh.sel << shift;
    mask |= 0xFFu << shift;
  }
  return prefix;
}

// Exact double-sum emulation: parallel sum + bound, sequential on ambiguity.
// vals(j) gives the j-th addend in index order, j < n; all addends >= 0.
template <int NT, typename Vals>
__device__ float InvOfSequentialSum(int n, Vals vals, Shared<NT>& sh, unsigned long long* fallbacks) {
  double part = 0.0;
  const int chunk = (n + NT - 1) / NT;
  const int b = threadIdx.x * chunk, e = min(n, b + chunk);
  for (int j = b; j < e; ++j) part += static_cast<double>(vals(j));
  const double S = BlockSumD(part, sh);
  const double B = 2.0 * static_cast<double>(n) * S * 0x1p-52;
  const float lo = static_cast<float>(1.0 / (S + B));
  const float hi = static_cast<float>(1.0 / (S - B));
  if (lo == hi && S - B > 0.0) return lo;
  BlockSync<NT>();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int j = 0; j < n; ++j) s += static_cast<double>(vals(j));
    sh.inv = static_cast<float>(1.0 / s);
    atomicAdd(fallbacks, 1ull);
  }
  BlockSync<NT>();
  return sh.inv;
}

// Steps 3-5 on the survivors: work[j] holds s of survivor j (index order,
// original index idx[j]); on return work[j] holds its final probability.
// Returns the chosen original index.
template <int NT>
__device__ int Finish(float* work, const int32_t* idx, int n_surv, const SamplerParamsDev& P, float u,
                      Shared<NT>& sh, unsigned long long* fallbacks) {
  const int tid = threadIdx.x;
  const int schunk = (n_surv + NT - 1) / NT;
  const int s0 = tid * schunk, s1 = min(n_surv, s0 + schunk);

  // ---- 3. softmax (masked entries are exactly 0 and add nothing)
  float mx = -__builtin_inff();
  for (int j = s0; j < s1; ++j) mx = fmaxf(mx, work[j]);
  mx = BlockMaxF(mx, sh);
  for (int j = s0; j < s1; ++j) work[j] = GlibcExpf(work[j] - mx);
  BlockSync<NT>();
  const float inv = InvOfSequentialSum(n_surv, [&](int j) { return work[j]; }, sh, fallbacks);
  for (int j = s0; j < s1; ++j) work[j] = work[j] * inv;
  BlockSync<NT>();

  // ---- 4. top-p
  if (P.top_p > 0.0f && P.top_p < 1.0f) {
    const double thr = 1.0 - static_cast<double>(P.top_p);
    const unsigned long long THR = static_cast<unsigned long long>(thr * 0x1p57);
    unsigned long long cum_below = 0;
    uint32_t prefix = 0, mask = 0;
    int all_zero = 0;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int b = tid; b < 256; b += NT) {
        sh.cnt[b] = 0;
        sh.mass[b] = 0;
      }
      BlockSync<NT>();
      for (int base = 0; base < n_surv; base += NT) {
        const int j = base + tid;
        bool act = false;
        uint32_t bin = 0;
        unsigned long long mj = 0;
        if (j < n_surv) {
          const float p = work[j];
          const uint32_t key = __float_as_uint(p);
          act = (key & mask) == prefix;
          bin = (key >> shift) & 255u;
          mj = static_cast<unsigned long long>(static_cast<double>(p) * 0x1p57);
        }
        AggAdd(sh.cnt, sh.mass, act, bin, mj);
      }
      BlockSync<NT>();
      // flag: every cumulative stays <= 1 - p
      if (tid < 64) SelectBinAsc(sh.mass, cum_below, THR, &sh.sel, &sh.u[0], &sh.flag);
      BlockSync<NT>();
      cum_below = sh.u[0];
      all_zero = sh.flag;
      prefix |= sh.sel << shift;
      mask |= 0xFFu << shift;
      if (all_zero) break;
    }
    if (all_zero) {
      // the reference zeroes all, keeps the largest, renormalises to 1.0
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
      BlockSync<NT>();
    } else {
      const float vstar = __uint_as_float(prefix);
      const unsigned long long V = static_cast<unsigned long long>(static_cast<double>(vstar) * 0x1p57);
      const unsigned long long room = THR - cum_below;
      const long long J = V > 0 ? static_cast<long long>(room / V) : 0;
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
      BlockSync<NT>();
      const float inv2 = InvOfSequentialSum(n_surv, [&](int j) { return work[j]; }, sh, fallbacks);
      for (int j = s0; j < s1; ++j) work[j] = work[j] * inv2;
      BlockSync<NT>();
    }
  }

  // ---- 5. inverse CDF: first j with cum > u; exact uint64 fixed point
  // (2^-52 units) when every nonzero p >= 2^-29
  int tiny = 0;
  for (int j = s0; j < s1; ++j) {
    const float p = work[j];
    tiny |= (p != 0.0f && p < 0x1p-29f) ? 1 : 0;
  }
  tiny = BlockOrI(tiny, sh);
  if (tid == 0) sh.answer = -1;
  BlockSync<NT>();
  if (!tiny) {
    unsigned long long mine = 0;
    for (int j = s0; j < s1; ++j) mine += static_cast<unsigned long long>(static_cast<double>(work[j]) * 0x1p52);
    const unsigned long long incl = lanes::WaveInclusiveAdd(mine);
    BlockSync<NT>();
    if ((tid & 63) == 63) sh.u[tid >> 6] = incl;
    BlockSync<NT>();
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
  BlockSync<NT>();
  int ans = sh.answer;
  if (ans < 0) {
    // ArgMax(probs) over the full vocabulary: the first maximum among
    // survivors, or index 0 when every probability is 0.
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
    if (m <= 0.0f) return 0;
    ans = cand;
  }
  return idx[ans];
}

template <int NT>
__device__ void WriteProbs(float* probs_out, int n, const float* work, const int32_t* idx, int n_surv) {
  for (int i = threadIdx.x; i < n; i += NT) probs_out[i] = 0.0f;
  __syncthreads();
  for (int j = threadIdx.x; j < n_surv; j += NT) probs_out[idx[j]] = work[j];
}

struct Ctx {
  const float* logits;
  int64_t ld;
  int n;
  const SamplerParamsDev* params;
  const int32_t* counter_dev;
  int64_t counter_host;
  int32_t* token_out;
  float* work;    // [rows][n]
  int32_t* idx;   // [rows][n]
  float* cand_v;  // [rows][n]
  int32_t* cand_i;
  int32_t* cand_cnt;  // [rows][slices]
  float* probs_out;
  unsigned long long* fallbacks;
};

__device__ __forceinline__ float ScaledLogit(const float* logits, int i, const SamplerParamsDev& P) {
  return P.temperature != 1.0f ? logits[i] * (1.0f / P.temperature) : logits[i];
}

// Top-k filtering runs in the two-stage form; k >= slice length is allowed
// (every logit of such a slice becomes a candidate).
__device__ __forceinline__ bool TopKMode(const SamplerParamsDev& P, int n) {
  return P.temperature > 0.0f && P.top_k > 1 && P.top_k < n;
}

// Stage 2 (and the whole job when there is no top-k): one 1024-thread
// workgroup per row; greedy rows take the first index of the maximum.
__global__ __launch_bounds__(kThreads) void SampleKernel(Ctx c, int n_slices) {
  __shared__ Shared<kThreads> sh;
  __shared__ Shared<64> sw;
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* logits = c.logits + row * c.ld;
  const int n = c.n;
  float* work = c.work + static_cast<int64_t>(row) * n;
  int32_t* idx = c.idx + static_cast<int64_t>(row) * n;
  const SamplerParamsDev P = c.params[row];
  const bool write_probs = c.probs_out != nullptr && row == 0;
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
    const int tok = (cand == 0x7fffffff || logits[0] != logits[0]) ? 0 : cand;
    if (tid == 0) c.token_out[row] = tok;
    if (write_probs)
      for (int i = tid; i < n; i += kThreads) c.probs_out[i] = (i == tok) ? 1.0f : 0.0f;
    return;
  }
  const uint64_t pos = c.counter_dev ? static_cast<uint64_t>(c.counter_dev[row]) : static_cast<uint64_t>(c.counter_host);
  const float u = CounterUniform(P.seed, pos);
  float* sv = work;
  int32_t* si = idx;
  int n_surv = n;
  if (TopKMode(P, n)) {
    // gather the candidates of every slice (slices in order, each in index
    // order): candidate j belongs to the slice whose inclusive count first
    // exceeds j
    const int my = tid < n_slices ? c.cand_cnt[row * n_slices + tid] : 0;
    int excl;
    const int nc = BlockExclusiveScan(my, &excl, sh);
    const float* cv = c.cand_v + static_cast<int64_t>(row) * n;
    const int32_t* ci = c.cand_i + static_cast<int64_t>(row) * n;
    for (int j = tid; j < nc; j += kThreads) {
      int lo = 0, hi = n_slices - 1;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sh.scan[mid] > j)
          hi = mid;
        else
          lo = mid + 1;
      }
      const int t = j - (lo > 0 ? sh.scan[lo - 1] : 0);
      work[j] = cv[lo * kSlice + t];
      idx[j] = ci[lo * kSlice + t];
    }
    __syncthreads();
    // global k-th over the candidates; survivors (s >= kth) compacted in
    // order into the candidate arrays, which are no longer read
    const float kth = FromOrderKey(RadixKth(nc, P.top_k, [&](int j) { return OrderKey(work[j]); }, sh));
    const int chunk = (nc + kThreads - 1) / kThreads;
    const int c0 = tid * chunk, c1 = min(nc, c0 + chunk);
    int keep = 0;
    for (int j = c0; j < c1; ++j) keep += work[j] >= kth ? 1 : 0;
    int dst;
    n_surv = BlockExclusiveScan(keep, &dst, sh);
    sv = c.cand_v + static_cast<int64_t>(row) * n;
    si = c.cand_i + static_cast<int64_t>(row) * n;
    for (int j = c0; j < c1; ++j) {
      if (work[j] >= kth) {
        sv[dst] = work[j];
        si[dst] = idx[j];
        ++dst;
      }
    }
  } else {
    for (int i = tid; i < n; i += kThreads) {
      work[i] = ScaledLogit(logits, i, P);
      idx[i] = i;
    }
  }
  __syncthreads();
  if (n_surv <= kWaveFinish) {
    // few survivors (the top-k case): one wave finishes, free of workgroup
    // barriers
    if (tid < 64) {
      const int tok = Finish<64>(sv, si, n_surv, P, u, sw, c.fallbacks);
      if (tid == 0) c.token_out[row] = tok;
    }
    __syncthreads();
  } else {
    const int tok = Finish<kThreads>(sv, si, n_surv, P, u, sh, c.fallbacks);
    if (tid == 0) c.token_out[row] = tok;
  }
  if (write_probs) WriteProbs<kThreads>(c.probs_out, n, sv, si, n_surv);
}

// Top-k, stage 1: grid (slices, rows). Local k-th largest of the slice, then
// the slice's candidates (s >= local k-th) in index order. Rows not in top-k
// mode return at once (the mode is read on the device, so one captured graph
// serves every parameter set).
__global__ __launch_bounds__(kSelThreads) void TopKSelectKernel(Ctx c) {
  __shared__ Shared<kSelThreads> sh;
  __shared__ uint32_t keys[kSlice];
  const int row = blockIdx.y, slice = blockIdx.x, tid = threadIdx.x;
  const SamplerParamsDev P = c.params[row];
  if (!TopKMode(P, c.n)) return;
  const float* logits = c.logits + row * c.ld;
  const int i0 = slice * kSlice, m = min(kSlice, c.n - i0);
  for (int t = tid; t < m; t += kSelThreads) keys[t] = OrderKey(ScaledLogit(logits, i0 + t, P));
  __syncthreads();
  const int k = P.top_k < m ? P.top_k : m;
  const uint32_t kth = RadixKth(m, k, [&](int i) { return keys[i]; }, sh);
  constexpr int per = kSlice / kSelThreads;  // contiguous elements per thread
  int my = 0;
  for (int t = tid * per; t < min(m, (tid + 1) * per); ++t) my += keys[t] >= kth ? 1 : 0;
  int base;
  const int total = BlockExclusiveScan(my, &base, sh);
  float* cv = c.cand_v + static_cast<int64_t>(row) * c.n + i0;
  int32_t* ci = c.cand_i + static_cast<int64_t>(row) * c.n + i0;
  for (int t = tid * per; t < min(m, (tid + 1) * per); ++t) {
    if (keys[t] >= kth) {
      cv[base] = FromOrderKey(keys[t]);
      ci[base] = i0 + t;
      ++base;
    }
  }
  if (tid == 0) c.cand_cnt[row * gridDim.x + slice] = total;
}

}  // namespace

Sampler::Sampler(int rows, int vocab) : rows_(rows), vocab_(vocab) {
  RPG_CHECK(vocab > 0 && CeilDiv(vocab, kSlice) <= kThreads, "sampler: vocab %d outside [1, %d]", vocab,
            kThreads * kSlice);
  const size_t n = static_cast<size_t>(rows) * vocab;
  HIP_CHECK(hipMalloc(&params_, sizeof(SamplerParamsDev) * rows));
  HIP_CHECK(hipMalloc(&work_, sizeof(float) * n));
  HIP_CHECK(hipMalloc(&idx_, sizeof(int32_t) * n));
  HIP_CHECK(hipMalloc(&cand_v_, sizeof(float) * n));
  HIP_CHECK(hipMalloc(&cand_i_, sizeof(int32_t) * n));
  HIP_CHECK(hipMalloc(&cand_cnt_, sizeof(int32_t) * static_cast<size_t>(rows) * CeilDiv(vocab, kSlice)));
  HIP_CHECK(hipMalloc(&fallbacks_, sizeof(unsigned long long)));
  HIP_CHECK(hipMemset(fallbacks_, 0, sizeof(unsigned long long)));
  HIP_CHECK(hipMemset(params_, 0, sizeof(SamplerParamsDev) * rows));
}

Sampler::~Sampler() {
  for (void* p : {static_cast<void*>(params_), static_cast<void*>(work_), static_cast<void*>(idx_),
                  static_cast<void*>(cand_v_), static_cast<void*>(cand_i_), static_cast<void*>(cand_cnt_),
                  static_cast<void*>(fallbacks_)})
    (void)hipFree(p);
}

void Sampler::SetParams(const SamplerParamsDev* p, int rows, hipStream_t s) {
  RPG_CHECK(rows <= rows_, "sampler: %d rows > capacity %d", rows, rows_);
  HIP_CHECK(hipMemcpyAsync(params_, p, sizeof(SamplerParamsDev) * rows, hipMemcpyHostToDevice, s));
}

void Sampler::Enqueue(const float* logits, int64_t ld, const int32_t* counter, int64_t counter_host, int32_t* token,
                      float* probs_out, hipStream_t s) {
  Ctx c{logits, ld, vocab_, params_, counter, counter_host, token, work_, idx_, cand_v_, cand_i_, cand_cnt_,
        probs_out, fallbacks_};
  const int n_slices = static_cast<int>(CeilDiv(vocab_, kSlice));
  hipLaunchKernelGGL(TopKSelectKernel, dim3(static_cast<unsigned>(n_slices), static_cast<unsigned>(rows_)),
                     dim3(kSelThreads), 0, s, c);
  hipLaunchKernelGGL(SampleKernel, dim3(static_cast<unsigned>(rows_)), dim3(kThreads), 0, s, c, n_slices);
  HIP_CHECK(hipGetLastError());
}

int64_t Sampler::FallbackCount(hipStream_t s) const {
  unsigned long long v = 0;
  HIP_CHECK(hipMemcpyAsync(&v, fallbacks_, sizeof(v), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  return static_cast<int64_t>(v);
}

}  // namespace rpg
