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
//                                             2^-57); when only some of the
//                                             ties at v* are zeroed, which ones
//                                             follows a replay of libstdc++'s
//                                             introsort (TieOrder); renormalise
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
// a sampled row of >= 16384 logits runs each pass over the whole vocabulary
// on one workgroup per slice and row, in a chain of launches (the
// full-vocabulary kernels below); smaller rows, and greedy rows, finish on
// one 1024-thread workgroup per row.
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
constexpr int kCandLds = 4096;     // top-k candidates the finishing workgroup holds in LDS

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

// Outcome of the top-p selection, shared by the finishing threads and the
// tie-order pass between them.
struct TopPCut {
  int32_t mode;  // 0: no top-p; 1: every cumulative stays <= 1 - p; 2: cut at vstar
  float vstar;   // probabilities below it are zeroed
  long long J;   // how many of the `ties` probabilities equal to vstar are zeroed too
  int32_t ties;
};

// Step 4a for at most 64 survivors on one wave (lane j holds survivor j):
// the radix selection's answer formed directly. vstar is the smallest value
// whose mass at or below it exceeds THR (the first ascending bin the radix
// passes would pick), cum_below the exact mass strictly below it -- that
// mass less the ties' (equal values have equal masses); no such value means
// every cumulative stays <= 1 - p.
__device__ __forceinline__ void TopPCutWave(const float* work, int n_surv, unsigned long long THR, Shared<64>& sh,
                                            TopPCut* cut) {
  const int lane = threadIdx.x & 63;
  const bool act = lane < n_surv;
  const float p = act ? work[lane] : 0.0f;
  const unsigned long long m = act ? static_cast<unsigned long long>(static_cast<double>(p) * 0x1p57) : 0ull;
  // every lane reads all (value, mass) pairs, four at a time, from LDS
  sh.cnt[lane] = __float_as_uint(p);
  sh.mass[lane] = m;
  BlockSync<64>();
  unsigned long long le = 0;  // mass at or below this lane's value
  for (int j = 0; j < n_surv; j += 4) {
    const uint4 pk = *reinterpret_cast<const uint4*>(&sh.cnt[j]);
    const ulonglong2 ma = *reinterpret_cast<const ulonglong2*>(&sh.mass[j]);
    const ulonglong2 mb = *reinterpret_cast<const ulonglong2*>(&sh.mass[j + 2]);
    const uint32_t pv[4] = {pk.x, pk.y, pk.z, pk.w};
    const unsigned long long mv[4] = {ma.x, ma.y, mb.x, mb.y};
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (j + q < n_surv) le += __uint_as_float(pv[q]) <= p ? mv[q] : 0ull;
  }
  const bool cross = act && le > THR;
  if (__ballot(cross) == 0) {
    if (lane == 0) cut->mode = 1;
    BlockSync<64>();
    return;
  }
  // non-negative floats order as their bits
  const uint32_t key = WaveReduce(cross ? __float_as_uint(p) : 0xFFFFFFFFu,
                                  [](uint32_t a, uint32_t b) { return a < b ? a : b; });
  const float vstar = __uint_as_float(key);
  const unsigned long long tb = __ballot(act && p == vstar);
  const int first = __ffsll(static_cast<long long>(tb)) - 1;
  const unsigned long long V = static_cast<unsigned long long>(static_cast<double>(vstar) * 0x1p57);
  const unsigned long long cum_below = lanes::ReadLaneT(le, first) - static_cast<unsigned long long>(__popcll(tb)) * V;
  if (lane == 0) {
    cut->mode = 2;
    cut->vstar = vstar;
    cut->J = V > 0 ? static_cast<long long>((THR - cum_below) / V) : 0;
    cut->ties = __popcll(tb);
  }
  BlockSync<64>();
}

// Steps 3-4a on the survivors: work[j] holds s of survivor j (index order);
// on return work[j] holds its softmax probability and *cut (written by
// thread 0) what top-p removes.
template <int NT>
__device__ void FinishHead(float* work, int n_surv, const SamplerParamsDev& P, Shared<NT>& sh,
                           unsigned long long* fallbacks, TopPCut* cut) {
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

  // ---- 4a. top-p: the value vstar where the ascending cumulative crosses
  // 1 - p, by radix selection over exact fixed-point mass
  if (!(P.top_p > 0.0f && P.top_p < 1.0f)) {
    if (tid == 0) cut->mode = 0;
    BlockSync<NT>();
    return;
  }
  const double thr = 1.0 - static_cast<double>(P.top_p);
  const unsigned long long THR = static_cast<unsigned long long>(thr * 0x1p57);
  if constexpr (NT == 64) {
    if (n_surv <= 64) {
      TopPCutWave(work, n_surv, THR, sh, cut);
      return;
    }
  }
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
    if (tid == 0) cut->mode = 1;
    BlockSync<NT>();
    return;
  }
  const float vstar = __uint_as_float(prefix);
  const unsigned long long V = static_cast<unsigned long long>(static_cast<double>(vstar) * 0x1p57);
  const unsigned long long room = THR - cum_below;
  int ties = 0;
  for (int j = s0; j < s1; ++j) ties += work[j] == vstar ? 1 : 0;
  int dummy;
  const int total_ties = BlockExclusiveScan(ties, &dummy, sh);
  if (tid == 0) {
    cut->mode = 2;
    cut->vstar = vstar;
    cut->J = V > 0 ? static_cast<long long>(room / V) : 0;
    cut->ties = total_ties;
  }
  BlockSync<NT>();
}

// Steps 4b-5: apply the cut (zero below vstar and the first J ties in index
// order -- J is 0 after TieOrder has zeroed the ties the reference's sort
// order puts first), renormalise, inverse CDF. Returns the chosen original
// index.
template <int NT>
__device__ int FinishTail(float* work, const int32_t* idx, int n_surv, const TopPCut& cut, float u, Shared<NT>& sh,
                          unsigned long long* fallbacks) {
  const int tid = threadIdx.x;
  const int schunk = (n_surv + NT - 1) / NT;
  const int s0 = tid * schunk, s1 = min(n_surv, s0 + schunk);
  if (cut.mode == 1) {
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
  } else if (cut.mode == 2) {
    const float vstar = cut.vstar;
    const long long J = cut.J;
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

// ---------------------------------------------------------------------------
// Top-p tie order. The reference sorts the indices 0..n-1 of the softmax
// output ascending with std::sort and zeroes a prefix of that order
// (reference src/sampler.cc:72-82). When equal probabilities vstar straddle
// the cut, which J of them are zeroed is the order libstdc++'s introsort
// (GCC 11 bits/stl_algo.h: __introsort_loop with depth budget 2 floor(log2
// n), median-of-three pivot moved to the front, unguarded Hoare partition,
// ranges of <= 16 left to a final insertion sort, heap sort when the budget
// runs out) leaves them in. TieOrder replays that sort on a copy of the
// keys, following only the ranges that hold vstar: a range without vstar
// never moves a vstar element, the final insertion sort is stable and never
// crosses a partition boundary, so after the partitions the vstar elements'
// order of positions is their sorted order.
//
// A partition of [f+1, l) against the pivot P at f is computed in parallel:
// with L the ascending positions of keys >= P and R the descending positions
// of keys <= P, the Hoare scan swaps L[k] with R[k] for k < K, where K is
// the number of k with L[k] < R[k] (= max over x of min(#L below x, #R at
// or above x)), and stops at min(L[K], R[K-1]) (L[0] when K = 0). Each wave
// ranks its tile of positions with ballots; one block scan joins the tiles.
// The model (the same partitions, sequentially) is checked against libstdc++
// itself by oracle/checks/tie_order_check.cc.
// ---------------------------------------------------------------------------

constexpr int kTieStack = 64;

struct TieShared {
  int32_t f[kTieStack], l[kTieStack], d[kTieStack];
  int32_t sp;
  int32_t cf, cl, cd;  // current range and its depth budget
  int32_t active, done, err;
  uint32_t pivot;
  int32_t cut;
  int32_t wl[16], wr[16];
};

// libstdc++ heap sort of positions [f, l) (partial_sort(f, l, l): make_heap,
// then sort_heap), by one thread. Only reached when a range exhausts its
// depth budget.
__device__ void TieAdjustHeap(uint32_t* key, int32_t* pos, int f, int hole, int len, uint32_t vk, int32_t vi) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (key[f + second] < key[f + second - 1]) --second;
    key[f + hole] = key[f + second];
    pos[f + hole] = pos[f + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    key[f + hole] = key[f + second - 1];
    pos[f + hole] = pos[f + second - 1];
    hole = second - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && key[f + parent] < vk) {
    key[f + hole] = key[f + parent];
    pos[f + hole] = pos[f + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  key[f + hole] = vk;
  pos[f + hole] = vi;
}

__device__ void TieHeapSort(uint32_t* key, int32_t* pos, int f, int l) {
  const int len = l - f;
  if (len >= 2) {
    for (int parent = (len - 2) / 2;; --parent) {
      TieAdjustHeap(key, pos, f, parent, len, key[f + parent], pos[f + parent]);
      if (parent == 0) break;
    }
  }
  for (int last = l; last - f > 1;) {
    --last;
    const uint32_t vk = key[last];
    const int32_t vi = pos[last];
    key[last] = key[f];
    pos[last] = pos[f];
    TieAdjustHeap(key, pos, f, 0, last - f, vk, vi);
  }
}

// Zeroes, in sv (survivor j at original index si[j], ascending; sv indexed by
// original index when si is null), the J entries equal to vstar that the
// reference's sort order puts first. n: vocabulary size (the reference sorts
// all of it, masked entries as probability 0). Scratch: key, pos, lbuf, rbuf
// of n entries. All NT threads call it. Returns false when the replay could
// not run (a guard tripped; the caller then keeps index order and counts it).
template <int NT>
__device__ bool TieOrder(float* sv, const int32_t* si, int n_surv, int n, float vstar, long long J, uint32_t* key,
                         int32_t* pos, int32_t* lbuf, int32_t* rbuf, TieShared& ts, Shared<NT>& sh) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t vbits = __float_as_uint(vstar);
  const unsigned long long below = (1ull << lane) - 1ull;
  if (si == nullptr) {
    for (int i = tid; i < n; i += NT) {
      key[i] = __float_as_uint(sv[i]);
      pos[i] = i;
    }
  } else {
    for (int i = tid; i < n; i += NT) {
      key[i] = 0u;
      pos[i] = i;
    }
    __syncthreads();
    for (int j = tid; j < n_surv; j += NT) key[si[j]] = __float_as_uint(sv[j]);
  }
  if (tid == 0) {
    ts.sp = 0;
    ts.err = 0;
    ts.done = 0;
    ts.active = 0;
    if (n > 16) {
      ts.f[0] = 0;
      ts.l[0] = n;
      ts.d[0] = 2 * (31 - __clz(n));
      ts.sp = 1;
    }
  }
  __syncthreads();
  for (;;) {
    if (tid == 0) {
      if (!ts.active || ts.cl - ts.cf <= 16) {
        if (ts.sp == 0 || ts.err) {
          ts.done = 1;
        } else {
          --ts.sp;
          ts.cf = ts.f[ts.sp];
          ts.cl = ts.l[ts.sp];
          ts.cd = ts.d[ts.sp];
          ts.active = 1;
        }
      }
      if (!ts.done && ts.cd > 0) {
        // median of (f+1, mid, l-1) to f
        const int f = ts.cf, l = ts.cl;
        const int pa = f + 1, pb = f + (l - f) / 2, pc = l - 1;
        const uint32_t ka = key[pa], kb = key[pb], kc = key[pc];
        int m;
        if (ka < kb)
          m = kb < kc ? pb : (ka < kc ? pc : pa);
        else
          m = ka < kc ? pa : (kb < kc ? pc : pb);
        const uint32_t tk = key[f];
        const int32_t tp = pos[f];
        key[f] = key[m];
        pos[f] = pos[m];
        key[m] = tk;
        pos[m] = tp;
        ts.pivot = key[f];
      }
    }
    __syncthreads();
    if (ts.done) break;
    const int f = ts.cf, l = ts.cl;
    if (ts.cd == 0) {
      if (tid == 0) {
        TieHeapSort(key, pos, f, l);
        ts.active = 0;
      }
      __syncthreads();
      continue;
    }
    const uint32_t P = ts.pivot;
    // pass 1: per-wave counts of the two stop sets over the wave's tile
    const int len = l - (f + 1);
    const int tile = ((len + NW - 1) / NW + 63) & ~63;
    const int t0 = f + 1 + w * tile, t1 = min(l, t0 + tile);
    int cl = 0, cr = 0;
    for (int b = t0; b < t1; b += 64) {
      const int i = b + lane;
      const bool in = i < t1;
      const uint32_t k = in ? key[i] : 0u;
      cl += __popcll(__ballot(in && k >= P));
      cr += __popcll(__ballot(in && k <= P));
    }
    if (lane == 0) {
      ts.wl[w] = cl;
      ts.wr[w] = cr;
    }
    __syncthreads();
    int baseL = 0, baseR = 0, totL = 0, totR = 0;
    for (int q = 0; q < NW; ++q) {
      baseL += q < w ? ts.wl[q] : 0;
      baseR += q < w ? ts.wr[q] : 0;
      totL += ts.wl[q];
      totR += ts.wr[q];
    }
    // pass 2: positions of the stops by rank; the number of swaps
    int runL = baseL, runR = baseR, best = 0;
    for (int b = t0; b < t1; b += 64) {
      const int i = b + lane;
      const bool in = i < t1;
      const uint32_t k = in ? key[i] : 0u;
      const bool isL = in && k >= P, isR = in && k <= P;
      const unsigned long long mL = __ballot(isL), mR = __ballot(isR);
      const int preL = runL + __popcll(mL & below), preR = runR + __popcll(mR & below);
      if (isL) lbuf[preL] = i;
      if (isR) rbuf[totR - 1 - preR] = i;
      if (in) best = max(best, min(preL, totR - preR));
      runL += __popcll(mL);
      runR += __popcll(mR);
    }
    // max over the block (values >= 0): block OR is not a max, use the
    // minimum of the negation
    const int K = -BlockMinI(-best, sh);
    __syncthreads();
    if (tid == 0) {
      if (totL == 0 || totR == 0) {
        ts.err = 1;  // no sentinel on one side: impossible after the median step
        ts.cut = f;
      } else if (K == 0) {
        ts.cut = lbuf[0];
      } else {
        const int lk = K < totL ? lbuf[K] : 0x7fffffff;
        ts.cut = min(lk, rbuf[K - 1]);
      }
    }
    // pass 3: the swaps (disjoint pairs)
    for (int k = tid; k < K; k += NT) {
      const int a = lbuf[k], c = rbuf[k];
      const uint32_t ka = key[a], kc = key[c];
      const int32_t pa = pos[a], pc = pos[c];
      key[a] = kc;
      pos[a] = pc;
      key[c] = ka;
      pos[c] = pa;
    }
    __syncthreads();
    if (ts.err) break;
    const int cut = ts.cut;
    // pass 4: which side still holds vstar
    int hl = 0, hr = 0;
    for (int i = f + tid; i < l; i += NT) {
      if (key[i] == vbits) {
        if (i < cut)
          hl = 1;
        else
          hr = 1;
      }
    }
    hl = BlockOrI(hl, sh);
    hr = BlockOrI(hr, sh);
    if (tid == 0) {
      const int dn = ts.cd - 1;
      if (hr && l - cut > 16) {
        if (ts.sp < kTieStack) {
          ts.f[ts.sp] = cut;
          ts.l[ts.sp] = l;
          ts.d[ts.sp] = dn;
          ++ts.sp;
        } else {
          ts.err = 1;
        }
      }
      if (hl) {
        ts.cl = cut;
        ts.cd = dn;
      } else {
        ts.active = 0;
      }
    }
    __syncthreads();
  }
  if (ts.err) return false;
  // the vstar entries in order of position: zero the first J
  const int tile = ((n + NW - 1) / NW + 63) & ~63;
  const int t0 = w * tile, t1 = min(n, t0 + tile);
  int cv = 0;
  for (int b = t0; b < t1; b += 64) {
    const int i = b + lane;
    cv += __popcll(__ballot(i < t1 && key[i] == vbits));
  }
  if (lane == 0) ts.wl[w] = cv;
  __syncthreads();
  int run = 0;
  for (int q = 0; q < w; ++q) run += ts.wl[q];
  for (int b = t0; b < t1; b += 64) {
    const int i = b + lane;
    const bool hit = i < t1 && key[i] == vbits;
    const unsigned long long mv = __ballot(hit);
    const int r = run + __popcll(mv & below);
    if (hit && r < J) {
      const int o = pos[i];
      if (si == nullptr) {
        sv[o] = 0.0f;
      } else {
        int lo = 0, hi = n_surv - 1;  // survivor slot of original index o
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (si[mid] < o)
            lo = mid + 1;
          else
            hi = mid;
        }
        sv[lo] = 0.0f;
      }
    }
    run += __popcll(mv);
  }
  __syncthreads();
  return true;
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
  unsigned long long* fallbacks;  // [0] sequential sums, [1] tie-order replays, [2] replays refused
  uint32_t* tie_key;              // [rows][n] scratch of the tie-order replay
  int32_t* tie_pos;
  int32_t* tie_l;
  int32_t* tie_r;
};

__device__ __forceinline__ float ScaledLogit(const float* logits, int i, const SamplerParamsDev& P) {
  return P.temperature != 1.0f ? logits[i] * (1.0f / P.temperature) : logits[i];
}

// Top-k filtering runs in the two-stage form; k >= slice length is allowed
// (every logit of such a slice becomes a candidate).
__device__ __forceinline__ bool TopKMode(const SamplerParamsDev& P, int n) {
  return P.temperature > 0.0f && P.top_k > 1 && P.top_k < n;
}

// Rows drawn by the full-vocabulary kernels below: sampled, no top-k filter, and a vocabulary
// whose per-row scratch fits (WideRowBytesA / B below).
__device__ __host__ __forceinline__ bool WideVocab(int n) { return n >= 16384; }
__device__ __forceinline__ bool WideMode(const SamplerParamsDev& P, int n) {
  return P.temperature > 0.0f && !TopKMode(P, n) && WideVocab(n);
}

// Stage 2 (and the whole job when there is no top-k): one 1024-thread
// workgroup per row; greedy rows take the first index of the maximum.
__global__ __launch_bounds__(kThreads) void SampleKernel(Ctx c, int n_slices, int wide) {
  __shared__ Shared<kThreads> sh;
  __shared__ Shared<64> sw;
  __shared__ float lv[kCandLds];
  __shared__ int32_t li[kCandLds];
  const int row = blockIdx.x, tid = threadIdx.x;
  // the slice counts of the top-k stage, requested with the parameters (the
  // buffer exists whatever the mode; only the top-k mode reads the values)
  const int my_cnt = tid < n_slices ? c.cand_cnt[row * n_slices + tid] : 0;
  const float* logits = c.logits + row * c.ld;
  const int n = c.n;
  float* work = c.work + static_cast<int64_t>(row) * n;
  int32_t* idx = c.idx + static_cast<int64_t>(row) * n;
  const SamplerParamsDev P = c.params[row];
  if (wide && WideMode(P, n)) return;  // drawn by the full-vocabulary kernels
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
    // exceeds j. Up to kCandLds of them stay in LDS for the selection and
    // the finish; more go through the row's global work arrays.
    int excl;
    const int nc = BlockExclusiveScan(my_cnt, &excl, sh);
    const float* cv = c.cand_v + static_cast<int64_t>(row) * n;
    const int32_t* ci = c.cand_i + static_cast<int64_t>(row) * n;
    const bool in_lds = nc <= kCandLds;
    float* gv = in_lds ? lv : work;
    int32_t* gi = in_lds ? li : idx;
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
      gv[j] = cv[lo * kSlice + t];
      gi[j] = ci[lo * kSlice + t];
    }
    __syncthreads();
    // global k-th over the candidates; survivors (s >= kth) compacted in
    // order: in place in LDS (each thread's chunk read before any is
    // written), else into the candidate arrays, which are no longer read
    const float kth = FromOrderKey(RadixKth(nc, P.top_k, [&](int j) { return OrderKey(gv[j]); }, sh));
    const int chunk = (nc + kThreads - 1) / kThreads;
    const int c0 = tid * chunk, c1 = min(nc, c0 + chunk);
    int keep = 0;
    for (int j = c0; j < c1; ++j) keep += gv[j] >= kth ? 1 : 0;
    int dst;
    n_surv = BlockExclusiveScan(keep, &dst, sh);
    if (in_lds) {
      constexpr int kPer = kCandLds / kThreads;
      float v[kPer];
      int32_t ix[kPer];
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int j = c0 + q;
        v[q] = j < c1 ? lv[j] : 0.0f;
        ix[q] = j < c1 ? li[j] : 0;
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        if (c0 + q < c1 && v[q] >= kth) {
          lv[dst] = v[q];
          li[dst] = ix[q];
          ++dst;
        }
      }
      sv = lv;
      si = li;
    } else {
      sv = c.cand_v + static_cast<int64_t>(row) * n;
      si = c.cand_i + static_cast<int64_t>(row) * n;
      for (int j = c0; j < c1; ++j) {
        if (work[j] >= kth) {
          sv[dst] = work[j];
          si[dst] = idx[j];
          ++dst;
        }
      }
    }
  } else {
    for (int i = tid; i < n; i += kThreads) {
      work[i] = ScaledLogit(logits, i, P);
      idx[i] = i;
    }
  }
  __syncthreads();
  // few survivors (the top-k case): one wave finishes, free of workgroup
  // barriers; the tie-order replay between the two halves takes them all
  const bool one_wave = n_surv <= kWaveFinish;
  __shared__ TopPCut cut;
  __shared__ TieShared ts;
  if (one_wave) {
    if (tid < 64) FinishHead<64>(sv, n_surv, P, sw, c.fallbacks, &cut);
  } else {
    FinishHead<kThreads>(sv, n_surv, P, sh, c.fallbacks, &cut);
  }
  __syncthreads();
  if (cut.mode == 2 && cut.J > 0 && cut.J < cut.ties) {
    // equal probabilities straddle the top-p cut: zero the ones the
    // reference's sort order puts first
    const int64_t o = static_cast<int64_t>(row) * n;
    const bool ok = TieOrder<kThreads>(sv, TopKMode(P, n) ? si : nullptr, n_surv, n, cut.vstar, cut.J,
                                       c.tie_key + o, c.tie_pos + o, c.tie_l + o, c.tie_r + o, ts, sh);
    if (tid == 0) {
      if (ok) cut.J = 0;  // done: the tail zeroes only what is below vstar
      atomicAdd(&c.fallbacks[ok ? 1 : 2], 1ull);
    }
    __syncthreads();
  }
  if (one_wave) {
    if (tid < 64) {
      const int tok = FinishTail<64>(sv, si, n_surv, cut, u, sw, c.fallbacks);
      if (tid == 0) c.token_out[row] = tok;
    }
    __syncthreads();
  } else {
    const int tok = FinishTail<kThreads>(sv, si, n_surv, cut, u, sh, c.fallbacks);
    if (tid == 0) c.token_out[row] = tok;
  }
  if (write_probs) WriteProbs<kThreads>(c.probs_out, n, sv, si, n_surv);
}

// ---------------------------------------------------------------------------
// The full-vocabulary draw (temperature > 0 without top-k) over many
// workgroups. Every pass over the vocabulary runs on one 256-thread
// workgroup per 4096-logit slice and row (thread t takes elements t, t + 256,
// ... of the slice); a launch boundary stands wherever a pass needs a
// whole-row result. A launch reads only what earlier launches wrote; a
// whole-row result that several of its workgroups need is recomputed by each
// of them from the per-slice partials in one fixed order, so all hold the
// same value:
//   scale    (inside the top-k selection launch) s = logit * (1/T), slice max
//   exp      e = expf(s - max), slice double sums
//   norm     inv = float(1 / sum) (bounded parallel sum, else sequential),
//            p = e * inv into a second buffer (a sequential fallback of
//            another workgroup may still read e); top-p radix pass 0 slice
//            histograms (count and exact 2^-57 fixed-point mass: order-free
//            integer sums)
//   radix    passes 1..3: the previous pass's selection from its summed
//            histograms (slice 0 records it for the next launch), then this
//            pass's histograms
//   cut      (one workgroup per row) the last selection: vstar and the tie
//            count J the reference zeroes; a tie set straddling the cut
//            replays the reference's sort (TieOrder), which zeroes its first J
//   apply    zero below vstar (and every tie when J covers them), slice sums
//            of what survives, slice maxima
//   renorm   inv2 as in norm, p2 = p * inv2 back into the first buffer
//            (one-hot at the first maximum when every cumulative stays
//            below 1 - top_p); per slice: any nonzero p2 < 2^-29, the 2^-52
//            fixed-point mass, the maximum
//   draw     (one workgroup per row) the slice where the exact fixed-point
//            cumulative first exceeds u, then the index inside it; the
//            sequential double walk when some p2 < 2^-29; ArgMax otherwise
// These are SampleKernel's steps (FinishHead, TieOrder, FinishTail) for a
// row whose survivors are the whole vocabulary, with the same arithmetic.
// ---------------------------------------------------------------------------

constexpr int kRadixPasses = 4;
constexpr int kPer = kSlice / kSelThreads;  // elements per thread of a slice

// Whole-row results that later launches read, each written by one workgroup.
struct WideState {
  int32_t mode;       // 0 no top-p, 1 every cumulative stays <= 1 - top_p, 2 cut at vstar
  float vstar;
  int32_t zero_ties;  // the entries equal to vstar are zeroed too
  int32_t pad;
  // after radix pass p's selection: the key prefix, its mask, the mass
  // below, whether no bin crossed (then every cumulative stays <= 1 - top_p)
  uint32_t prefix[kRadixPasses], mask[kRadixPasses];
  unsigned long long cum[kRadixPasses];
  int32_t all_zero[kRadixPasses];
  uint32_t cnt_sel[kRadixPasses];  // count in the selected bin
};

// Views of a row's scratch: small per-slice arrays in the row's cand_v
// region, the radix histograms in its cand_i region.
struct WideRow {
  WideState* st;
  float* smax;                // [S] slice max of s
  double* ssum;               // [S] slice sums of e
  double* ssum2;              // [S] slice sums of the cut p
  float* sv;                  // [S] slice max of p (for a one-hot cut)
  int32_t* si;                // [S] its first index
  float* sv2;                 // [S] slice max of p2 (for ArgMax)
  int32_t* si2;               // [S] its first index
  unsigned long long* smass;  // [S] slice 2^-52 fixed-point mass of p2
  int32_t* stiny;             // [S] a nonzero p2 < 2^-29 in the slice
  int32_t* sexp;              // [S] smallest exponent field of a nonzero e in the slice (255: none)
  int32_t* sexp2;             // [S] the same for the cut p
  uint32_t* hcnt;             // [pass][S][256]
  unsigned long long* hmass;  // [pass][S][256]
};

constexpr size_t kWideStateBytes = (sizeof(WideState) + 15) & ~static_cast<size_t>(15);

__device__ __forceinline__ WideRow WideView(const Ctx& c, int row, int S) {
  WideRow w;
  uint8_t* a = reinterpret_cast<uint8_t*>(c.cand_v + static_cast<int64_t>(row) * c.n);
  a = reinterpret_cast<uint8_t*>((reinterpret_cast<uintptr_t>(a) + 15) & ~static_cast<uintptr_t>(15));
  w.st = reinterpret_cast<WideState*>(a);
  a += kWideStateBytes;
  w.ssum = reinterpret_cast<double*>(a);
  a += 8 * S;
  w.ssum2 = reinterpret_cast<double*>(a);
  a += 8 * S;
  w.smass = reinterpret_cast<unsigned long long*>(a);
  a += 8 * S;
  w.smax = reinterpret_cast<float*>(a);
  a += 4 * S;
  w.sv = reinterpret_cast<float*>(a);
  a += 4 * S;
  w.si = reinterpret_cast<int32_t*>(a);
  a += 4 * S;
  w.stiny = reinterpret_cast<int32_t*>(a);
  a += 4 * S;
  w.sv2 = reinterpret_cast<float*>(a);
  a += 4 * S;
  w.si2 = reinterpret_cast<int32_t*>(a);
  a += 4 * S;
  w.sexp = reinterpret_cast<int32_t*>(a);
  a += 4 * S;
  w.sexp2 = reinterpret_cast<int32_t*>(a);
  uint8_t* b = reinterpret_cast<uint8_t*>(c.cand_i + static_cast<int64_t>(row) * c.n);
  b = reinterpret_cast<uint8_t*>((reinterpret_cast<uintptr_t>(b) + 15) & ~static_cast<uintptr_t>(15));
  w.hmass = reinterpret_cast<unsigned long long*>(b);
  w.hcnt = reinterpret_cast<uint32_t*>(b + static_cast<size_t>(8) * kRadixPasses * S * 256);
  return w;
}

// Bytes of each of the two regions a row needs (checked on the host).
__host__ __device__ constexpr size_t WideRowBytesA(int S) { return 16 + kWideStateBytes + 52 * static_cast<size_t>(S); }
__host__ __device__ constexpr size_t WideRowBytesB(int S) { return 16 + 12 * static_cast<size_t>(kRadixPasses) * S * 256; }

using WSh = Shared<kSelThreads>;

// The row's p buffer: the idx region, which this path does not use.
__device__ __forceinline__ float* WideP(const Ctx& c, int row) {
  return reinterpret_cast<float*>(c.idx + static_cast<int64_t>(row) * c.n);
}

// Element t of this thread in `slice` (t < kPer), or -1 past the vocabulary.
__device__ __forceinline__ int SliceElem(int slice, int t, int n) {
  const int i = slice * kSlice + t * kSelThreads + static_cast<int>(threadIdx.x);
  return i < n ? i : -1;
}

// scale: work = s, slice max
__device__ void WideScale(const Ctx& c, int row, int slice, WSh& sh) {
  const SamplerParamsDev P = c.params[row];
  const int n = c.n, S = gridDim.x;
  const WideRow w = WideView(c, row, S);
  const float* logits = c.logits + row * c.ld;
  float* work = c.work + static_cast<int64_t>(row) * n;
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? ScaledLogit(logits, i, P) : -__builtin_inff();
  }
  float mx = -__builtin_inff();
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    if (i >= 0) work[i] = v[t];
    mx = fmaxf(mx, v[t]);
  }
  mx = BlockMaxF(mx, sh);
  if (threadIdx.x == 0) w.smax[slice] = mx;
}

// The smallest exponent field among the block's nonzero values v[t] of
// elements in range (255 when there is none).
__device__ int BlockMinExp(const float (&v)[kPer], int slice, int n, WSh& sh) {
  int e = 255;
#pragma unroll
  for (int t = 0; t < kPer; ++t)
    if (SliceElem(slice, t, n) >= 0 && v[t] != 0.0f) e = min(e, static_cast<int>((__float_as_uint(v[t]) >> 23) & 255u));
  return BlockMinI(e, sh);
}

__global__ __launch_bounds__(kSelThreads) void WideExpKernel(Ctx c) {
  __shared__ WSh sh;
  const int row = blockIdx.y, slice = blockIdx.x, n = c.n, S = gridDim.x;
  if (!WideMode(c.params[row], n)) return;
  const WideRow w = WideView(c, row, S);
  float* work = c.work + static_cast<int64_t>(row) * n;
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? work[i] : 0.0f;
  }
  float mx = w.smax[0];
  for (int q = 1; q < S; ++q) mx = fmaxf(mx, w.smax[q]);
  double part = 0.0;
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? GlibcExpf(v[t] - mx) : 0.0f;
    if (i >= 0) {
      work[i] = v[t];
      part += static_cast<double>(v[t]);
    }
  }
  const double tot = BlockSumD(part, sh);
  const int me = BlockMinExp(v, slice, n, sh);
  if (threadIdx.x == 0) {
    w.ssum[slice] = tot;
    w.sexp[slice] = me;
  }
}

// The reference's sequential double sum of vals[0..n), by thread 0, the
// workgroup staging each 4096-value chunk in LDS (every thread calls it).
__device__ double SequentialSum(const float* vals, int n, float* buf) {
  double s = 0.0;
  for (int base = 0; base < n; base += kSlice) {
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
      const int j = base + t * kSelThreads + static_cast<int>(threadIdx.x);
      buf[t * kSelThreads + threadIdx.x] = j < n ? vals[j] : 0.0f;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      const int m = min(kSlice, n - base);
      const float4* b4 = reinterpret_cast<const float4*>(buf);
      int j = 0;
      for (; j + 4 <= m; j += 4) {
        const float4 q = b4[j >> 2];
        s += static_cast<double>(q.x);
        s += static_cast<double>(q.y);
        s += static_cast<double>(q.z);
        s += static_cast<double>(q.w);
      }
      for (; j < m; ++j) s += static_cast<double>(buf[j]);
    }
  }
  return s;
}

// float(1 / sum) of the row's values as the reference's sequential double
// sum gives it: the bounded parallel sum from the slice sums when it
// decides, else the sequential sum (every workgroup of the launch computes
// it; slice 0 counts it).
__device__ float WideInv(const double* ssum, const int32_t* sexp, int S, const float* vals, int n, int slice, WSh& sh,
                         unsigned long long* fallbacks) {
  __shared__ float buf[kSlice];
  double T = 0.0;
  int E = 255;
  for (int q = 0; q < S; ++q) {
    T += ssum[q];
    E = min(E, sexp[q]);
  }
  // Every value is a multiple of the quantum 2^(E - 150) (2^-149 for a
  // subnormal, E = 0): when the total stays below 2^53 quanta every partial
  // sum, in any order, is exact in double, so the parallel sum is the
  // sequential one (tested against 2^52 quanta: T itself may carry rounding
  // when the condition fails).
  if (E < 255 && T < __builtin_ldexp(1.0, (E == 0 ? 1 : E) - 150 + 52)) return static_cast<float>(1.0 / T);
  const double B = 2.0 * static_cast<double>(n) * T * 0x1p-52;
  const float lo = static_cast<float>(1.0 / (T + B));
  const float hi = static_cast<float>(1.0 / (T - B));
  if (lo == hi && T - B > 0.0) return lo;
  const double s = SequentialSum(vals, n, buf);
  if (threadIdx.x == 0) {
    sh.inv = static_cast<float>(1.0 / s);
    if (slice == 0) atomicAdd(fallbacks, 1ull);
  }
  __syncthreads();
  return sh.inv;
}

__device__ __forceinline__ bool TopPActive(const SamplerParamsDev& P) { return P.top_p > 0.0f && P.top_p < 1.0f; }
__device__ __forceinline__ unsigned long long TopPThreshold(const SamplerParamsDev& P) {
  return static_cast<unsigned long long>((1.0 - static_cast<double>(P.top_p)) * 0x1p57);
}

// This slice's histogram of radix pass `pass` over p[] (values held by the
// thread, v[t] for element t) with keys matching (prefix, mask): count and
// 2^-57 fixed-point mass per 8-bit bin.
__device__ void WideHistogram(const WideRow& w, const float (&v)[kPer], int n, int slice, int S, int pass,
                              uint32_t prefix, uint32_t mask, WSh& sh) {
  const int shift = 24 - 8 * pass;
  for (int b = threadIdx.x; b < 256; b += kSelThreads) {
    sh.cnt[b] = 0;
    sh.mass[b] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    const uint32_t key = __float_as_uint(v[t]);
    const bool act = i >= 0 && (key & mask) == prefix;
    const unsigned long long mj = act ? static_cast<unsigned long long>(static_cast<double>(v[t]) * 0x1p57) : 0ull;
    AggAdd(sh.cnt, sh.mass, act, (key >> shift) & 255u, mj);
  }
  __syncthreads();
  const size_t o = (static_cast<size_t>(pass) * S + slice) * 256;
  for (int b = threadIdx.x; b < 256; b += kSelThreads) {
    w.hcnt[o + b] = sh.cnt[b];
    w.hmass[o + b] = sh.mass[b];
  }
}

// Radix pass `pass`'s selection, as FinishHead's pass makes it, from its
// slice histograms (summed over the slices: exact) and the state after the
// previous pass (in: prefix, mask, cum). Every thread returns the new state;
// the return value is the "no bin crosses" flag.
template <int NT>
__device__ int WideSelect(const WideRow& w, int S, int pass, unsigned long long THR, uint32_t* prefix, uint32_t* mask,
                          unsigned long long* cum, uint32_t* cnt_sel, Shared<NT>& sh) {
  const int shift = 24 - 8 * pass;
  for (int b = threadIdx.x; b < 256; b += NT) {
    uint32_t cs = 0;
    unsigned long long ms = 0;
    for (int q = 0; q < S; ++q) {
      const size_t o = (static_cast<size_t>(pass) * S + q) * 256 + b;
      cs += w.hcnt[o];
      ms += w.hmass[o];
    }
    sh.cnt[b] = cs;
    sh.mass[b] = ms;
  }
  __syncthreads();
  if (threadIdx.x < 64) SelectBinAsc(sh.mass, *cum, THR, &sh.sel, &sh.u[0], &sh.flag);
  __syncthreads();
  const int all_zero = sh.flag;
  *cum = sh.u[0];
  *prefix |= sh.sel << shift;
  *mask |= 0xFFu << shift;
  *cnt_sel = sh.cnt[sh.sel];
  __syncthreads();
  return all_zero;
}

// The state after pass `pass` (-1: none yet), from the record an earlier
// launch wrote. Returns false when an earlier pass found no crossing.
__device__ __forceinline__ bool WideStateAfter(const WideRow& w, int pass, uint32_t* prefix, uint32_t* mask,
                                               unsigned long long* cum) {
  if (pass < 0) {
    *prefix = 0;
    *mask = 0;
    *cum = 0;
    return true;
  }
  if (w.st->all_zero[pass]) return false;
  *prefix = w.st->prefix[pass];
  *mask = w.st->mask[pass];
  *cum = w.st->cum[pass];
  return true;
}

// norm: inv, p, radix pass 0
__global__ __launch_bounds__(kSelThreads) void WideNormKernel(Ctx c) {
  __shared__ WSh sh;
  const int row = blockIdx.y, slice = blockIdx.x, n = c.n, S = gridDim.x;
  const SamplerParamsDev P = c.params[row];
  if (!WideMode(P, n)) return;
  const WideRow w = WideView(c, row, S);
  const float* work = c.work + static_cast<int64_t>(row) * n;
  float* pb = WideP(c, row);
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? work[i] : 0.0f;
  }
  const float inv = WideInv(w.ssum, w.sexp, S, work, n, slice, sh, c.fallbacks);
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = v[t] * inv;
    if (i >= 0) pb[i] = v[t];
  }
  if (!TopPActive(P)) return;
  WideHistogram(w, v, n, slice, S, 0, 0u, 0u, sh);
}

// radix pass `pass` (1..3): the previous pass's selection, then this pass's
// histograms
__global__ __launch_bounds__(kSelThreads) void WideRadixKernel(Ctx c, int pass) {
  __shared__ WSh sh;
  const int row = blockIdx.y, slice = blockIdx.x, n = c.n, S = gridDim.x;
  const SamplerParamsDev P = c.params[row];
  if (!WideMode(P, n) || !TopPActive(P)) return;
  const WideRow w = WideView(c, row, S);
  const float* pb = WideP(c, row);
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? pb[i] : 0.0f;
  }
  uint32_t prefix, mask, cnt;
  unsigned long long cum;
  if (!WideStateAfter(w, pass - 2, &prefix, &mask, &cum)) {
    if (slice == 0 && threadIdx.x == 0) w.st->all_zero[pass - 1] = 1;  // carried to the later passes
    return;
  }
  const int all_zero = WideSelect(w, S, pass - 1, TopPThreshold(P), &prefix, &mask, &cum, &cnt, sh);
  if (slice == 0 && threadIdx.x == 0) {
    w.st->prefix[pass - 1] = prefix;
    w.st->mask[pass - 1] = mask;
    w.st->cum[pass - 1] = cum;
    w.st->all_zero[pass - 1] = all_zero;
    w.st->cnt_sel[pass - 1] = cnt;
  }
  if (all_zero) return;
  WideHistogram(w, v, n, slice, S, pass, prefix, mask, sh);
}

// cut: one 1024-thread workgroup per row
__global__ __launch_bounds__(kThreads) void WideCutKernel(Ctx c) {
  __shared__ Shared<kThreads> sh;
  __shared__ TieShared ts;
  const int row = blockIdx.x, n = c.n, S = (n + kSlice - 1) / kSlice;
  const SamplerParamsDev P = c.params[row];
  if (!WideMode(P, n)) return;
  const WideRow w = WideView(c, row, S);
  if (!TopPActive(P)) {
    if (threadIdx.x == 0) w.st->mode = 0;
    return;
  }
  const unsigned long long THR = TopPThreshold(P);
  uint32_t prefix, mask, ties;
  unsigned long long cum;
  if (!WideStateAfter(w, kRadixPasses - 2, &prefix, &mask, &cum) ||
      WideSelect(w, S, kRadixPasses - 1, THR, &prefix, &mask, &cum, &ties, sh)) {
    if (threadIdx.x == 0) w.st->mode = 1;
    return;
  }
  const float vstar = __uint_as_float(prefix);
  const unsigned long long V = static_cast<unsigned long long>(static_cast<double>(vstar) * 0x1p57);
  const long long J = V > 0 ? static_cast<long long>((THR - cum) / V) : 0;
  int zero_ties = J >= static_cast<long long>(ties) && J > 0;
  if (J > 0 && J < static_cast<long long>(ties)) {
    // equal probabilities straddle the cut: zero the ones the reference's
    // sort order puts first; the rest of the ties stay
    const int64_t o = static_cast<int64_t>(row) * n;
    float* pb = WideP(c, row);
    const bool ok = TieOrder<kThreads>(pb, nullptr, n, n, vstar, J, c.tie_key + o, c.tie_pos + o, c.tie_l + o,
                                       c.tie_r + o, ts, sh);
    if (!ok) {
      // (never expected) the first J ties in index order, as FinishTail does
      const int chunk = (n + kThreads - 1) / kThreads;
      const int s0 = threadIdx.x * chunk, s1 = min(n, s0 + chunk);
      int mine = 0;
      for (int j = s0; j < s1; ++j) mine += pb[j] == vstar ? 1 : 0;
      int r;
      (void)BlockExclusiveScan(mine, &r, sh);
      for (int j = s0; j < s1; ++j) {
        if (pb[j] == vstar) {
          if (r < J) pb[j] = 0.0f;
          ++r;
        }
      }
    }
    if (threadIdx.x == 0) atomicAdd(&c.fallbacks[ok ? 1 : 2], 1ull);
    zero_ties = 0;
  }
  if (threadIdx.x == 0) {
    w.st->mode = 2;
    w.st->vstar = vstar;
    w.st->zero_ties = zero_ties;
  }
}

// The block's maximum of v (elements of `slice`) and its first index.
__device__ void SliceArgMax(const float (&v)[kPer], int slice, int n, WSh& sh, float* mv, int* mi) {
  float bv = -1.0f;
  int bi = 0x7fffffff;
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    if (i >= 0 && v[t] > bv) {
      bv = v[t];
      bi = i;
    }
  }
  const float m = BlockMaxF(bv, sh);
  const int cand = BlockMinI(bv == m ? bi : 0x7fffffff, sh);
  *mv = m;
  *mi = cand;
}

// apply: the cut, sums of what survives, slice maxima
__global__ __launch_bounds__(kSelThreads) void WideApplyKernel(Ctx c) {
  __shared__ WSh sh;
  const int row = blockIdx.y, slice = blockIdx.x, n = c.n, S = gridDim.x;
  const SamplerParamsDev P = c.params[row];
  if (!WideMode(P, n)) return;
  const WideRow w = WideView(c, row, S);
  const int mode = TopPActive(P) ? w.st->mode : 0;
  if (mode == 0) return;
  float* pb = WideP(c, row);
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? pb[i] : 0.0f;
  }
  if (mode == 2) {
    const float vstar = w.st->vstar;
    const bool zt = w.st->zero_ties != 0;
    double part = 0.0;
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
      const int i = SliceElem(slice, t, n);
      const float q = (v[t] < vstar || (v[t] == vstar && zt)) ? 0.0f : v[t];
      if (i >= 0) {
        pb[i] = q;
        part += static_cast<double>(q);
      }
    }
    const double tot = BlockSumD(part, sh);
#pragma unroll
    for (int t = 0; t < kPer; ++t) v[t] = (v[t] < vstar || (v[t] == vstar && zt)) ? 0.0f : v[t];
    const int me = BlockMinExp(v, slice, n, sh);
    if (threadIdx.x == 0) {
      w.ssum2[slice] = tot;
      w.sexp2[slice] = me;
    }
  } else {
    float mv;
    int mi;
    SliceArgMax(v, slice, n, sh, &mv, &mi);
    if (threadIdx.x == 0) {
      w.sv[slice] = mv;
      w.si[slice] = mi;
    }
  }
}

// renorm: p2 and the draw's per-slice statistics
__global__ __launch_bounds__(kSelThreads) void WideRenormKernel(Ctx c) {
  __shared__ WSh sh;
  const int row = blockIdx.y, slice = blockIdx.x, n = c.n, S = gridDim.x;
  const SamplerParamsDev P = c.params[row];
  if (!WideMode(P, n)) return;
  const WideRow w = WideView(c, row, S);
  const int mode = TopPActive(P) ? w.st->mode : 0;
  const float* pb = WideP(c, row);
  float* work = c.work + static_cast<int64_t>(row) * n;
  float v[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    v[t] = i >= 0 ? pb[i] : 0.0f;
  }
  if (mode == 2) {
    const float inv2 = WideInv(w.ssum2, w.sexp2, S, pb, n, slice, sh, c.fallbacks);
#pragma unroll
    for (int t = 0; t < kPer; ++t) v[t] = v[t] * inv2;
  } else if (mode == 1) {
    // the reference zeroes all, keeps the largest, renormalises to 1.0
    float bv = -1.0f;
    int bi = 0x7fffffff;
    for (int q = 0; q < S; ++q) {
      if (w.sv[q] > bv) {
        bv = w.sv[q];
        bi = w.si[q];
      }
    }
#pragma unroll
    for (int t = 0; t < kPer; ++t) v[t] = SliceElem(slice, t, n) == bi ? 1.0f : 0.0f;
  }
  int tiny = 0;
  unsigned long long mass = 0;
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int i = SliceElem(slice, t, n);
    if (i >= 0) {
      work[i] = v[t];
      tiny |= (v[t] != 0.0f && v[t] < 0x1p-29f) ? 1 : 0;
      mass += static_cast<unsigned long long>(static_cast<double>(v[t]) * 0x1p52);
      if (c.probs_out != nullptr && row == 0) c.probs_out[i] = v[t];
    }
  }
  tiny = BlockOrI(tiny, sh);
  mass = WaveReduce(mass, [](unsigned long long x, unsigned long long y) { return x + y; });
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.u[threadIdx.x >> 6] = mass;
  __syncthreads();
  float mv;
  int mi;
  SliceArgMax(v, slice, n, sh, &mv, &mi);
  if (threadIdx.x == 0) {
    unsigned long long tot = 0;
    for (int q = 0; q < WSh::kW; ++q) tot += sh.u[q];
    w.smass[slice] = tot;
    w.stiny[slice] = tiny;
    w.sv2[slice] = mv;
    w.si2[slice] = mi;
  }
}

// draw: one workgroup per row
__global__ __launch_bounds__(kSelThreads) void WideDrawKernel(Ctx c) {
  __shared__ WSh sh;
  const int row = blockIdx.x, n = c.n, S = (n + kSlice - 1) / kSlice;
  const SamplerParamsDev P = c.params[row];
  if (!WideMode(P, n)) return;
  const WideRow w = WideView(c, row, S);
  const float* work = c.work + static_cast<int64_t>(row) * n;
  const uint64_t pos = c.counter_dev ? static_cast<uint64_t>(c.counter_dev[row]) : static_cast<uint64_t>(c.counter_host);
  const float u = CounterUniform(P.seed, pos);
  int tiny = 0;
  for (int q = 0; q < S; ++q) tiny |= w.stiny[q];
  int ans = -1;
  if (!tiny) {
    // exact: every partial sum is a multiple of 2^-52 below 2
    const unsigned long long U = static_cast<unsigned long long>(static_cast<double>(u) * 0x1p52);
    unsigned long long cum = 0;
    int hit = -1;
    for (int q = 0; q < S; ++q) {
      if (cum + w.smass[q] > U) {
        hit = q;
        break;
      }
      cum += w.smass[q];
    }
    if (hit >= 0) {
      // the slice in index order: thread t takes elements kPer t .. kPer t + kPer
      const int i0 = hit * kSlice, m = min(kSlice, n - i0);
      const int b = i0 + min(m, static_cast<int>(threadIdx.x) * kPer);
      const int e = i0 + min(m, (static_cast<int>(threadIdx.x) + 1) * kPer);
      unsigned long long mine = 0;
      for (int i = b; i < e; ++i) mine += static_cast<unsigned long long>(static_cast<double>(work[i]) * 0x1p52);
      const unsigned long long incl = lanes::WaveInclusiveAdd(mine);
      __syncthreads();
      if ((threadIdx.x & 63) == 63) sh.u[threadIdx.x >> 6] = incl;
      __syncthreads();
      unsigned long long run = cum;
      for (int q = 0; q < static_cast<int>(threadIdx.x >> 6); ++q) run += sh.u[q];
      run += incl - mine;
      int found = 0x7fffffff;
      for (int i = b; i < e; ++i) {
        run += static_cast<unsigned long long>(static_cast<double>(work[i]) * 0x1p52);
        if (run > U) {
          found = i;
          break;
        }
      }
      found = BlockMinI(found, sh);
      if (found != 0x7fffffff) ans = found;
    }
  } else {
    __shared__ float buf[kSlice];
    // the reference's sequential double walk; chunks staged in LDS
    int found = -1;
    double cum = 0.0;
    for (int base = 0; base < n && found < 0; base += kSlice) {
      __syncthreads();
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const int j = base + t * kSelThreads + static_cast<int>(threadIdx.x);
        buf[t * kSelThreads + threadIdx.x] = j < n ? work[j] : 0.0f;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        const int m = min(kSlice, n - base);
        int a = -1;
        for (int j = 0; j < m; ++j) {
          cum += static_cast<double>(buf[j]);
          if (cum > static_cast<double>(u)) {
            a = base + j;
            break;
          }
        }
        sh.answer = a;
      }
      __syncthreads();
      found = sh.answer;
    }
    if (threadIdx.x == 0) atomicAdd(c.fallbacks, 1ull);
    ans = found;
  }
  if (ans < 0) {
    // ArgMax(probs): the first maximum, or index 0 when every probability is 0
    float bv = -1.0f;
    int bi = 0x7fffffff;
    for (int q = 0; q < S; ++q) {
      if (w.sv2[q] > bv) {
        bv = w.sv2[q];
        bi = w.si2[q];
      }
    }
    ans = bv <= 0.0f ? 0 : bi;
  }
  if (threadIdx.x == 0) c.token_out[row] = ans;
}

// Top-k, stage 1: grid (slices, rows). A threshold no larger than the
// slice's k-th largest value, then the slice's candidates (s >= threshold)
// in index order. Thread t holds the slice's elements 16 t .. 16 t + 15,
// loaded all at once. For k <= 256 the threshold is the k-th largest of the
// 256 per-thread maxima (by rank counting in LDS, one barrier each side):
// those are k distinct elements at or above it, so
// it cannot exceed the slice's k-th largest (nor, the slice being part of
// the row, the row's k-th largest), and every survivor of the row's top-k
// is a candidate; the candidates number about k (a thread rarely holds two
// of the slice's top k). Larger k selects the slice's exact k-th value.
// Stage 2 finds the row's exact k-th value over all candidates either way.
// Rows not in top-k mode return at once (the mode is read on the device,
// so one captured graph serves every parameter set).
__global__ __launch_bounds__(kSelThreads) void TopKSelectKernel(Ctx c, int wide) {
  __shared__ Shared<kSelThreads> sh;
  __shared__ uint32_t keys[kSlice];
  const int row = blockIdx.y, slice = blockIdx.x, tid = threadIdx.x;
  const float* logits = c.logits + row * c.ld;
  const int i0 = slice * kSlice, m = min(kSlice, c.n - i0);
  constexpr int per = kSlice / kSelThreads;  // contiguous elements per thread
  const int e0 = tid * per;
  // every load issued before any is used, the slice's logits with the
  // parameters (one round trip; indices clamped into the slice, the
  // elements past it masked below)
  float v[per];
#pragma unroll
  for (int e = 0; e < per; ++e) v[e] = logits[i0 + min(e0 + e, m - 1)];
  const SamplerParamsDev P = c.params[row];
  if (!TopKMode(P, c.n)) {
    if (wide && WideMode(P, c.n)) WideScale(c, row, slice, sh);
    return;
  }
  uint32_t key[per];
  uint32_t tmax = 0u;  // below every key of a real value
#pragma unroll
  for (int e = 0; e < per; ++e) {
    key[e] = OrderKey(P.temperature != 1.0f ? v[e] * (1.0f / P.temperature) : v[e]);
    if (e0 + e < m) tmax = key[e] > tmax ? key[e] : tmax;
  }
  uint32_t kth;
  if (P.top_k <= kSelThreads) {
    // the k-th largest of the 256 maxima (counting duplicates): the value
    // with fewer than k maxima above it and at least k at or above it,
    // found by each thread ranking its own maximum against all of them
    keys[tid] = tmax;
    __syncthreads();
    const uint4* k4 = reinterpret_cast<const uint4*>(keys);
    int gt = 0, ge = 0;
#pragma unroll 8
    for (int j = 0; j < kSelThreads / 4; ++j) {
      const uint4 q = k4[j];
      gt += (q.x > tmax) + (q.y > tmax) + (q.z > tmax) + (q.w > tmax);
      ge += (q.x >= tmax) + (q.y >= tmax) + (q.z >= tmax) + (q.w >= tmax);
    }
    if (gt < P.top_k && ge >= P.top_k) sh.sel = tmax;  // the threads that write agree on the value
    __syncthreads();
    kth = sh.sel;
  } else {
#pragma unroll
    for (int e = 0; e < per; ++e)
      if (e0 + e < m) keys[e0 + e] = key[e];
    __syncthreads();
    kth = RadixKth(m, P.top_k < m ? P.top_k : m, [&](int i) { return keys[i]; }, sh);
  }
  int my = 0;
#pragma unroll
  for (int e = 0; e < per; ++e) my += (e0 + e < m && key[e] >= kth) ? 1 : 0;
  int base;
  const int total = BlockExclusiveScan(my, &base, sh);
  float* cv = c.cand_v + static_cast<int64_t>(row) * c.n + i0;
  int32_t* ci = c.cand_i + static_cast<int64_t>(row) * c.n + i0;
#pragma unroll
  for (int e = 0; e < per; ++e) {
    if (e0 + e < m && key[e] >= kth) {
      cv[base] = FromOrderKey(key[e]);
      ci[base] = i0 + e0 + e;
      ++base;
    }
  }
  if (tid == 0) c.cand_cnt[row * gridDim.x + slice] = total;
}

}  // namespace

size_t Sampler::ScratchBytes(int rows, int vocab) {
  auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  const size_t n = static_cast<size_t>(rows) * vocab;
  return up(sizeof(SamplerParamsDev) * rows) + 8 * up(4 * n) +
         up(sizeof(int32_t) * static_cast<size_t>(rows) * CeilDiv(vocab, kSlice)) + up(3 * sizeof(unsigned long long));
}

// Buffers in the order ScratchBytes counts them, each 256-byte aligned.
void Sampler::Carve(char* base, size_t bytes) {
  RPG_CHECK(vocab_ > 0 && CeilDiv(vocab_, kSlice) <= kThreads, "sampler: vocab %d outside [1, %d]", vocab_,
            kThreads * kSlice);
  RPG_CHECK(bytes >= ScratchBytes(rows_, vocab_), "sampler: %zu scratch bytes, %zu needed", bytes,
            ScratchBytes(rows_, vocab_));
  auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  const size_t n = static_cast<size_t>(rows_) * vocab_;
  char* p = base;
  auto take = [&](size_t b) {
    char* q = p;
    p += up(b);
    return q;
  };
  params_ = reinterpret_cast<SamplerParamsDev*>(take(sizeof(SamplerParamsDev) * rows_));
  work_ = reinterpret_cast<float*>(take(4 * n));
  idx_ = reinterpret_cast<int32_t*>(take(4 * n));
  cand_v_ = reinterpret_cast<float*>(take(4 * n));
  cand_i_ = reinterpret_cast<int32_t*>(take(4 * n));
  tie_key_ = reinterpret_cast<uint32_t*>(take(4 * n));
  tie_pos_ = reinterpret_cast<int32_t*>(take(4 * n));
  tie_l_ = reinterpret_cast<int32_t*>(take(4 * n));
  tie_r_ = reinterpret_cast<int32_t*>(take(4 * n));
  cand_cnt_ = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(rows_) * CeilDiv(vocab_, kSlice)));
  fallbacks_ = reinterpret_cast<unsigned long long*>(take(3 * sizeof(unsigned long long)));
}

Sampler::Sampler(int rows, int vocab) : rows_(rows), vocab_(vocab) {
  RPG_CHECK(vocab > 0 && CeilDiv(vocab, kSlice) <= kThreads, "sampler: vocab %d outside [1, %d]", vocab,
            kThreads * kSlice);
  const size_t bytes = ScratchBytes(rows, vocab);
  void* base = nullptr;
  DeviceAlloc(&base, bytes);
  try {
    Carve(static_cast<char*>(base), bytes);  // params_ is the base: the destructor frees it
    HIP_CHECK(hipMemset(fallbacks_, 0, 3 * sizeof(unsigned long long)));
    HIP_CHECK(hipMemset(params_, 0, sizeof(SamplerParamsDev) * rows));
  } catch (...) {
    (void)hipFree(base);
    throw;
  }
}

Sampler::Sampler(int rows, int vocab, void* external, size_t external_bytes)
    : rows_(rows), vocab_(vocab), owns_(false) {
  RPG_CHECK(external != nullptr && (reinterpret_cast<uintptr_t>(external) & 255) == 0,
            "sampler: external scratch must be 256-byte aligned device memory");
  Carve(static_cast<char*>(external), external_bytes);
}

Sampler::~Sampler() {
  if (owns_) (void)hipFree(params_);  // the base of the one allocation
}

// A row the full-vocabulary kernels draw (WideMode, from host values).
bool Sampler::RowIsWide(const SamplerParamsDev& p) const {
  return p.temperature > 0.0f && !(p.top_k > 1 && p.top_k < vocab_) && WideVocab(vocab_);
}

void Sampler::SetParams(const SamplerParamsDev* p, int rows, hipStream_t s) {
  RPG_CHECK(rows <= rows_, "sampler: %d rows > capacity %d", rows, rows_);
  wide_ = false;
  for (int r = 0; r < rows; ++r) wide_ = wide_ || RowIsWide(p[r]);
  HIP_CHECK(hipMemcpyAsync(params_, p, sizeof(SamplerParamsDev) * rows, hipMemcpyHostToDevice, s));
}

void Sampler::Enqueue(const float* logits, int64_t ld, const int32_t* counter, int64_t counter_host, int32_t* token,
                      float* probs_out, hipStream_t s) {
  Ctx c{logits, ld, vocab_, params_, counter, counter_host, token, work_, idx_, cand_v_, cand_i_, cand_cnt_,
        probs_out, fallbacks_, tie_key_, tie_pos_, tie_l_, tie_r_};
  const int n_slices = static_cast<int>(CeilDiv(vocab_, kSlice));
  const int wide = wide_ && WideVocab(vocab_) ? 1 : 0;
  // a row's scratch: the small arrays in its cand_v slot, the histograms in
  // its cand_i slot (each 4 * vocab bytes, 4-byte aligned)
  RPG_CHECK(!wide || (WideRowBytesA(n_slices) + 16 <= 4 * static_cast<size_t>(vocab_) &&
                      WideRowBytesB(n_slices) + 16 <= 4 * static_cast<size_t>(vocab_)),
            "sampler: vocabulary %d too small for the full-vocabulary kernels", vocab_);
  const dim3 grid(static_cast<unsigned>(n_slices), static_cast<unsigned>(rows_));
  hipLaunchKernelGGL(TopKSelectKernel, grid, dim3(kSelThreads), 0, s, c, wide);
  if (wide) {
    hipLaunchKernelGGL(WideExpKernel, grid, dim3(kSelThreads), 0, s, c);
    hipLaunchKernelGGL(WideNormKernel, grid, dim3(kSelThreads), 0, s, c);
    for (int pass = 1; pass < kRadixPasses; ++pass)
      hipLaunchKernelGGL(WideRadixKernel, grid, dim3(kSelThreads), 0, s, c, pass);
    hipLaunchKernelGGL(WideCutKernel, dim3(static_cast<unsigned>(rows_)), dim3(kThreads), 0, s, c);
    hipLaunchKernelGGL(WideApplyKernel, grid, dim3(kSelThreads), 0, s, c);
    hipLaunchKernelGGL(WideRenormKernel, grid, dim3(kSelThreads), 0, s, c);
    hipLaunchKernelGGL(WideDrawKernel, dim3(static_cast<unsigned>(rows_)), dim3(kSelThreads), 0, s, c);
  }
  hipLaunchKernelGGL(SampleKernel, dim3(static_cast<unsigned>(rows_)), dim3(kThreads), 0, s, c, n_slices, wide);
  HIP_CHECK(hipGetLastError());
}

namespace {
__global__ void SetParamsKernel(SamplerParamsDev* params, SamplerParamsDev p, unsigned long long* counters) {
  params[0] = p;
  counters[0] = 0ull;
  counters[1] = 0ull;
  counters[2] = 0ull;
}
}  // namespace

void Sampler::SetParamsByKernel(const SamplerParamsDev& p, hipStream_t s) {
  wide_ = RowIsWide(p);
  hipLaunchKernelGGL(SetParamsKernel, dim3(1), dim3(1), 0, s, params_, p, fallbacks_);
  HIP_CHECK(hipGetLastError());
}

int64_t Sampler::FallbackCount(hipStream_t s, int which) const {
  RPG_CHECK(which >= 0 && which < 3, "sampler: no counter %d", which);
  unsigned long long v = 0;
  HIP_CHECK(hipMemcpyAsync(&v, fallbacks_ + which, sizeof(v), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  return static_cast<int64_t>(v);
}

}  // namespace rpg
