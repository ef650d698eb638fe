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

// Outcome of the top-p selection, shared by the finishing threads and the
// tie-order pass between them.
struct TopPCut {
  int32_t mode;  // 0: no top-p; 1: every cumulative stays <= 1 - p; 2: cut at vstar
  float vstar;   // probabilities below it are zeroed
  long long J;   // how many of the `ties` probabilities equal to vstar are zeroed too
  int32_t ties;
};

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
  HIP_CHECK(hipMalloc(&base, bytes));
  Carve(static_cast<char*>(base), bytes);
  HIP_CHECK(hipMemset(fallbacks_, 0, 3 * sizeof(unsigned long long)));
  HIP_CHECK(hipMemset(params_, 0, sizeof(SamplerParamsDev) * rows));
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

void Sampler::SetParams(const SamplerParamsDev* p, int rows, hipStream_t s) {
  RPG_CHECK(rows <= rows_, "sampler: %d rows > capacity %d", rows, rows_);
  HIP_CHECK(hipMemcpyAsync(params_, p, sizeof(SamplerParamsDev) * rows, hipMemcpyHostToDevice, s));
}

void Sampler::Enqueue(const float* logits, int64_t ld, const int32_t* counter, int64_t counter_host, int32_t* token,
                      float* probs_out, hipStream_t s) {
  Ctx c{logits, ld, vocab_, params_, counter, counter_host, token, work_, idx_, cand_v_, cand_i_, cand_cnt_,
        probs_out, fallbacks_, tie_key_, tie_pos_, tie_l_, tie_r_};
  const int n_slices = static_cast<int>(CeilDiv(vocab_, kSlice));
  hipLaunchKernelGGL(TopKSelectKernel, dim3(static_cast<unsigned>(n_slices), static_cast<unsigned>(rows_)),
                     dim3(kSelThreads), 0, s, c);
  hipLaunchKernelGGL(SampleKernel, dim3(static_cast<unsigned>(rows_)), dim3(kThreads), 0, s, c, n_slices);
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
