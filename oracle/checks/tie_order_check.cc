// Check of the model behind the GPU sampler's top-p tie order
// (rpgbarengine_amd/csrc/sampler.hip, TieOrder) against libstdc++ itself.
// Test infrastructure.
//
// The reference sorts the indices 0..n-1 of the softmax output ascending with
// std::sort (reference src/sampler.cc:72-76) and zeroes a prefix of that
// order. When equal probabilities straddle the cut, which of them are zeroed
// is the order libstdc++'s introsort leaves equal keys in. The model
// reproduces that order for one key value v* while partitioning only the
// ranges that hold v*:
//  * a partition of [f, l) (median of f+1, mid, l-1 moved to f, then the
//    unguarded Hoare scan of [f+1, l) against it) swaps the k-th position
//    holding a key >= P (ascending) with the k-th holding a key <= P
//    (descending) for every k with L[k] < R[k]; the scan stops at
//    min(L[K], R[K-1]) where K is the number of such pairs;
//  * ranges that hold no v* never move a v* element, so they are skipped;
//  * a range of at most 16 elements is left to the final insertion sort,
//    which is stable and never moves an element across a partition boundary,
//    so the v* elements keep their order of positions;
//  * a range whose depth budget (2 floor(log2 n)) runs out is heap-sorted
//    exactly as libstdc++'s partial_sort does.
// The GPU kernel computes the same partitions in parallel (prefix counts of
// the two stop sets); this program checks the model on random and structured
// inputs, including a forced small depth budget that exercises the heap path.
//
// Usage: tie_order_check [trials]   -- prints "ok N cases" or the first mismatch.

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

namespace {

struct Arr {
  std::vector<uint32_t> key;  // key at each position
  std::vector<int32_t> idx;   // original index at each position
  void Swap(int a, int b) {
    std::swap(key[a], key[b]);
    std::swap(idx[a], idx[b]);
  }
};

// libstdc++ __adjust_heap / __push_heap / __pop_heap / __make_heap /
// __sort_heap on [f, l), comparing keys with <.
void AdjustHeap(Arr& a, int f, int hole, int len, uint32_t vk, int32_t vi) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (a.key[f + second] < a.key[f + second - 1]) --second;
    a.key[f + hole] = a.key[f + second];
    a.idx[f + hole] = a.idx[f + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    a.key[f + hole] = a.key[f + second - 1];
    a.idx[f + hole] = a.idx[f + second - 1];
    hole = second - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && a.key[f + parent] < vk) {
    a.key[f + hole] = a.key[f + parent];
    a.idx[f + hole] = a.idx[f + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a.key[f + hole] = vk;
  a.idx[f + hole] = vi;
}

void HeapSort(Arr& a, int f, int l) {
  const int len = l - f;
  if (len >= 2) {
    for (int parent = (len - 2) / 2;; --parent) {
      AdjustHeap(a, f, parent, len, a.key[f + parent], a.idx[f + parent]);
      if (parent == 0) break;
    }
  }
  for (int last = l; last - f > 1;) {
    --last;
    const uint32_t vk = a.key[last];
    const int32_t vi = a.idx[last];
    a.key[last] = a.key[f];
    a.idx[last] = a.idx[f];
    AdjustHeap(a, f, 0, last - f, vk, vi);
  }
}

int Lg(int n) { return 31 - __builtin_clz(static_cast<unsigned>(n)); }

// The model: returns the original indices holding key v, in sorted order.
std::vector<int32_t> ModelTieOrder(const std::vector<uint32_t>& keys, uint32_t v, int depth0) {
  const int n = static_cast<int>(keys.size());
  Arr a;
  a.key = keys;
  a.idx.resize(n);
  for (int i = 0; i < n; ++i) a.idx[i] = i;
  struct R {
    int f, l, depth;
  };
  std::vector<R> stack;
  if (n > 16) stack.push_back({0, n, depth0});
  auto holds = [&](int f, int l) {
    for (int i = f; i < l; ++i)
      if (a.key[i] == v) return true;
    return false;
  };
  while (!stack.empty()) {
    R r = stack.back();
    stack.pop_back();
    int f = r.f, l = r.l, depth = r.depth;
    while (l - f > 16) {
      if (depth == 0) {
        HeapSort(a, f, l);
        break;
      }
      --depth;
      // median of three to f
      const int pa = f + 1, pb = f + (l - f) / 2, pc = l - 1;
      const uint32_t ka = a.key[pa], kb = a.key[pb], kc = a.key[pc];
      int m;
      if (ka < kb) {
        m = kb < kc ? pb : (ka < kc ? pc : pa);
      } else {
        m = ka < kc ? pa : (kb < kc ? pc : pb);
      }
      a.Swap(f, m);
      const uint32_t P = a.key[f];
      std::vector<int> L, Rv;
      for (int i = f + 1; i < l; ++i)
        if (a.key[i] >= P) L.push_back(i);
      for (int i = l - 1; i > f; --i)
        if (a.key[i] <= P) Rv.push_back(i);
      int K = 0;
      while (K < static_cast<int>(L.size()) && K < static_cast<int>(Rv.size()) && L[K] < Rv[K]) ++K;
      int cut;
      if (K == 0) {
        cut = L[0];
      } else {
        const int lk = K < static_cast<int>(L.size()) ? L[K] : 0x7fffffff;
        cut = std::min(lk, Rv[K - 1]);
      }
      for (int k = 0; k < K; ++k) a.Swap(L[k], Rv[k]);
      if (l - cut > 16 && holds(cut, l)) stack.push_back({cut, l, depth});
      if (!holds(f, cut)) break;
      l = cut;
    }
  }
  std::vector<int32_t> out;
  for (int i = 0; i < n; ++i)
    if (a.key[i] == v) out.push_back(a.idx[i]);
  return out;
}

// libstdc++'s answer: std::sort of the indices by key (reference
// comparator), or its internal loop with a chosen depth budget.
std::vector<int32_t> LibTieOrder(const std::vector<uint32_t>& keys, uint32_t v, int depth) {
  const int n = static_cast<int>(keys.size());
  std::vector<int32_t> asc(n);
  for (int i = 0; i < n; ++i) asc[i] = i;
  auto comp = [&](int32_t x, int32_t y) { return keys[x] < keys[y]; };
  if (depth < 0) {
    std::sort(asc.begin(), asc.end(), comp);
  } else if (n > 1) {
    std::__introsort_loop(asc.begin(), asc.end(), depth, __gnu_cxx::__ops::__iter_comp_iter(comp));
    std::__final_insertion_sort(asc.begin(), asc.end(), __gnu_cxx::__ops::__iter_comp_iter(comp));
  }
  std::vector<int32_t> out;
  for (int i = 0; i < n; ++i)
    if (keys[asc[i]] == v) out.push_back(asc[i]);
  return out;
}

std::vector<uint32_t> MakeKeys(std::mt19937_64& rng, int n, int kind) {
  std::vector<uint32_t> k(n);
  std::uniform_int_distribution<uint32_t> small(0, 7), mid(0, 200), big(0, 0x3F800000u);
  for (int i = 0; i < n; ++i) {
    switch (kind) {
      case 0: k[i] = small(rng); break;                            // few distinct values
      case 1: k[i] = mid(rng); break;                              // many ties
      case 2: k[i] = (i % 50 == 0) ? mid(rng) + 1 : 0; break;      // mostly zeros (top-k survivors)
      case 3: k[i] = static_cast<uint32_t>(i / 3); break;          // ascending runs of ties
      case 4: k[i] = static_cast<uint32_t>((n - i) / 4); break;    // descending runs
      case 5: k[i] = static_cast<uint32_t>(std::min(i, n - i) / 2); break;  // organ pipe
      case 6: k[i] = 5; break;                                     // all equal
      default: k[i] = big(rng) >> (i % 7 == 0 ? 20 : 0); break;    // wide values, some ties
    }
  }
  return k;
}

}  // namespace

int main(int argc, char** argv) {
  const int trials = argc > 1 ? std::atoi(argv[1]) : 300;
  std::mt19937_64 rng(20261202);
  const int sizes[] = {17, 18, 33, 64, 100, 257, 1000, 4096, 20000, 151936};
  long cases = 0;
  for (int t = 0; t < trials; ++t) {
    const int n = sizes[t % 10] + (t / 10 % 3);
    const int kind = t % 8;
    const std::vector<uint32_t> keys = MakeKeys(rng, n, kind);
    // a few tied values per array (most frequent first, then random ones)
    std::vector<uint32_t> vals;
    for (int j = 0; j < 3; ++j) vals.push_back(keys[rng() % n]);
    for (int forced = 0; forced < 2; ++forced) {
      const int depth = forced ? 1 + static_cast<int>(rng() % 4) : 2 * Lg(n);
      for (uint32_t v : vals) {
        const std::vector<int32_t> want = LibTieOrder(keys, v, forced ? depth : -1);
        const std::vector<int32_t> got = ModelTieOrder(keys, v, depth);
        ++cases;
        if (want != got) {
          std::printf("MISMATCH trial %d n %d kind %d value %u depth %d (forced %d): %zu vs %zu ties\n", t, n, kind,
                      v, depth, forced, got.size(), want.size());
          for (size_t i = 0; i < std::min<size_t>(want.size(), 12); ++i)
            std::printf("  %zu: model %d lib %d\n", i, i < got.size() ? got[i] : -1, want[i]);
          return 1;
        }
      }
    }
  }
  std::printf("ok %ld cases\n", cases);
  return 0;
}
