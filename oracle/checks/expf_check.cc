// Exhaustive check: rpg::GlibcExpf (rpgbarengine_amd/csrc/expf_glibc.h) against
// the host's glibc expf over every float bit pattern in [lo, hi). Prints the
// number of mismatching inputs and the first few. Test infrastructure.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>
#include <atomic>

#include "../../rpgbarengine_amd/csrc/expf_glibc.h"

int main(int argc, char** argv) {
  const uint64_t lo = argc > 1 ? std::strtoull(argv[1], nullptr, 0) : 0;
  const uint64_t hi = argc > 2 ? std::strtoull(argv[2], nullptr, 0) : (1ull << 32);
  const int nt = argc > 3 ? std::atoi(argv[3]) : 8;
  std::atomic<uint64_t> bad{0};
  std::vector<std::thread> th;
  for (int t = 0; t < nt; ++t) {
    th.emplace_back([&, t]() {
      uint64_t local = 0;
      for (uint64_t u = lo + t; u < hi; u += nt) {
        const uint32_t b = static_cast<uint32_t>(u);
        float x;
        std::memcpy(&x, &b, 4);
        const float a = std::exp(x);
        const float c = rpg::GlibcExpf(x);
        uint32_t ba, bc;
        std::memcpy(&ba, &a, 4);
        std::memcpy(&bc, &c, 4);
        if (ba != bc && !(std::isnan(a) && std::isnan(c))) {
          if (local < 3) std::printf("mismatch x=%a (0x%08x): glibc %a ours %a\n", x, b, a, c);
          ++local;
        }
      }
      bad += local;
    });
  }
  for (auto& x : th) x.join();
  std::printf("range [0x%llx, 0x%llx): %llu mismatches\n", (unsigned long long)lo, (unsigned long long)hi,
              (unsigned long long)bad.load());
  return bad.load() == 0 ? 0 : 1;
}
