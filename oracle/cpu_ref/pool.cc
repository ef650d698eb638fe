// Persistent row-partitioned thread pool -- restates the contract of reference
// src/threads.cc:118-234: equal chunks of ceil(n / threads), the caller runs
// chunk 0, results do not depend on the thread count (parallelism is over
// independent output rows only).

#include <algorithm>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <thread>

#include "oracle.h"

namespace orc {

struct Pool::Impl {
  int n = 1;
  std::vector<std::thread> workers;
  std::mutex mu;
  std::condition_variable start, done;
  uint64_t generation = 0;
  std::vector<int64_t> begin, end;
  const std::function<void(int64_t, int64_t)>* body = nullptr;
  int pending = 0;
  bool stop = false;
};

namespace {
thread_local bool t_in_worker = false;
}

Pool::Pool(int n_threads) : impl_(new Impl) {
  Impl& p = *impl_;
  p.n = std::max(1, n_threads);
  p.begin.assign(p.n, 0);
  p.end.assign(p.n, 0);
  for (int i = 1; i < p.n; ++i) {
    p.workers.emplace_back([this, i]() {
      Impl& q = *impl_;
      t_in_worker = true;
      uint64_t seen = 0;
      for (;;) {
        int64_t b, e;
        const std::function<void(int64_t, int64_t)>* fn;
        {
          std::unique_lock<std::mutex> lk(q.mu);
          q.start.wait(lk, [&] { return q.stop || q.generation != seen; });
          if (q.stop) return;
          seen = q.generation;
          b = q.begin[i];
          e = q.end[i];
          fn = q.body;
        }
        if (b < e && fn) (*fn)(b, e);
        std::lock_guard<std::mutex> lk(q.mu);
        if (--q.pending == 0) q.done.notify_all();
      }
    });
  }
}

Pool::~Pool() {
  {
    std::lock_guard<std::mutex> lk(impl_->mu);
    impl_->stop = true;
  }
  impl_->start.notify_all();
  for (auto& t : impl_->workers) t.join();
}

int Pool::size() const { return impl_->n; }

void Pool::ParallelForRange(int64_t n, const std::function<void(int64_t, int64_t)>& body) {
  if (n <= 0) return;
  Impl& p = *impl_;
  if (p.n <= 1 || t_in_worker) {
    body(0, n);
    return;
  }
  const int64_t chunk = (n + p.n - 1) / p.n;
  {
    std::lock_guard<std::mutex> lk(p.mu);
    p.body = &body;
    p.pending = p.n - 1;
    for (int i = 0; i < p.n; ++i) {
      p.begin[i] = std::min<int64_t>(n, chunk * i);
      p.end[i] = std::min<int64_t>(n, chunk * (i + 1));
    }
    ++p.generation;
  }
  p.start.notify_all();
  if (p.begin[0] < p.end[0]) body(p.begin[0], p.end[0]);
  std::unique_lock<std::mutex> lk(p.mu);
  p.done.wait(lk, [&] { return p.pending == 0; });
  p.body = nullptr;
}

// Distinct (physical id, core id) pairs of /proc/cpuinfo (reference
// src/threads.cc:70-123); falls back to the hardware thread count.
int PhysicalCores() {
  std::FILE* f = std::fopen("/proc/cpuinfo", "r");
  std::set<std::pair<int, int>> cores;
  if (f) {
    char line[512];
    int phys = -1, core = -1;
    auto flush = [&]() {
      if (phys >= 0 && core >= 0) cores.emplace(phys, core);
      phys = core = -1;
    };
    while (std::fgets(line, sizeof(line), f)) {
      const char* colon = std::strchr(line, ':');
      if (std::strncmp(line, "physical id", 11) == 0 && colon) phys = std::atoi(colon + 1);
      else if (std::strncmp(line, "core id", 7) == 0 && colon) core = std::atoi(colon + 1);
      else if (line[0] == '\n') flush();
    }
    flush();
    std::fclose(f);
  }
  if (!cores.empty()) return static_cast<int>(cores.size());
  const unsigned hw = std::thread::hardware_concurrency();
  return hw ? static_cast<int>(std::min(hw, 1024u)) : 1;
}

}  // namespace orc
