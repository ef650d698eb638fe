#include "common.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>

namespace rpg {

namespace {
thread_local std::string t_last_error;

int LogThreshold() {
  static const int level = [] {
    const char* v = std::getenv("RPGBAR_ENGINE_LOG");  // same knob as reference src/common.cc:30-84
    if (!v || !*v) return static_cast<int>(kLogWarn);
    const std::string s(v);
    if (s == "error") return static_cast<int>(kLogError);
    if (s == "warn") return static_cast<int>(kLogWarn);
    if (s == "info") return static_cast<int>(kLogInfo);
    if (s == "debug") return static_cast<int>(kLogDebug);
    return std::atoi(v);
  }();
  return level;
}
}  // namespace

void Throw(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Error(buf);
}

namespace {
// allocations left before an injected failure; negative = injection off
std::atomic<int64_t> g_alloc_countdown{-1};
}  // namespace

void FailDeviceAllocAfter(int64_t n) { g_alloc_countdown.store(n < 0 ? -1 : n); }

void DeviceAlloc(void** p, size_t bytes) {
  *p = nullptr;
  int64_t left = g_alloc_countdown.load();
  while (left >= 0 && !g_alloc_countdown.compare_exchange_weak(left, left - 1)) {
  }
  if (left == 0) {
    g_alloc_countdown.store(-1);  // one failure per arming
    Throw("HIP error hipErrorOutOfMemory (%d) allocating %zu bytes (injected allocation failure)",
          static_cast<int>(hipErrorOutOfMemory), bytes);
  }
  HIP_CHECK(hipMalloc(p, bytes));
}

void SetLastError(const std::string& msg) { t_last_error = msg; }
const char* LastError() { return t_last_error.c_str(); }

void Log(int level, const char* fmt, ...) {
  if (level > LogThreshold()) return;
  static std::mutex mu;
  static const char* names[] = {"error", "warn", "info", "debug"};
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  std::lock_guard<std::mutex> lk(mu);
  std::fprintf(stderr, "[rpg_engine_hip %s] %s\n", names[level < 0 ? 0 : (level > 3 ? 3 : level)], buf);
}

// Block geometry of every ggml type the reference reads (reference
// src/quant.cc:29-45).
int64_t BlockElems(uint32_t type) {
  switch (type) {
    case kF32: case kF16: case kBF16: return 1;
    case kQ4_0: case kQ4_1: case kQ5_0: case kQ5_1: case kQ8_0: case kQ8_1: return 32;
    case kQ2_K: case kQ3_K: case kQ4_K: case kQ5_K: case kQ6_K: case kQ8_K: return 256;
    default: return -1;
  }
}

int64_t BlockBytes(uint32_t type) {
  switch (type) {
    case kF32: return 4;
    case kF16: case kBF16: return 2;
    case kQ4_0: return 18;
    case kQ4_1: return 20;
    case kQ5_0: return 22;
    case kQ5_1: return 24;
    case kQ8_0: return 34;
    case kQ8_1: return 36;
    case kQ2_K: return 84;
    case kQ3_K: return 110;
    case kQ4_K: return 144;
    case kQ5_K: return 176;
    case kQ6_K: return 210;
    case kQ8_K: return 292;
    default: return -1;
  }
}

int64_t RowBytes(uint32_t type, int64_t n) {
  const int64_t be = BlockElems(type);
  RPG_CHECK(be > 0, "ggml type %u is not supported by the GPU engine", type);
  RPG_CHECK(n % be == 0, "%lld elements is not a multiple of the %s block (%lld)", (long long)n,
            TypeName(type), (long long)be);
  return n / be * BlockBytes(type);
}

const char* TypeName(uint32_t type) {
  switch (type) {
    case kF32: return "F32";
    case kF16: return "F16";
    case kBF16: return "BF16";
    case kQ4_0: return "Q4_0";
    case kQ4_1: return "Q4_1";
    case kQ5_0: return "Q5_0";
    case kQ5_1: return "Q5_1";
    case kQ8_0: return "Q8_0";
    case kQ8_1: return "Q8_1";
    case kQ2_K: return "Q2_K";
    case kQ3_K: return "Q3_K";
    case kQ4_K: return "Q4_K";
    case kQ5_K: return "Q5_K";
    case kQ6_K: return "Q6_K";
    case kQ8_K: return "Q8_K";
    default: return "unsupported";
  }
}

}  // namespace rpg
