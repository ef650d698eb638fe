// Shared host-side plumbing: errors, HIP checks, logging.
//
// Error contract (mirrors reference src/common.h:28-62 and src/engine.cc:175-191):
// internal code throws rpg::Error; every extern "C" entry point catches, stores
// the message in a thread-local last-error slot and returns -1 / NULL.

#ifndef RPG_HIP_COMMON_H_
#define RPG_HIP_COMMON_H_

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace rpg {

class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

[[noreturn]] void Throw(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

void SetLastError(const std::string& msg);
const char* LastError();

enum LogLevel { kLogError = 0, kLogWarn = 1, kLogInfo = 2, kLogDebug = 3 };
void Log(int level, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define RPG_CHECK(cond, ...)              \
  do {                                    \
    if (!(cond)) ::rpg::Throw(__VA_ARGS__); \
  } while (0)

#define HIP_CHECK(expr)                                                            \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      ::rpg::Throw("HIP error %s (%d) at %s:%d: %s", hipGetErrorName(e_), (int)e_, \
                   __FILE__, __LINE__, #expr);                                     \
  } while (0)

// Device allocation of every session, batch, sampler and model buffer. Throws
// like HIP_CHECK(hipMalloc(...)) on failure, so callers follow the error
// contract above. An allocation that fails leaves *p == nullptr.
void DeviceAlloc(void** p, size_t bytes);
template <typename T>
inline void DeviceAlloc(T** p, size_t bytes) {
  void* v = nullptr;
  try {
    DeviceAlloc(&v, bytes);
  } catch (...) {
    *p = nullptr;
    throw;
  }
  *p = static_cast<T*>(v);
}
// Failure injection for tests of the out-of-memory contract: after `n` more
// successful DeviceAlloc calls (process-wide), the next one throws the error
// a failed hipMalloc gives, without calling it; n < 0 switches injection off.
void FailDeviceAllocAfter(int64_t n);

// ggml type ids (reference src/quant.h:22-38)
enum GgmlType : uint32_t {
  kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ8_1 = 9, kQ2_K = 10, kQ3_K = 11,
  kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kQ8_K = 15, kBF16 = 30,
};

// True for the types with dedicated kernels (F32, Q8_0, Q4_K, Q6_K); the
// others run on the generic per-unit dequant kernels.
inline bool FastType(uint32_t t) { return t == kF32 || t == kQ8_0 || t == kQ4_K || t == kQ6_K; }

int64_t BlockElems(uint32_t type);  // -1 when unsupported
int64_t BlockBytes(uint32_t type);
int64_t RowBytes(uint32_t type, int64_t n);  // throws when n is not a block multiple
const char* TypeName(uint32_t type);

inline int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace rpg

#endif  // RPG_HIP_COMMON_H_
