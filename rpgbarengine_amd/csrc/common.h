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

// ggml type ids (reference src/quant.h)
enum GgmlType : uint32_t {
  kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kBF16 = 30,
};

int64_t BlockElems(uint32_t type);  // -1 when unsupported
int64_t BlockBytes(uint32_t type);
int64_t RowBytes(uint32_t type, int64_t n);  // throws when n is not a block multiple
const char* TypeName(uint32_t type);

inline int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace rpg

#endif  // RPG_HIP_COMMON_H_
