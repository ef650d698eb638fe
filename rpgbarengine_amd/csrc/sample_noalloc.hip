// rpg_hip_sample_noalloc (include/rpg_hip.h): rpg_hip_sample on caller-owned
// device buffers, with the sampler's scratch in a static device array
// instead of an allocation, for callers that cannot call hipMalloc (code
// under HIP graph capture, serving loops).
//
// The array `scratch` exists once per GPU for the life of the process. In
// host code its name is only a stand-in for the device variable: its device
// address on the current GPU comes from hipGetSymbolAddress, looked up once
// per device on the first call there, and only that address is ever passed
// to kernels. Every call on one GPU shares the array, so calls that overlap
// on one GPU (different streams, or different host threads) race; calls
// ordered on one stream do not. Whatever must start at zero (the slow-path
// counters) is cleared by the first kernel of every call.

#include <hip/hip_runtime.h>

#include <mutex>

#include "common.h"
#include "rpg_hip.h"
#include "sampler.h"

namespace rpg {
namespace {

constexpr int kNoAllocMaxVocab = 1 << 18;  // logits per call
// Sampler::ScratchBytes(1, kNoAllocMaxVocab) = 8 arrays of 4 bytes per
// logit + parameters, slice counts and counters (each 256-byte aligned):
// 8 MiB + 1 KiB; 4 KiB of slack.
constexpr size_t kScratchBytes = (static_cast<size_t>(32) << 18) + 4096;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current GPU.
void* ScratchOnCurrentDevice() {
  int dev = -1;
  HIP_CHECK(hipGetDevice(&dev));
  RPG_CHECK(dev >= 0 && dev < kMaxDevices, "sample_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    RPG_CHECK(p != nullptr, "sample_noalloc: no device address for the scratch array on device %d", dev);
    g_scratch_dev[dev] = p;
  }
  return g_scratch_dev[dev];
}

}  // namespace
}  // namespace rpg

extern "C" int32_t rpg_hip_sample_noalloc(const float* logits_dev, int32_t n, float temperature, int32_t top_k,
                                          float top_p, uint64_t seed, int64_t counter, int32_t* token_dev,
                                          float* probs_dev, void* stream) {
  try {
    rpg::SetLastError("");
    RPG_CHECK(n > 0 && n <= rpg::kNoAllocMaxVocab,
              "sample_noalloc: %d logits outside [1, %d] (the size of its static scratch)", n,
              rpg::kNoAllocMaxVocab);
    RPG_CHECK(logits_dev != nullptr && token_dev != nullptr, "sample_noalloc: null logits or token buffer");
    static_assert(rpg::kScratchBytes >= 8 * 4 * static_cast<size_t>(rpg::kNoAllocMaxVocab) + 1024,
                  "scratch smaller than the sampler's buffers");
    RPG_CHECK(rpg::Sampler::ScratchBytes(1, n) <= rpg::kScratchBytes, "sample_noalloc: scratch too small for %d",
              n);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    rpg::Sampler sm(1, n, rpg::ScratchOnCurrentDevice(), rpg::kScratchBytes);
    sm.SetParamsByKernel(rpg::SamplerParamsDev{temperature, top_k, top_p, 0, seed}, s);
    sm.Enqueue(logits_dev, n, nullptr, counter, token_dev, probs_dev, s);
    return 0;
  } catch (const std::exception& e) {
    rpg::SetLastError(e.what());
    return -1;
  }
}
