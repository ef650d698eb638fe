// On-GPU sampling that reproduces the reference sampler exactly for the same
// logits, options and (seed, position) (reference src/sampler.cc:16-112).
//
// With top-k, two launches per draw: a per-slice top-k candidate selection
// over the whole grid, then one 1024-thread workgroup per logits row (a batch
// of sessions samples in one launch). Without top-k, the passes over the whole
// vocabulary run on one workgroup per 4096-logit slice and row, in a chain of
// launches (sampler.hip). Parameters, including which filters apply, are read
// in device memory, so a captured decode graph keeps working when the caller
// changes temperature / top-k / seed between calls.

#ifndef RPG_HIP_SAMPLER_H_
#define RPG_HIP_SAMPLER_H_

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rpg {

struct SamplerParamsDev {
  float temperature;
  int32_t top_k;
  float top_p;
  int32_t pad;
  uint64_t seed;
};

class Sampler {
 public:
  // rows: logits rows sampled per launch; vocab: row length.
  Sampler(int rows, int vocab);
  // Same, with every device buffer carved from `external` (device memory of
  // at least ScratchBytes(rows, vocab) bytes, 256-byte aligned, owned by the
  // caller): the constructor and destructor allocate and free nothing.
  Sampler(int rows, int vocab, void* external, size_t external_bytes);
  ~Sampler();
  // Device bytes the buffers of a (rows, vocab) sampler take.
  static size_t ScratchBytes(int rows, int vocab);
  Sampler(const Sampler&) = delete;
  Sampler& operator=(const Sampler&) = delete;

  // Host -> device copy of the per-row parameters (enqueued on s).
  void SetParams(const SamplerParamsDev* params_host, int rows, hipStream_t s);
  // The parameters of row 0 written by a one-thread kernel, which also
  // clears the slow-path counters: no host memory is read after the call
  // returns, and no memset node is recorded when the caller captures s.
  void SetParamsByKernel(const SamplerParamsDev& p, hipStream_t s);

  // token[r] = SampleToken(logits[r], params[r], u = CounterUniform(seed, counter[r]))
  // counter: device int32 per row (the absolute position), or nullptr with
  // counter_host used for every row. probs_out (optional, device): the filtered
  // distribution of row 0 (FilterToProbs), for parity tests.
  void Enqueue(const float* logits, int64_t ld, const int32_t* counter, int64_t counter_host, int32_t* token,
               float* probs_out, hipStream_t s);

  // Whether the parameters last set put some row on the full-vocabulary
  // kernels (sampled, no top-k): Enqueue then launches them. A graph
  // captured under one answer stays correct under the other (those rows
  // then take the one-workgroup path, or the extra launches exit at once);
  // callers recapture when it changes, for speed.
  bool wide() const { return wide_; }

  // Draws so far that took a slow path (test probe): which = 0 a sequential
  // double sum, 1 the top-p tie-order replay, 2 a tie-order replay that a
  // guard refused (index order kept; never expected).
  int64_t FallbackCount(hipStream_t s, int which = 0) const;

 private:
  void Carve(char* base, size_t bytes);
  bool RowIsWide(const SamplerParamsDev& p) const;
  int rows_, vocab_;
  bool wide_ = false;
  bool owns_ = true;
  SamplerParamsDev* params_ = nullptr;  // device [rows]
  float* work_ = nullptr;               // device [rows][vocab]
  int32_t* idx_ = nullptr;              // device [rows][vocab] compacted indices
  float* cand_v_ = nullptr;             // device [rows][vocab] top-k candidates per slice
  int32_t* cand_i_ = nullptr;           // device [rows][vocab]
  int32_t* cand_cnt_ = nullptr;         // device [rows][slices]
  unsigned long long* fallbacks_ = nullptr;  // [3]
  uint32_t* tie_key_ = nullptr;              // device [rows][vocab]: tie-order replay scratch
  int32_t* tie_pos_ = nullptr;
  int32_t* tie_l_ = nullptr;
  int32_t* tie_r_ = nullptr;
};

}  // namespace rpg

#endif  // RPG_HIP_SAMPLER_H_
