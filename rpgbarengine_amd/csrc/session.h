// One inference context on the GPU: KV cache, scratch buffers, stream and the
// captured decode-step graph.
//
// Semantics follow the reference token loop (reference src/qwen3.cc:208-363):
// * Prefill(ids) == ForwardFull with a cache: K/V of the segment are appended
//   at positions len..len+n-1, attention sees the whole history, len advances
//   only after every layer succeeded (reference :272-274).
// * Generate == reference Generate: pick (argmax, or CounterUniform(seed,
//   len) + SampleToken), append, stop check, capacity check, forward the picked
//   token -- every returned token, stop token included, is forwarded, so
//   len == prompt + returned afterwards (reference :317-354).
// The decode step runs device-resident: the picked token, the position and
// the step counter live in device memory, one hipGraph replay per token.

#ifndef RPG_HIP_SESSION_H_
#define RPG_HIP_SESSION_H_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "decode.h"
#include "decode_step.h"
#include "model.h"
#include "sampler.h"

namespace rpg {

struct SampleParams {
  float temperature = 0.0f;  // <= 0: greedy
  int32_t top_k = 0;
  float top_p = 1.0f;
  uint64_t seed = 0;
};

class Session {
 public:
  Session(const DeviceModel& m, int64_t max_seq);
  ~Session();
  Session(const Session&) = delete;
  Session& operator=(const Session&) = delete;

  int64_t len() const { return len_; }
  int64_t max_seq() const { return max_seq_; }
  void Reset() { len_ = 0; }
  void SetLen(int64_t n);

  // Forward n ids at positions len..len+n-1. Last-row logits stay on the
  // device (they seed Generate); optional host copies of the last row or of
  // every row.
  void Prefill(const int32_t* ids, int64_t n, float* last_logits_host, float* all_logits_host);

  // Returns the ids produced (stop id included). first_logits_host == nullptr
  // continues from the device logits of the last Prefill / step.
  // step_logits_host (optional) receives [returned, vocab].
  // force_host (optional, [max_tokens], parity tests): step i forwards
  // force_host[i] instead of the drawn id, and the returned ids are the ids
  // drawn (teacher forcing: every step decides on the logits of the forced
  // history); no stop ids.
  std::vector<int32_t> Generate(const float* first_logits_host, int32_t max_tokens, const SampleParams& sp,
                                const std::vector<int32_t>& stop_ids, float* step_logits_host,
                                const int32_t* force_host = nullptr);

  // Copy K (which = 0) or V (1) of (layer, kv head, positions [0, n)) to host.
  void ReadKv(int which, int layer, int head, int64_t n, float* out) const;

  hipStream_t stream() const { return stream_; }
  // True when a decode token runs as one persistent launch (decode_step.h).
  bool uses_step() const { return use_step_; }
  // Mean microseconds of `iters` back-to-back decode gate+up launches on this
  // session's stream (HIP events), on the current input, walking the layers
  // from `layer + 1` on; *bytes = the algorithmic bytes of one launch.
  double BenchGateUp(int layer, int iters, double* bytes);
  // The same launches inside decode steps: `tokens` greedy steps from the
  // current state through the per-launch path, each gate+up launch of every
  // layer bracketed by HIP events on the session stream (the interval also
  // holds the launch's dispatch after the previous kernel). Returns the mean
  // microseconds per launch; the session advances by `tokens`.
  double InStepGateUp(int tokens, double* bytes);
  // Milliseconds of the last Prefill and Generate calls (HIP events, on stream).
  float last_prefill_ms() const { return last_prefill_ms_; }
  float last_decode_ms() const { return last_decode_ms_; }

 private:
  friend class SessionBatch;  // steps several sessions' caches and logits together
  void Init();
  void Release();
  void EnsureScratch(int64_t tokens, int64_t logit_rows = 1);
  void RequireScratch(int64_t n) const;
  void ForwardSegment(const int32_t* ids_dev, int64_t n, int64_t pos0, const int32_t* pos_dev, int64_t logit_rows);
  void EnqueueDecodeStep(bool greedy, bool forced);
  void DecodeForward();
  void NormFirst(k::DecodeMatvecArgs* a);
  double GateUpBytes() const;
  k::DecodeMatvecArgs GateUpArgs(int layer) const;
  void CaptureDecode(bool greedy);
  // The persistent decode step's arguments for the current buffers.
  k::StepArgs StepArgsNow() const;
  void SetupStep();

  const DeviceModel& m_;
  int64_t max_seq_ = 0;
  int64_t len_ = 0;
  hipStream_t stream_ = nullptr;
  hipEvent_t ev0_ = nullptr, ev1_ = nullptr;
  // second prefill stream: a projection's second weight type runs beside
  // the first (fork / join events)
  hipStream_t side_ = nullptr;
  hipEvent_t ev_fork_ = nullptr, ev_join_ = nullptr;

  float* kcache_ = nullptr;  // [L][n_kv][max_seq][hd]
  float* vcache_ = nullptr;

  int64_t scratch_tokens_ = 0;
  float *x_ = nullptr, *h_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *attn_ = nullptr, *act_ = nullptr;
  float* logits_ = nullptr;  // [logit rows][vocab]
  float* gu_ = nullptr;      // [2][tokens][intermediate]: gate and up outputs of the GEMM path
  void* split_ = nullptr;    // split input of the GEMM path (k::SplitXBytes)
  int64_t logit_rows_cap_ = 0;
  float* attn_work_ = nullptr;
  float* dec_work_ = nullptr;  // decode attention partials + merge counters
  int32_t* ids_dev_ = nullptr;
  int64_t ids_cap_ = 0;

  // device-resident decode state
  int32_t* d_token_ = nullptr;
  uint64_t* d_pick_ = nullptr;  // the greedy pick's (key, count), zero between launches
  int32_t* d_pos_ = nullptr;  // [0] position, [1] epoch of the persistent step's tags
  int32_t* d_step_ = nullptr;
  int32_t* d_err_ = nullptr;
  int32_t* d_out_ids_ = nullptr;  // [max_seq]
  int32_t* d_force_ = nullptr;    // [max_seq] forced ids (teacher forcing), allocated on first use
  int32_t* d_drawn_ = nullptr;    // [max_seq] ids drawn under forcing
  Sampler* sampler_ = nullptr;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  int graph_mode_ = -1;  // -1 none, 0 sampled with top-k, 1 greedy, 2 sampled over the whole vocabulary
  bool use_graph_ = true;
  // in-step gate+up probe: event pairs DecodeForward records around each
  // gate+up launch while set (InStepGateUp)
  hipEvent_t* probe_ev_ = nullptr;
  size_t probe_i_ = 0;
  // the persistent decode step (decode_step.h): one launch per token when the
  // model fits it, else one launch per projection / attention stage
  bool use_step_ = false;
  int step_groups_ = 0;
  k::StepLayer* d_layers_ = nullptr;  // device [n_layers]
  uint2* tagged_ = nullptr;           // x, q, k, v, attn, act, attention partials
  int32_t* d_step_err_ = nullptr;

  // host sources of the small async uploads (must outlive the copy)
  int32_t h_pos_ = 0, h_zero_ = 0, h_token_ = 0;
  SamplerParamsDev h_params_{};

  float last_prefill_ms_ = 0.0f;
  float last_decode_ms_ = 0.0f;
};

}  // namespace rpg

#endif  // RPG_HIP_SESSION_H_
