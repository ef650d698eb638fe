// Decode steps for several sessions of one model at once.
//
// Each session keeps its own KV cache, position and sampling parameters and
// produces exactly the tokens it would produce alone (reference
// src/qwen3.cc:302-355, one Generate per session; sessions share only the
// weights, reference include/rpg_engine.h threading note). A step samples
// every session's next token from its own logits row, forwards all of them
// together -- every projection as one multi-token GEMM over the batch, so
// each weight matrix is read once per step for all sessions -- with each
// token attending to its own cache at its own position, and leaves the next
// logits rows. The step is captured once as a hipGraph and replayed.

#ifndef RPG_HIP_BATCH_H_
#define RPG_HIP_BATCH_H_

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "model.h"
#include "sampler.h"
#include "session.h"

namespace rpg {

class SessionBatch {
 public:
  // sessions: 1 .. k::kMaxDecodeBatch distinct sessions of model m; they must
  // outlive the batch.
  SessionBatch(const DeviceModel& m, const std::vector<Session*>& sessions);
  ~SessionBatch();
  SessionBatch(const SessionBatch&) = delete;
  SessionBatch& operator=(const SessionBatch&) = delete;

  // max_tokens tokens for every session, written to out[b * max_tokens + i]:
  // each session continues from its device logits (those of its last
  // prefill or generate) with params[b], and afterwards holds the cache,
  // length and logits it would hold had it generated them alone. Every
  // session needs room for max_tokens more positions (checked first).
  // step_logits (optional, host [B][max_tokens][vocab]): row i of session b
  // receives the logits after its i-th generated token.
  // force (optional, host [B][max_tokens], parity tests): session b forwards
  // force[b * max_tokens + i] at step i instead of the drawn id, and out
  // receives the ids drawn (teacher forcing).
  void Generate(int32_t max_tokens, const std::vector<SampleParams>& params, int32_t* out,
                float* step_logits = nullptr, const int32_t* force = nullptr);

  // Device milliseconds of the last Generate's steps.
  float last_decode_ms() const { return last_decode_ms_; }

 private:
  void Init();
  void Release();
  void EnqueueStep(bool forced);
  void Capture();

  const DeviceModel& m_;
  std::vector<Session*> ss_;
  int B_ = 0;
  int64_t max_seq_all_ = 0;
  hipStream_t stream_ = nullptr, side_ = nullptr;
  hipEvent_t ev0_ = nullptr, ev1_ = nullptr, ev_fork_ = nullptr, ev_join_ = nullptr;
  float *x_ = nullptr, *h_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *attn_ = nullptr;
  float *act_ = nullptr, *gu_ = nullptr, *logits_ = nullptr, *work_ = nullptr;
  void* split_ = nullptr;
  int64_t work_stride_ = 0;
  int32_t *d_tok_ = nullptr, *d_pos_ = nullptr, *d_step_ = nullptr, *d_err_ = nullptr, *d_out_ = nullptr;
  int64_t out_cap_ = 0;  // tokens per session that d_out_ (and d_force_, d_drawn_) hold
  int32_t *d_force_ = nullptr, *d_drawn_ = nullptr;  // teacher forcing: forced and drawn ids
  Sampler* sampler_ = nullptr;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  bool use_graph_ = true;  // RPG_NO_GRAPH=1: enqueue each step's kernels directly
  bool graph_wide_ = false;  // the sampler's full-vocabulary launches are in the graph
  std::vector<int32_t> h_pos_;
  std::vector<SamplerParamsDev> h_params_;
  int32_t h_zero_ = 0;
  float last_decode_ms_ = 0.0f;
};

}  // namespace rpg

#endif  // RPG_HIP_BATCH_H_
