#include "batch.h"

#include <cstdlib>

#include <algorithm>

#include "common.h"
#include "decode.h"
#include "forward.h"
#include "kernels.h"
#include "prefill.h"

namespace rpg {

SessionBatch::SessionBatch(const DeviceModel& m, const std::vector<Session*>& sessions) : m_(m), ss_(sessions) {
  const char* ng = std::getenv("RPG_NO_GRAPH");  // for tracers that do not follow graph launches
  use_graph_ = !(ng && *ng && *ng != '0');
  B_ = static_cast<int>(ss_.size());
  RPG_CHECK(B_ >= 1 && B_ <= k::kMaxDecodeBatch, "batch: %d sessions outside [1, %d]", B_, k::kMaxDecodeBatch);
  for (int b = 0; b < B_; ++b) {
    RPG_CHECK(ss_[b] != nullptr && &ss_[b]->m_ == &m, "batch: session %d belongs to another model", b);
    for (int o = 0; o < b; ++o) RPG_CHECK(ss_[o] != ss_[b], "batch: session %d appears twice", b);
    max_seq_all_ = std::max(max_seq_all_, ss_[b]->max_seq_);
  }
  try {
    Init();
  } catch (...) {
    Release();  // a failed constructor runs no destructor
    throw;
  }
}

void SessionBatch::Init() {
  const ModelConfig& c = m_.config();
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  HIP_CHECK(hipStreamCreateWithFlags(&side_, hipStreamNonBlocking));
  HIP_CHECK(hipEventCreate(&ev0_));
  HIP_CHECK(hipEventCreate(&ev1_));
  HIP_CHECK(hipEventCreateWithFlags(&ev_fork_, hipEventDisableTiming));
  HIP_CHECK(hipEventCreateWithFlags(&ev_join_, hipEventDisableTiming));
  auto alloc = [&](float** p, int64_t per_token) {
    DeviceAlloc(p, sizeof(float) * static_cast<size_t>(B_ * per_token));
  };
  alloc(&x_, c.hidden);
  alloc(&h_, c.hidden);
  alloc(&q_, c.q_dim());
  alloc(&k_, c.kv_dim());
  alloc(&v_, c.kv_dim());
  alloc(&attn_, c.q_dim());
  alloc(&act_, c.intermediate);
  alloc(&gu_, 2 * static_cast<int64_t>(c.intermediate));
  alloc(&logits_, c.vocab);
  work_stride_ = k::DecodeAttnBatchWorkFloats(c.n_heads, max_seq_all_);
  alloc(&work_, work_stride_);
  const int kmax = std::max({c.hidden, c.q_dim(), c.intermediate});
  DeviceAlloc(&split_, k::SplitXBytes(B_, kmax, SplitColumns(c)));
  DeviceAlloc(&d_tok_, sizeof(int32_t) * B_);
  DeviceAlloc(&d_pos_, sizeof(int32_t) * B_);
  DeviceAlloc(&d_step_, sizeof(int32_t));
  DeviceAlloc(&d_err_, sizeof(int32_t));
  HIP_CHECK(hipMemsetAsync(d_err_, 0, sizeof(int32_t), stream_));
  sampler_ = new Sampler(B_, c.vocab);
  h_pos_.resize(static_cast<size_t>(B_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

SessionBatch::~SessionBatch() { Release(); }

void SessionBatch::Release() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  graph_exec_ = nullptr;
  graph_ = nullptr;
  delete sampler_;
  sampler_ = nullptr;
  for (void* p : {static_cast<void*>(x_), static_cast<void*>(h_), static_cast<void*>(q_), static_cast<void*>(k_),
                  static_cast<void*>(v_), static_cast<void*>(attn_), static_cast<void*>(act_),
                  static_cast<void*>(gu_), static_cast<void*>(logits_), static_cast<void*>(work_), split_,
                  static_cast<void*>(d_tok_), static_cast<void*>(d_pos_), static_cast<void*>(d_step_),
                  static_cast<void*>(d_err_), static_cast<void*>(d_out_), static_cast<void*>(d_force_),
                  static_cast<void*>(d_drawn_)}) {
    if (p) (void)hipFree(p);
  }
  for (hipEvent_t e : {ev0_, ev1_, ev_fork_, ev_join_})
    if (e) (void)hipEventDestroy(e);
  if (side_) (void)hipStreamDestroy(side_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

// One step for every session: sample each row (u from the session's seed and
// position), record the tokens, forward them, advance the positions.
void SessionBatch::EnqueueStep(bool forced) {
  const ModelConfig& c = m_.config();
  const int H = c.hidden;
  sampler_->Enqueue(logits_, c.vocab, d_pos_, 0, d_tok_, nullptr, stream_);
  if (forced) k::ForceTokens(d_tok_, B_, d_force_, d_drawn_, d_step_, out_cap_, stream_);
  k::GatherRows(m_.embd(), d_tok_, B_, x_, H, d_err_, stream_, d_out_, d_step_, out_cap_);
  const FwdBufs b{x_, h_, q_, k_, v_, attn_, act_, gu_, split_, SplitColumns(c), stream_, side_, ev_fork_, ev_join_};
  ForwardLayers(m_, b, B_, [&](int l, const LayerDev& w) {
    k::DecodeAttnBatchArgs ab{};
    ab.base.q = q_;
    ab.base.k = k_;
    ab.base.v = v_;
    ab.base.q_norm = w.q_norm;
    ab.base.k_norm = w.k_norm;
    ab.base.rope = m_.rope();
    ab.base.out = attn_;
    ab.base.work = work_;
    ab.base.n_heads = c.n_heads;
    ab.base.n_kv = c.n_kv_heads;
    ab.base.eps = c.rms_eps;
    ab.base.pos_dev = d_pos_;
    for (int z = 0; z < B_; ++z) {
      const Session& s = *ss_[z];
      const int64_t layer_cache = static_cast<int64_t>(c.n_kv_heads) * s.max_seq_ * c.head_dim;
      ab.kcache[z] = s.kcache_ + l * layer_cache;
      ab.vcache[z] = s.vcache_ + l * layer_cache;
      ab.max_seq[z] = s.max_seq_;
    }
    ab.q_stride = c.q_dim();
    ab.kv_stride = c.kv_dim();
    ab.work_stride = work_stride_;
    k::DecodeAttentionBatch(ab, B_, max_seq_all_, stream_);
  });
  // final RMSNorm + lm_head: on the matrix cores from the tile-major copy
  // (the norm folded into the staging), else normed rows and the matvec
  bool done = false;
  if (m_.lm_head_tiled().w != nullptr) {
    k::DecodeBatchArgs a;
    const k::MatRef& t = m_.lm_head_tiled();
    a.job[0].w = t.w;
    a.job[0].row_bytes = t.row_bytes;
    a.job[0].type = t.type;
    a.job[0].rows = t.rows;
    a.job[0].y = logits_;
    a.job[0].tiled = 1;
    a.ldy[0] = c.vocab;
    a.x = x_;
    a.ldx = H;
    a.T = B_;
    a.K = H;
    a.norm_w = m_.output_norm();
    a.eps = c.rms_eps;
    done = k::DecodeMatvecBatch(a, stream_);
  }
  if (!done) {
    k::RmsNormRows(x_, H, m_.output_norm(), H, B_, c.rms_eps, h_, H, stream_);
    k::Matvec(m_.lm_head(), h_, H, B_, logits_, c.vocab, k::kStore, stream_);
  }
  k::AdvancePositions(d_pos_, B_, d_step_, stream_);
}

void SessionBatch::Capture() {
  if (!use_graph_) return;
  if (graph_exec_ && graph_wide_ != sampler_->wide()) {  // the sampler's launches differ
    HIP_CHECK(hipGraphExecDestroy(graph_exec_));
    HIP_CHECK(hipGraphDestroy(graph_));
    graph_exec_ = nullptr;
    graph_ = nullptr;
  }
  if (graph_exec_) return;
  graph_wide_ = sampler_->wide();
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
  try {
    EnqueueStep(false);
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream_, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  HIP_CHECK(hipStreamEndCapture(stream_, &graph_));
  HIP_CHECK(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
}

void SessionBatch::Generate(int32_t max_tokens, const std::vector<SampleParams>& params, int32_t* out,
                            float* step_logits, const int32_t* force) {
  const ModelConfig& c = m_.config();
  RPG_CHECK(max_tokens > 0, "max_tokens must be positive (got %d)", max_tokens);
  RPG_CHECK(static_cast<int>(params.size()) == B_, "batch: %zu parameter sets for %d sessions", params.size(), B_);
  for (int b = 0; b < B_; ++b) {
    const Session& s = *ss_[b];
    RPG_CHECK(s.len_ > 0 && s.logits_ != nullptr && s.scratch_tokens_ >= 1,
              "batch: session %d has no logits yet (prefill first)", b);
    // the reference stops with an error once the cache is full (reference
    // src/qwen3.cc:341-344); a batch checks every session up front instead
    RPG_CHECK(s.len_ + max_tokens <= s.max_seq_,
              "context full: session %d holds %lld of %lld positions and cannot take %d more", b, (long long)s.len_,
              (long long)s.max_seq_, max_tokens);
  }
  const bool forced = force != nullptr;
  if (forced) {
    for (int64_t i = 0; i < static_cast<int64_t>(B_) * max_tokens; ++i)
      RPG_CHECK(force[i] >= 0 && force[i] < c.vocab, "forced token %lld has id %d, outside the vocabulary",
                (long long)i, force[i]);
  }
  if (max_tokens > out_cap_ || (forced && !d_force_)) {
    if (graph_exec_) {  // the graph records into the old buffer
      HIP_CHECK(hipGraphExecDestroy(graph_exec_));
      HIP_CHECK(hipGraphDestroy(graph_));
      graph_exec_ = nullptr;
      graph_ = nullptr;
    }
    HIP_CHECK(hipStreamSynchronize(stream_));
    const int64_t cap = std::max<int64_t>(out_cap_, max_tokens);
    out_cap_ = 0;  // no capacity while the buffers are replaced
    for (int32_t** p : {&d_out_, &d_force_, &d_drawn_}) {
      if (*p) HIP_CHECK(hipFree(*p));
      *p = nullptr;
    }
    const size_t bytes = sizeof(int32_t) * static_cast<size_t>(B_) * cap;
    DeviceAlloc(&d_out_, bytes);
    if (forced) {
      DeviceAlloc(&d_force_, bytes);
      DeviceAlloc(&d_drawn_, bytes);
    }
    out_cap_ = cap;
  }
  if (forced)
    HIP_CHECK(hipMemcpy2DAsync(d_force_, sizeof(int32_t) * out_cap_, force, sizeof(int32_t) * max_tokens,
                               sizeof(int32_t) * max_tokens, static_cast<size_t>(B_), hipMemcpyHostToDevice, stream_));
  // the sessions' own work (prefills) is complete before their logits and
  // caches are read on this stream
  h_params_.clear();
  for (int b = 0; b < B_; ++b) {
    Session& s = *ss_[b];
    HIP_CHECK(hipStreamSynchronize(s.stream_));
    HIP_CHECK(hipMemcpyAsync(logits_ + static_cast<int64_t>(b) * c.vocab, s.logits_, sizeof(float) * c.vocab,
                             hipMemcpyDeviceToDevice, stream_));
    h_pos_[static_cast<size_t>(b)] = static_cast<int32_t>(s.len_);
    const SampleParams& p = params[static_cast<size_t>(b)];
    h_params_.push_back(SamplerParamsDev{p.temperature, p.top_k, p.top_p, 0, p.seed});
  }
  sampler_->SetParams(h_params_.data(), B_, stream_);
  h_zero_ = 0;
  HIP_CHECK(hipMemcpyAsync(d_pos_, h_pos_.data(), sizeof(int32_t) * B_, hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(d_step_, &h_zero_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
  // forced steps are enqueued directly (the captured graph draws freely)
  const bool graph = use_graph_ && !forced;
  if (graph) Capture();
  HIP_CHECK(hipEventRecord(ev0_, stream_));
  const size_t row = sizeof(float) * static_cast<size_t>(c.vocab);
  for (int32_t i = 0; i < max_tokens; ++i) {
    if (graph)
      HIP_CHECK(hipGraphLaunch(graph_exec_, stream_));
    else
      EnqueueStep(forced);
    if (step_logits)
      HIP_CHECK(hipMemcpy2DAsync(step_logits + static_cast<int64_t>(i) * c.vocab, row * max_tokens, logits_, row, row,
                                 static_cast<size_t>(B_), hipMemcpyDeviceToHost, stream_));
  }
  HIP_CHECK(hipEventRecord(ev1_, stream_));
  // the rows of d_out_ are out_cap_ apart
  HIP_CHECK(hipMemcpy2DAsync(out, sizeof(int32_t) * max_tokens, forced ? d_drawn_ : d_out_, sizeof(int32_t) * out_cap_,
                             sizeof(int32_t) * max_tokens, static_cast<size_t>(B_), hipMemcpyDeviceToHost, stream_));
  // each session continues from its own last logits row
  for (int b = 0; b < B_; ++b)
    HIP_CHECK(hipMemcpyAsync(ss_[b]->logits_, logits_ + static_cast<int64_t>(b) * c.vocab, sizeof(float) * c.vocab,
                             hipMemcpyDeviceToDevice, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipEventElapsedTime(&last_decode_ms_, ev0_, ev1_));
  int32_t err = 0;
  HIP_CHECK(hipMemcpy(&err, d_err_, sizeof(int32_t), hipMemcpyDeviceToHost));
  RPG_CHECK(err == 0, "a device-side token id fell outside the vocabulary");
  for (int b = 0; b < B_; ++b) ss_[b]->len_ += max_tokens;
}

}  // namespace rpg
