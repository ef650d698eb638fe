#include "session.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "common.h"
#include "decode.h"
#include "forward.h"
#include "kernels.h"
#include "prefill.h"
#include "sampler.h"

namespace rpg {

namespace {
// Tokens per prefill pass. Long passes keep the GEMMs and the attention
// wide (a 4000-token prompt in one pass: 55 ms, in passes of 512: 89 ms);
// the scratch grows with the pass, ~0.25 MB per token for the 4B shape.
constexpr int64_t kPrefillChunk = 4096;
// Tokens per pass when every position's logits are returned (the logits
// buffer holds a row per token of the pass, 0.6 MB each).
constexpr int64_t kLogitRowsChunk = 512;
constexpr int kGenChunk = 16;           // decode steps between host stop checks
// The persistent decode step needs every one of its workgroups resident at
// once; two of them running together (sessions generating from different
// host threads) could each hold compute units the other waits for. Its
// generations therefore run one at a time in the process.
std::mutex g_persistent_mu;
}  // namespace

Session::Session(const DeviceModel& m, int64_t max_seq) : m_(m), max_seq_(max_seq) {
  // RPG_NO_GRAPH=1 enqueues the same decode-step kernels directly on the
  // stream instead of replaying the captured graph (for tracers that do not
  // follow graph launches).
  const char* ng = std::getenv("RPG_NO_GRAPH");
  use_graph_ = !(ng && *ng && *ng != '0');
  RPG_CHECK(max_seq > 0, "max_seq must be positive (got %lld)", (long long)max_seq);
  RPG_CHECK(max_seq <= m.rope_positions(), "max_seq %lld exceeds the RoPE table (%lld positions)",
            (long long)max_seq, (long long)m.rope_positions());
  try {
    Init();
  } catch (...) {
    Release();  // a failed constructor runs no destructor
    throw;
  }
}

void Session::Init() {
  const ModelConfig& c = m_.config();
  const int64_t max_seq = max_seq_;
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  HIP_CHECK(hipEventCreate(&ev0_));
  HIP_CHECK(hipEventCreate(&ev1_));
  HIP_CHECK(hipStreamCreateWithFlags(&side_, hipStreamNonBlocking));
  HIP_CHECK(hipEventCreateWithFlags(&ev_fork_, hipEventDisableTiming));
  HIP_CHECK(hipEventCreateWithFlags(&ev_join_, hipEventDisableTiming));
  const size_t cache = static_cast<size_t>(c.n_layers) * c.n_kv_heads * max_seq * c.head_dim * sizeof(float);
  DeviceAlloc(&kcache_, cache);
  DeviceAlloc(&vcache_, cache);
  // zeroed like the reference cache (reference src/kv_cache.cc:25-26)
  HIP_CHECK(hipMemsetAsync(kcache_, 0, cache, stream_));
  HIP_CHECK(hipMemsetAsync(vcache_, 0, cache, stream_));
  DeviceAlloc(&attn_work_, sizeof(float) * k::AttnWorkFloats(c.n_heads, max_seq));
  const size_t dec_work = sizeof(float) * k::DecodeAttnWorkFloats(c.n_heads, c.n_kv_heads, max_seq);
  DeviceAlloc(&dec_work_, dec_work);
  HIP_CHECK(hipMemsetAsync(dec_work_, 0, dec_work, stream_));  // merge counters start at zero
  DeviceAlloc(&d_token_, sizeof(int32_t));
  DeviceAlloc(&d_pick_, 2 * sizeof(uint64_t));
  HIP_CHECK(hipMemsetAsync(d_pick_, 0, 2 * sizeof(uint64_t), stream_));  // the greedy pick's (key, count)
  DeviceAlloc(&d_pos_, 2 * sizeof(int32_t));
  DeviceAlloc(&d_step_, sizeof(int32_t));
  DeviceAlloc(&d_err_, sizeof(int32_t));
  DeviceAlloc(&d_out_ids_, sizeof(int32_t) * static_cast<size_t>(max_seq + 1));
  HIP_CHECK(hipMemsetAsync(d_err_, 0, sizeof(int32_t), stream_));
  sampler_ = new Sampler(1, c.vocab);
  EnsureScratch(1);
  SetupStep();
  HIP_CHECK(hipStreamSynchronize(stream_));
}

namespace {
// log2 of the waves per tile for a projection of `tiles` tiles over n_sb
// super-blocks: the most (at most 8, at most one per super-block) that keep
// the tiles within one slot per workgroup.
int32_t StepKwl(int64_t tiles, int n_sb, int groups) {
  int kwl = 3;
  while (kwl > 0 && ((1 << kwl) > n_sb || CeilDiv(tiles, k::kStepWaves >> kwl) > groups)) --kwl;
  return kwl;
}
}  // namespace

void Session::SetupStep() {
  const ModelConfig& c = m_.config();
  // Opt-in: on MI355X the persistent step measures slower than the
  // per-launch graph (each phase's input wait reads tagged words at device
  // coherence, past the compute unit's L2), so it runs only when asked for.
  const char* env = std::getenv("RPG_DECODE_STEP");
  if (!env || !*env || *env == '0') return;
  bool tiled = m_.lm_head_tiled().w != nullptr && c.n_layers <= 64;
  // (its matrix phases read Q4_K / Q6_K tile-major copies only)
  auto kq = [](const k::MatRef& r) { return r.type == kQ4_K || r.type == kQ6_K; };
  tiled = tiled && kq(m_.lm_head());
  for (const LayerDev& w : m_.layers())
    tiled = tiled && w.dq.w && w.dk.w && w.dv.w && w.dout.w && w.gate_up.w && w.ddown.w && kq(w.q) && kq(w.k) &&
            kq(w.v) && kq(w.o) && kq(w.gate) && kq(w.down);
  if (!tiled) return;
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  HIP_CHECK(hipDeviceGetAttribute(&step_groups_, hipDeviceAttributeMultiprocessorCount, dev));
  std::vector<k::StepLayer> host(static_cast<size_t>(c.n_layers));
  const int64_t layer_cache = static_cast<int64_t>(c.n_kv_heads) * max_seq_ * c.head_dim;
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerDev& w = m_.layers()[static_cast<size_t>(l)];
    k::StepLayer& L = host[static_cast<size_t>(l)];
    const k::MatRef* mats[6] = {&w.dq, &w.dk, &w.dv, &w.dout, &w.gate_up, &w.ddown};
    const k::MatRef* rm[6] = {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.down};
    for (int j = 0; j < 6; ++j) {
      L.w[j] = mats[j]->w;
      L.type[j] = static_cast<int32_t>(rm[j]->type);
    }
    const int n_sb_h = c.hidden / 256, n_sb_q = c.q_dim() / 256, n_sb_f = c.intermediate / 256;
    L.kwl[0] = L.kwl[1] = L.kwl[2] =
        StepKwl(CeilDiv(c.q_dim(), 16) + 2 * CeilDiv(c.kv_dim(), 16), n_sb_h, step_groups_);
    L.kwl[3] = StepKwl(CeilDiv(c.hidden, 16), n_sb_q, step_groups_);
    L.kwl[4] = StepKwl(CeilDiv(c.intermediate, 8), n_sb_h, step_groups_);
    L.kwl[5] = StepKwl(CeilDiv(c.hidden, 16), n_sb_f, step_groups_);
    L.attn_norm = w.attn_norm;
    L.ffn_norm = w.ffn_norm;
    L.q_norm = w.q_norm;
    L.k_norm = w.k_norm;
    L.kcache = kcache_ + l * layer_cache;
    L.vcache = vcache_ + l * layer_cache;
  }
  const int64_t n_part = static_cast<int64_t>(c.n_heads) * CeilDiv(max_seq_, 32) * (2 + c.head_dim);
  const int64_t words = 2 * static_cast<int64_t>(c.hidden) + 2 * c.q_dim() + 2 * c.kv_dim() + c.intermediate + n_part;
  DeviceAlloc(&d_layers_, sizeof(k::StepLayer) * host.size());
  HIP_CHECK(hipMemcpy(d_layers_, host.data(), sizeof(k::StepLayer) * host.size(), hipMemcpyHostToDevice));
  DeviceAlloc(&tagged_, sizeof(uint2) * static_cast<size_t>(words));
  // tags that no phase of any epoch writes (epoch * kTagSpan + phase < 2^32 - 1)
  HIP_CHECK(hipMemsetAsync(tagged_, 0xFF, sizeof(uint2) * static_cast<size_t>(words), stream_));
  DeviceAlloc(&d_step_err_, sizeof(int32_t));
  HIP_CHECK(hipMemsetAsync(d_step_err_, 0, sizeof(int32_t), stream_));
  const int32_t pos_epoch[2] = {0, 1};
  HIP_CHECK(hipMemcpy(d_pos_, pos_epoch, sizeof(pos_epoch), hipMemcpyHostToDevice));
  use_step_ = k::DecodeStepSupported(StepArgsNow(), step_groups_);
}

k::StepArgs Session::StepArgsNow() const {
  const ModelConfig& c = m_.config();
  k::StepArgs a{};
  a.layers = d_layers_;
  a.n_layers = c.n_layers;
  a.H = c.hidden;
  a.qd = c.q_dim();
  a.kvd = c.kv_dim();
  a.F = c.intermediate;
  a.V = c.vocab;
  a.n_heads = c.n_heads;
  a.n_kv = c.n_kv_heads;
  a.max_seq = max_seq_;
  a.eps = c.rms_eps;
  a.rope = m_.rope();
  a.embd = m_.embd();
  a.lm_head = m_.lm_head_tiled().w;
  a.lm_type = static_cast<int32_t>(m_.lm_head().type);
  a.lm_kwl = StepKwl(CeilDiv(c.vocab, 16), c.hidden / 256, step_groups_);
  a.output_norm = m_.output_norm();
  uint2* t = tagged_;
  a.x = t;
  t += c.hidden;
  a.q = t;
  t += c.q_dim();
  a.k = t;
  t += c.kv_dim();
  a.v = t;
  t += c.kv_dim();
  a.attn = t;
  t += c.q_dim();
  a.act = t;
  t += c.intermediate;
  a.part = t;
  a.logits = logits_;
  a.token = d_token_;
  a.pos = d_pos_;
  a.out_ids = d_out_ids_;
  a.step = d_step_;
  a.err = d_step_err_;
  return a;
}

Session::~Session() { Release(); }

void Session::Release() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  graph_exec_ = nullptr;
  graph_ = nullptr;
  delete sampler_;
  sampler_ = nullptr;
  for (void* p : {static_cast<void*>(kcache_), static_cast<void*>(vcache_), static_cast<void*>(x_),
                  static_cast<void*>(h_), static_cast<void*>(q_), static_cast<void*>(k_), static_cast<void*>(v_),
                  static_cast<void*>(attn_), static_cast<void*>(act_), static_cast<void*>(logits_),
                  static_cast<void*>(attn_work_), static_cast<void*>(dec_work_), static_cast<void*>(ids_dev_),
                  static_cast<void*>(d_token_), static_cast<void*>(d_pick_),
                  static_cast<void*>(d_pos_), static_cast<void*>(d_step_), static_cast<void*>(d_err_),
                  static_cast<void*>(d_out_ids_), static_cast<void*>(gu_), split_, static_cast<void*>(d_layers_),
                  static_cast<void*>(tagged_), static_cast<void*>(d_step_err_), static_cast<void*>(d_force_),
                  static_cast<void*>(d_drawn_)}) {
    if (p) (void)hipFree(p);
  }
  if (ev0_) (void)hipEventDestroy(ev0_);
  if (ev1_) (void)hipEventDestroy(ev1_);
  if (ev_fork_) (void)hipEventDestroy(ev_fork_);
  if (ev_join_) (void)hipEventDestroy(ev_join_);
  if (side_) (void)hipStreamDestroy(side_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void Session::SetLen(int64_t n) {
  RPG_CHECK(n >= 0 && n <= max_seq_, "length %lld out of range (capacity %lld)", (long long)n, (long long)max_seq_);
  len_ = n;
}

void Session::EnsureScratch(int64_t tokens, int64_t logit_rows) {
  if (tokens <= scratch_tokens_ && logit_rows <= logit_rows_cap_) return;
  tokens = std::max(tokens, scratch_tokens_);  // regrowth keeps what the session held
  logit_rows = std::max(logit_rows, logit_rows_cap_);
  // the decode graph holds pointers into these buffers
  if (graph_exec_) {
    (void)hipGraphExecDestroy(graph_exec_);
    (void)hipGraphDestroy(graph_);
    graph_exec_ = nullptr;
    graph_ = nullptr;
    graph_mode_ = -1;
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  // No capacity until every buffer is in place: an allocation that throws
  // below leaves a session whose next request allocates again from scratch.
  scratch_tokens_ = 0;
  logit_rows_cap_ = 0;
  const ModelConfig& c = m_.config();
  for (float** p : {&x_, &h_, &q_, &k_, &v_, &attn_, &act_, &logits_, &gu_}) {
    if (*p) HIP_CHECK(hipFree(*p));
    *p = nullptr;
  }
  if (split_) HIP_CHECK(hipFree(split_));
  split_ = nullptr;
  auto alloc = [&](float** p, int64_t per_token) {
    DeviceAlloc(p, sizeof(float) * static_cast<size_t>(tokens * per_token));
  };
  alloc(&x_, c.hidden);
  alloc(&h_, c.hidden);
  alloc(&q_, c.q_dim());
  alloc(&k_, c.kv_dim());
  alloc(&v_, c.kv_dim());
  alloc(&attn_, c.q_dim());
  alloc(&act_, c.intermediate);
  DeviceAlloc(&logits_, sizeof(float) * static_cast<size_t>(logit_rows * c.vocab));
  if (tokens >= 2) {  // GEMM operands of multi-token segments
    alloc(&gu_, 2 * static_cast<int64_t>(c.intermediate));
    const int kmax = std::max({c.hidden, c.q_dim(), c.intermediate});
    DeviceAlloc(&split_, k::SplitXBytes(static_cast<int>(tokens), kmax, SplitColumns(c)));
  }
  scratch_tokens_ = tokens;
  logit_rows_cap_ = logit_rows;
}

// Host-side guard before any enqueue: the buffers a segment of n tokens
// uses are in place (a failed allocation never reaches a kernel).
void Session::RequireScratch(int64_t n) const {
  RPG_CHECK(n >= 1 && n <= scratch_tokens_ && x_ && h_ && q_ && k_ && v_ && attn_ && act_ && logits_ &&
                (n < 2 || (gu_ && split_)),
            "internal: scratch for %lld tokens is not allocated (capacity %lld)", (long long)n,
            (long long)scratch_tokens_);
}

// Forward n tokens (device ids) at positions pos0.. (pos_dev overrides pos0
// for the captured decode step). Logits of the last `logit_rows` tokens go to
// logits_[0 .. logit_rows).
void Session::ForwardSegment(const int32_t* ids_dev, int64_t n, int64_t pos0, const int32_t* pos_dev,
                             int64_t logit_rows) {
  const ModelConfig& c = m_.config();
  const int H = c.hidden, N = static_cast<int>(n);
  const int64_t layer_cache = static_cast<int64_t>(c.n_kv_heads) * max_seq_ * c.head_dim;
  RequireScratch(n);
  RPG_CHECK(logit_rows <= logit_rows_cap_, "internal: %lld logits rows, capacity %lld", (long long)logit_rows,
            (long long)logit_rows_cap_);
  k::GatherRows(m_.embd(), ids_dev, N, x_, H, d_err_, stream_);
  const FwdBufs b{x_, h_, q_, k_, v_, attn_, act_, gu_, split_, SplitColumns(c), stream_, side_, ev_fork_, ev_join_};
  ForwardLayers(m_, b, N, [&](int l, const LayerDev& w) {
    k::QkvArgs qa;
    qa.q = q_;
    qa.k = k_;
    qa.v = v_;
    qa.q_norm = w.q_norm;
    qa.k_norm = w.k_norm;
    qa.rope = m_.rope();
    qa.kcache = kcache_ + l * layer_cache;
    qa.vcache = vcache_ + l * layer_cache;
    qa.seq = N;
    qa.n_heads = c.n_heads;
    qa.n_kv = c.n_kv_heads;
    qa.hd = c.head_dim;
    qa.max_seq = max_seq_;
    qa.eps = c.rms_eps;
    qa.pos0_dev = pos_dev;
    qa.pos0_host = static_cast<int32_t>(pos0);
    k::QkNormRopeCache(qa, stream_);
    k::AttnArgs aa;
    aa.q = q_;
    aa.kcache = qa.kcache;
    aa.vcache = qa.vcache;
    aa.out = attn_;
    aa.work = attn_work_;
    aa.seq = N;
    aa.n_heads = c.n_heads;
    aa.n_kv = c.n_kv_heads;
    aa.hd = c.head_dim;
    aa.max_seq = max_seq_;
    aa.pos0_dev = pos_dev;
    aa.pos0_host = static_cast<int32_t>(pos0);
    k::Attention(aa, stream_);
  });
  if (logit_rows == 1 && m_.lm_head_tiled().w != nullptr) {
    // the last position's logits as the decode step forms them: RMSNorm
    // folded into the matrix-core launch over the tile-major lm_head copy
    k::DecodeMatvecArgs lm;
    lm.x = x_ + (n - 1) * H;
    lm.K = H;
    lm.norm_w = m_.output_norm();
    lm.eps = c.rms_eps;
    lm.job[0].w = m_.lm_head_tiled().w;
    lm.job[0].tiled = 1;
    lm.job[0].row_bytes = m_.lm_head().row_bytes;
    lm.job[0].type = m_.lm_head().type;
    lm.job[0].rows = m_.lm_head().rows;
    lm.job[0].y = logits_;
    NormFirst(&lm);
    k::DecodeMatvec(lm, stream_);
  } else if (logit_rows > 0) {
    const int64_t r0 = n - logit_rows;
    k::RmsNormRows(x_ + r0 * H, H, m_.output_norm(), H, static_cast<int>(logit_rows), c.rms_eps, h_, H, stream_);
    k::Matvec(m_.lm_head(), h_, H, static_cast<int>(logit_rows), logits_, c.vocab, k::kStore, stream_);
  }
}

void Session::Prefill(const int32_t* ids, int64_t n, float* last_logits_host, float* all_logits_host) {
  const ModelConfig& c = m_.config();
  RPG_CHECK(n > 0, "empty prompt");
  for (int64_t t = 0; t < n; ++t) {
    RPG_CHECK(ids[t] >= 0 && ids[t] < c.vocab, "token %lld has id %d, outside the vocabulary (%d)", (long long)t,
              ids[t], c.vocab);
  }
  const int64_t pos0 = len_;
  RPG_CHECK(pos0 + n <= m_.rope_positions(), "position %lld beyond the RoPE table (%lld positions)",
            (long long)(pos0 + n), (long long)m_.rope_positions());
  RPG_CHECK(pos0 + n <= max_seq_, "position %lld beyond the KV cache capacity %lld", (long long)(pos0 + n),
            (long long)max_seq_);
  const int64_t chunk = std::min<int64_t>(n, all_logits_host ? kLogitRowsChunk : kPrefillChunk);
  EnsureScratch(chunk, all_logits_host ? chunk : 1);
  if (ids_cap_ < n) {
    ids_cap_ = 0;  // no capacity while the buffer is replaced
    if (ids_dev_) HIP_CHECK(hipFree(ids_dev_));
    ids_dev_ = nullptr;
    DeviceAlloc(&ids_dev_, sizeof(int32_t) * static_cast<size_t>(n));
    ids_cap_ = n;
  }
  HIP_CHECK(hipMemcpyAsync(ids_dev_, ids, sizeof(int32_t) * static_cast<size_t>(n), hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipEventRecord(ev0_, stream_));
  for (int64_t c0 = 0; c0 < n; c0 += chunk) {
    const int64_t cn = std::min(chunk, n - c0);
    const bool last_chunk = c0 + cn == n;
    const int64_t rows = all_logits_host ? cn : (last_chunk ? 1 : 0);
    ForwardSegment(ids_dev_ + c0, cn, pos0 + c0, nullptr, rows);
    if (all_logits_host) {
      HIP_CHECK(hipMemcpyAsync(all_logits_host + c0 * c.vocab, logits_, sizeof(float) * cn * c.vocab,
                               hipMemcpyDeviceToHost, stream_));
      if (last_chunk && cn > 1)
        HIP_CHECK(hipMemcpyAsync(logits_, logits_ + (cn - 1) * c.vocab, sizeof(float) * c.vocab,
                                 hipMemcpyDeviceToDevice, stream_));
    }
  }
  HIP_CHECK(hipEventRecord(ev1_, stream_));
  if (last_logits_host)
    HIP_CHECK(hipMemcpyAsync(last_logits_host, logits_, sizeof(float) * c.vocab, hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipEventElapsedTime(&last_prefill_ms_, ev0_, ev1_));
  len_ = pos0 + n;  // committed once every layer ran (reference src/qwen3.cc:272-274)
}

void Session::EnqueueDecodeStep(bool greedy, bool forced) {
  const ModelConfig& c = m_.config();
  if (greedy) {
    k::ArgMaxRows(logits_, c.vocab, c.vocab, 1, d_token_, stream_, d_pick_);
  } else {
    sampler_->Enqueue(logits_, c.vocab, d_pos_, 0, d_token_, nullptr, stream_);
  }
  if (forced) k::ForceTokens(d_token_, 1, d_force_, d_drawn_, d_step_, 0, stream_);
  if (use_step_) {
    // one launch forwards the token (and records it); then position, epoch
    // and record slot advance
    k::DecodeStep(StepArgsNow(), step_groups_, stream_);
    k::AdvancePositions(d_pos_, 2, d_step_, stream_);
  } else {
    DecodeForward();  // also records the token and advances the position
  }
}

// One token at the device position *d_pos_: embedding of *d_token_ (whose
// launch also records the token: d_out_ids_[*d_step_++]), per layer
// [norm+QKV] [QK-norm+RoPE+cache+attention] [O + residual] [norm+gate/up+SwiGLU]
// [down + residual], then [norm + lm_head] -> logits_[0] (whose launch also
// advances *d_pos_).
void Session::DecodeForward() {
  const ModelConfig& c = m_.config();
  const int H = c.hidden, F = c.intermediate, qd = c.q_dim();
  const int64_t layer_cache = static_cast<int64_t>(c.n_kv_heads) * max_seq_ * c.head_dim;
  RequireScratch(1);
  // A launch reads the tile-major copies `t` when every job has one and the
  // matrix cores take its types together (Q4_K with Q6_K, or Q8_0 alone),
  // else the row-major matrices `m` of every job.
  auto tiled = [](std::initializer_list<std::pair<const k::MatRef*, const k::MatRef*>> jobs) {
    bool q8 = false, kq = false;
    for (const auto& p : jobs) {
      if (p.second->w == nullptr) return false;
      (p.first->type == kQ8_0 ? q8 : kq) = true;
    }
    return !(q8 && kq);
  };
  auto job = [](const k::MatRef& m, const k::MatRef& t, bool use_t, float* y) {
    k::DecodeJob j;
    j.w = use_t ? t.w : m.w;
    j.tiled = use_t;
    j.row_bytes = m.row_bytes;
    j.type = m.type;
    j.rows = m.rows;
    j.y = y;
    return j;
  };
  k::GatherRows(m_.embd(), d_token_, 1, x_, H, d_err_, stream_, d_out_ids_, d_step_);
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerDev& w = m_.layers()[static_cast<size_t>(l)];
    k::DecodeMatvecArgs qkv;
    qkv.x = x_;
    qkv.K = H;
    qkv.norm_w = w.attn_norm;
    qkv.eps = c.rms_eps;
    qkv.n_jobs = 3;
    const bool tq = tiled({{&w.q, &w.dq}, {&w.k, &w.dk}, {&w.v, &w.dv}});
    qkv.job[0] = job(w.q, w.dq, tq, q_);
    qkv.job[1] = job(w.k, w.dk, tq, k_);
    qkv.job[2] = job(w.v, w.dv, tq, v_);
    NormFirst(&qkv);
    k::DecodeMatvec(qkv, stream_);
    k::DecodeAttnArgs at;
    at.q = q_;
    at.k = k_;
    at.v = v_;
    at.q_norm = w.q_norm;
    at.k_norm = w.k_norm;
    at.rope = m_.rope();
    at.kcache = kcache_ + l * layer_cache;
    at.vcache = vcache_ + l * layer_cache;
    at.out = attn_;
    at.work = dec_work_;
    at.n_heads = c.n_heads;
    at.n_kv = c.n_kv_heads;
    at.max_seq = max_seq_;
    at.eps = c.rms_eps;
    at.pos_dev = d_pos_;
    k::DecodeAttention(at, stream_);
    k::DecodeMatvecArgs o;
    o.x = attn_;
    o.K = qd;
    o.job[0] = job(w.o, w.dout, w.dout.w != nullptr, x_);
    o.epi = k::kAdd;
    k::DecodeMatvec(o, stream_);
    k::DecodeMatvecArgs gu = GateUpArgs(l);
    NormFirst(&gu);
    if (probe_ev_) HIP_CHECK(hipEventRecord(probe_ev_[probe_i_++], stream_));
    k::DecodeMatvec(gu, stream_);
    if (probe_ev_) HIP_CHECK(hipEventRecord(probe_ev_[probe_i_++], stream_));
    k::DecodeMatvecArgs dn;
    dn.x = act_;
    dn.K = F;
    dn.job[0] = job(w.down, w.ddown, w.ddown.w != nullptr, x_);
    dn.epi = k::kAdd;
    k::DecodeMatvec(dn, stream_);
  }
  k::DecodeMatvecArgs lm;
  lm.x = x_;
  lm.K = H;
  lm.norm_w = m_.output_norm();
  lm.eps = c.rms_eps;
  lm.job[0] = job(m_.lm_head(), m_.lm_head_tiled(), m_.lm_head_tiled().w != nullptr, logits_);
  lm.inc = d_pos_;
  NormFirst(&lm);
  k::DecodeMatvec(lm, stream_);
}

// A decode matvec folds RMSNorm into its staging for inputs up to
// k::kDecodeNormMaxK; a wider hidden size is normed into h_ first.
void Session::NormFirst(k::DecodeMatvecArgs* a) {
  if (a->norm_w == nullptr || a->K <= k::kDecodeNormMaxK) return;
  k::RmsNormRows(a->x, a->K, a->norm_w, a->K, 1, a->eps, h_, a->K, stream_);
  a->x = h_;
  a->norm_w = nullptr;
}

// norm(x) -> act = silu(gate . x) * (up . x) of layer l, one decode token.
k::DecodeMatvecArgs Session::GateUpArgs(int l) const {
  const ModelConfig& c = m_.config();
  const LayerDev& w = m_.layers()[static_cast<size_t>(l)];
  k::DecodeMatvecArgs gu;
  gu.x = x_;
  gu.K = c.hidden;
  gu.norm_w = w.ffn_norm;
  gu.eps = c.rms_eps;
  gu.job[0].row_bytes = w.gate.row_bytes;
  gu.job[0].type = w.gate.type;
  gu.job[0].rows = w.gate.rows;
  gu.job[0].y = act_;
  if (w.gate_up.w != nullptr) {  // tile-major pair copy
    gu.job[0].w = w.gate_up.w;
    gu.job[0].tiled = 1;
    gu.job[0].pair = 1;
  } else {
    gu.job[0].w = w.gate.w;
    gu.job[0].w2 = w.up.w;
    gu.job[0].row_bytes2 = w.up.row_bytes;
    gu.job[0].type2 = w.up.type;
  }
  return gu;
}

// Algorithmic bytes of one decode gate+up launch: both weight matrices, the
// input, its norm gain and the output (every layer has the same shapes).
double Session::GateUpBytes() const {
  const ModelConfig& c = m_.config();
  const LayerDev& w = m_.layers()[0];
  return static_cast<double>(w.gate.row_bytes * w.gate.rows + w.up.row_bytes * w.up.rows) +
         4.0 * (2.0 * c.hidden + c.intermediate);
}

double Session::BenchGateUp(int layer, int iters, double* bytes) {
  const ModelConfig& c = m_.config();
  RPG_CHECK(layer >= 0 && layer < c.n_layers && iters > 0, "bench: bad layer or iteration count");
  EnsureScratch(1);
  *bytes = GateUpBytes();
  // launches walk the layers from `layer` on, so that no launch finds its
  // weights in the memory-side cache left by the previous one (36 layers of
  // 28 MB exceed it)
  k::DecodeMatvec(GateUpArgs(layer), stream_);  // warm
  HIP_CHECK(hipEventRecord(ev0_, stream_));
  for (int i = 0; i < iters; ++i) k::DecodeMatvec(GateUpArgs((layer + 1 + i) % c.n_layers), stream_);
  HIP_CHECK(hipEventRecord(ev1_, stream_));
  HIP_CHECK(hipEventSynchronize(ev1_));
  float ms = 0.0f;
  HIP_CHECK(hipEventElapsedTime(&ms, ev0_, ev1_));
  return 1e3 * static_cast<double>(ms) / iters;
}

double Session::InStepGateUp(int tokens, double* bytes) {
  const ModelConfig& c = m_.config();
  RPG_CHECK(tokens > 0 && len_ > 0 && len_ + tokens <= max_seq_,
            "bench: %d in-step tokens need a prefilled session with room for them (len %lld of %lld)", tokens,
            (long long)len_, (long long)max_seq_);
  EnsureScratch(1);
  *bytes = GateUpBytes();
  std::vector<hipEvent_t> ev(static_cast<size_t>(2) * c.n_layers * tokens, nullptr);
  struct Cleanup {
    Session* s;
    std::vector<hipEvent_t>& ev;
    ~Cleanup() {
      s->probe_ev_ = nullptr;
      for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    }
  } cleanup{this, ev};
  for (hipEvent_t& e : ev) HIP_CHECK(hipEventCreate(&e));
  h_pos_ = static_cast<int32_t>(len_);
  h_zero_ = 0;
  HIP_CHECK(hipMemcpyAsync(d_pos_, &h_pos_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(d_step_, &h_zero_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
  probe_ev_ = ev.data();
  probe_i_ = 0;
  for (int t = 0; t < tokens; ++t) {
    k::ArgMaxRows(logits_, c.vocab, c.vocab, 1, d_token_, stream_, d_pick_);
    DecodeForward();
  }
  probe_ev_ = nullptr;
  RPG_CHECK(probe_i_ == ev.size(), "bench: %zu of %zu probe events recorded", probe_i_, ev.size());
  HIP_CHECK(hipStreamSynchronize(stream_));
  len_ += tokens;
  double sum = 0.0;
  for (size_t i = 0; i < ev.size(); i += 2) {
    float ms = 0.0f;
    HIP_CHECK(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
    sum += ms;
  }
  return 1e3 * sum / static_cast<double>(ev.size() / 2);
}

void Session::CaptureDecode(bool greedy) {
  // the sampler's launches differ between the top-k and full-vocabulary draws
  const int mode = greedy ? 1 : sampler_->wide() ? 2 : 0;
  if (graph_exec_ && graph_mode_ == mode) return;
  if (graph_exec_) {
    HIP_CHECK(hipGraphExecDestroy(graph_exec_));
    HIP_CHECK(hipGraphDestroy(graph_));
    graph_exec_ = nullptr;
    graph_ = nullptr;
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
  try {
    EnqueueDecodeStep(greedy, false);
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream_, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  HIP_CHECK(hipStreamEndCapture(stream_, &graph_));
  HIP_CHECK(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
  graph_mode_ = mode;
}

std::vector<int32_t> Session::Generate(const float* first_logits_host, int32_t max_tokens, const SampleParams& sp,
                                       const std::vector<int32_t>& stop_ids, float* step_logits_host,
                                       const int32_t* force_host) {
  const ModelConfig& c = m_.config();
  RPG_CHECK(max_tokens > 0, "max_tokens must be positive (got %d)", max_tokens);
  EnsureScratch(1);
  std::unique_lock<std::mutex> persistent(g_persistent_mu, std::defer_lock);
  if (use_step_) persistent.lock();
  const bool forced = force_host != nullptr;
  if (forced) {
    RPG_CHECK(stop_ids.empty(), "forced decode takes no stop ids");
    RPG_CHECK(len_ + max_tokens <= max_seq_, "forced decode: %d tokens do not fit (len %lld of %lld)", max_tokens,
              (long long)len_, (long long)max_seq_);
    for (int32_t i = 0; i < max_tokens; ++i)
      RPG_CHECK(force_host[i] >= 0 && force_host[i] < c.vocab, "forced token %d has id %d, outside the vocabulary",
                i, force_host[i]);
    if (!d_force_) {
      DeviceAlloc(&d_force_, sizeof(int32_t) * static_cast<size_t>(max_seq_ + 1));
      DeviceAlloc(&d_drawn_, sizeof(int32_t) * static_cast<size_t>(max_seq_ + 1));
    }
    HIP_CHECK(hipMemcpyAsync(d_force_, force_host, sizeof(int32_t) * static_cast<size_t>(max_tokens),
                             hipMemcpyHostToDevice, stream_));
  }
  if (first_logits_host)
    HIP_CHECK(hipMemcpyAsync(logits_, first_logits_host, sizeof(float) * c.vocab, hipMemcpyHostToDevice, stream_));
  const bool greedy = !(sp.temperature > 0.0f);
  if (!greedy) {
    h_params_ = SamplerParamsDev{sp.temperature, sp.top_k, sp.top_p, 0, sp.seed};
    sampler_->SetParams(&h_params_, 1, stream_);
  }
  // forced steps are enqueued directly (the captured graph draws freely)
  const bool graph = use_graph_ && !forced;
  if (graph) CaptureDecode(greedy);
  h_pos_ = static_cast<int32_t>(len_);
  h_zero_ = 0;
  HIP_CHECK(hipMemcpyAsync(d_pos_, &h_pos_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(d_step_, &h_zero_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
  const int64_t capacity = max_seq_ - len_;
  const int64_t n_run = std::min<int64_t>(max_tokens, capacity);
  std::vector<int32_t> out;
  int64_t done = 0;
  int64_t returned = -1;
  HIP_CHECK(hipEventRecord(ev0_, stream_));
  while (done < n_run && returned < 0) {
    const int64_t step = step_logits_host ? 1 : (stop_ids.empty() ? n_run - done : std::min<int64_t>(kGenChunk, n_run - done));
    for (int64_t i = 0; i < step; ++i) {
      if (graph)
        HIP_CHECK(hipGraphLaunch(graph_exec_, stream_));
      else
        EnqueueDecodeStep(greedy, forced);
    }
    if (step_logits_host)
      HIP_CHECK(hipMemcpyAsync(step_logits_host + done * c.vocab, logits_, sizeof(float) * c.vocab,
                               hipMemcpyDeviceToHost, stream_));
    out.resize(static_cast<size_t>(done + step));
    // forced: the ids the sampler drew (the forwarded ones are the caller's)
    HIP_CHECK(hipMemcpyAsync(out.data() + done, (forced ? d_drawn_ : d_out_ids_) + done, sizeof(int32_t) * step,
                             hipMemcpyDeviceToHost, stream_));
    HIP_CHECK(hipStreamSynchronize(stream_));
    for (int64_t i = done; i < done + step && returned < 0; ++i) {
      if (std::find(stop_ids.begin(), stop_ids.end(), out[static_cast<size_t>(i)]) != stop_ids.end()) returned = i + 1;
    }
    done += step;
  }
  HIP_CHECK(hipEventRecord(ev1_, stream_));
  HIP_CHECK(hipEventSynchronize(ev1_));
  HIP_CHECK(hipEventElapsedTime(&last_decode_ms_, ev0_, ev1_));
  int32_t err = 0;
  HIP_CHECK(hipMemcpy(&err, d_err_, sizeof(int32_t), hipMemcpyDeviceToHost));
  RPG_CHECK(err == 0, "a device-side token id fell outside the vocabulary");
  if (use_step_) {
    HIP_CHECK(hipMemcpy(&err, d_step_err_, sizeof(int32_t), hipMemcpyDeviceToHost));
    if (err != 0) {
      use_step_ = false;  // later calls take the per-launch path
      Throw("decode step failed (code %d: %s)", err,
            err == 1 ? "a wait for a phase input gave up" : err == 2 ? "a stale residual" : "a token outside the vocabulary");
    }
  }
  if (returned < 0) returned = n_run;
  out.resize(static_cast<size_t>(returned));
  if (returned < done) {
    // Steps queued past the stop token already ran, so the device logits
    // belong to a later position. Forward the stop token again at its own
    // position: attention there reads only positions up to it, so the
    // logits come out as the step that forwarded it first left them, and a
    // continuation (first_logits == NULL) starts from the right row.
    h_token_ = out[static_cast<size_t>(returned - 1)];
    h_pos_ = static_cast<int32_t>(len_ + returned - 1);
    HIP_CHECK(hipMemcpyAsync(d_token_, &h_token_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
    HIP_CHECK(hipMemcpyAsync(d_pos_, &h_pos_, sizeof(int32_t), hipMemcpyHostToDevice, stream_));
    DecodeForward();
    HIP_CHECK(hipStreamSynchronize(stream_));
  }
  len_ += returned;
  // The reference appends a token and then finds the cache full
  // (reference src/qwen3.cc:341-344): same error once the capacity is used up.
  if (returned == n_run && n_run < max_tokens)
    Throw("context full (%lld positions, %lld tokens generated): use a larger max_seq or reset the session",
          (long long)max_seq_, (long long)returned + 1);
  return out;
}

void Session::ReadKv(int which, int layer, int head, int64_t n, float* out) const {
  const ModelConfig& c = m_.config();
  RPG_CHECK(layer >= 0 && layer < c.n_layers && head >= 0 && head < c.n_kv_heads && n >= 0 && n <= max_seq_,
            "KV read out of range");
  const float* base = (which == 0 ? kcache_ : vcache_) +
                      ((static_cast<int64_t>(layer) * c.n_kv_heads + head) * max_seq_) * c.head_dim;
  HIP_CHECK(hipMemcpy(out, base, sizeof(float) * static_cast<size_t>(n) * c.head_dim, hipMemcpyDeviceToHost));
}

}  // namespace rpg
