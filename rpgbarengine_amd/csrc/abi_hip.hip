// extern "C" token-level and kernel-level entry points (include/rpg_hip.h).

#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "batch.h"
#include "common.h"
#include "decode.h"
#include "expf_glibc.h"
#include "kernels.h"
#include "model.h"
#include "prefill.h"
#include "rpg_hip.h"
#include "sampler.h"
#include "session.h"

namespace rpg {
namespace {

std::mutex g_mu;
std::map<int32_t, std::shared_ptr<DeviceModel>> g_models;
struct SessEntry {
  std::shared_ptr<DeviceModel> model;  // keeps the model alive
  std::unique_ptr<Session> s;
};
std::map<int32_t, std::shared_ptr<SessEntry>> g_sessions;
int32_t g_next_model = 1, g_next_session = 1;
std::atomic<int64_t> g_sampler_fallbacks{0};
std::atomic<int64_t> g_sampler_tie_orders{0};

template <typename F>
auto Guard(F&& f, decltype(f()) fail) -> decltype(f()) {
  try {
    SetLastError("");
    return f();
  } catch (const std::exception& e) {
    SetLastError(e.what());
    return fail;
  } catch (...) {
    SetLastError("unknown exception");
    return fail;
  }
}

std::shared_ptr<DeviceModel> RequireModel(int32_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_models.find(h);
  RPG_CHECK(it != g_models.end(), "invalid model handle %d", h);
  return it->second;
}

std::shared_ptr<SessEntry> RequireSession(int32_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_sessions.find(h);
  RPG_CHECK(it != g_sessions.end(), "invalid session handle %d", h);
  return it->second;
}

void RequireGpu() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    Throw("no GPU is visible: the HIP engine needs an MI355X (gfx950)");
  }
}

// RAII device buffer for the host-buffer entry points.
struct DevBuf {
  void* p = nullptr;
  explicit DevBuf(size_t n) { DeviceAlloc(&p, n ? n : 1); }
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

__global__ void ExpfKernel(const float* x, int64_t n, float* out) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) out[i] = GlibcExpf(x[i]);
}

// Plain copy of n 16-byte words, grid-stride: the stream bandwidth probe and
// the calibration kernel of the byte counters.
__global__ __launch_bounds__(256) void CopyKernel(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

k::MatRef HostMat(uint32_t type, const uint8_t* w_dev, int64_t rows, int64_t cols) {
  k::MatRef r;
  r.w = w_dev;
  r.type = type;
  r.rows = static_cast<int32_t>(rows);
  r.cols = static_cast<int32_t>(cols);
  r.row_bytes = RowBytes(type, cols);
  return r;
}

// Y = X . W^T the way the engine runs a projection of n tokens: up to
// FewTokenLimit() through the decode matvecs on the tile-major copy when
// there is one, more through the matrix-core GEMM when the weight type has
// one (split buffer: k::SplitXBytes(n, cols, rows) bytes).
void Project(const k::MatRef& m, const float* X, int n, float* Y, void* split, hipStream_t s,
             const uint8_t* tiled = nullptr) {
  if (n == 1 && tiled != nullptr) {  // the decode step's path: the tile-major copy
    k::DecodeMatvecArgs a;
    a.x = X;
    a.K = m.cols;
    a.job[0].w = tiled;
    a.job[0].tiled = 1;
    a.job[0].row_bytes = m.row_bytes;
    a.job[0].type = m.type;
    a.job[0].rows = m.rows;
    a.job[0].y = Y;
    k::DecodeMatvec(a, s);
  } else if (n <= k::FewTokenLimit() && tiled != nullptr) {  // a few tokens: the batch matvec
    k::DecodeBatchArgs a;
    a.x = X;
    a.ldx = m.cols;
    a.T = n;
    a.K = m.cols;
    a.job[0].w = tiled;
    a.job[0].tiled = 1;
    a.job[0].row_bytes = m.row_bytes;
    a.job[0].type = m.type;
    a.job[0].rows = m.rows;
    a.job[0].y = Y;
    a.ldy[0] = m.rows;
    RPG_CHECK(k::DecodeMatvecBatch(a, s), "matmul: the batch matvec refused %d tokens", n);
  } else if (n >= 2 && k::QGemmSupports(m)) {
    const k::SplitX sx = k::SplitXView(split, n, m.cols, static_cast<int>(m.rows));
    k::SplitRows(X, m.cols, n, m.cols, nullptr, 0.0f, sx, s);
    k::GemmJob job;
    job.w = m;
    job.y = Y;
    job.ldy = m.rows;
    k::QGemm(sx, &job, 1, s);
  } else {
    k::Matvec(m, X, m.cols, n, Y, m.rows, k::kStore, s);
  }
}

}  // namespace
}  // namespace rpg

using namespace rpg;

extern "C" {

const char* rpg_hip_last_error(void) { return LastError(); }

int32_t rpg_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int32_t rpg_hip_model_load(const char* path, int32_t max_pos) {
  return Guard([&]() -> int32_t {
    RPG_CHECK(path && *path, "empty model path");
    RPG_CHECK(max_pos > 0, "max_pos must be positive");
    RequireGpu();
    std::shared_ptr<DeviceModel> m(DeviceModel::Load(path, max_pos).release());
    std::lock_guard<std::mutex> lk(g_mu);
    const int32_t h = g_next_model++;
    g_models[h] = m;
    return h;
  }, -1);
}

void rpg_hip_model_free(int32_t model) {
  Guard([&]() -> int32_t {
    std::lock_guard<std::mutex> lk(g_mu);
    g_models.erase(model);
    return 0;
  }, -1);
}

int32_t rpg_hip_model_config(int32_t model, int32_t* out) {
  return Guard([&]() -> int32_t {
    const ModelConfig& c = RequireModel(model)->config();
    const int32_t v[9] = {c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.intermediate, c.vocab,
                          c.context_length, c.eos_id};
    for (int i = 0; i < 9; ++i) out[i] = v[i];
    return 0;
  }, -1);
}

int64_t rpg_hip_model_decode_bytes(int32_t model) {
  return Guard([&]() -> int64_t { return RequireModel(model)->decode_weight_bytes(); }, int64_t(-1));
}

int32_t rpg_hip_model_rope_row(int32_t model, int64_t pos, float* out) {
  return Guard([&]() -> int32_t {
    auto m = RequireModel(model);
    RPG_CHECK(pos >= 0 && pos < m->rope_positions(), "position %lld outside the RoPE table", (long long)pos);
    const int hd = m->config().head_dim;
    for (int i = 0; i < hd; ++i) out[i] = m->rope_host()[static_cast<size_t>(pos * hd + i)];
    return 0;
  }, -1);
}

int32_t rpg_hip_session_new(int32_t model, int64_t max_seq) {
  return Guard([&]() -> int32_t {
    auto m = RequireModel(model);
    auto e = std::make_shared<SessEntry>();
    e->model = m;
    e->s.reset(new Session(*m, max_seq));
    std::lock_guard<std::mutex> lk(g_mu);
    const int32_t h = g_next_session++;
    g_sessions[h] = e;
    return h;
  }, -1);
}

void rpg_hip_session_free(int32_t session) {
  Guard([&]() -> int32_t {
    std::lock_guard<std::mutex> lk(g_mu);
    g_sessions.erase(session);
    return 0;
  }, -1);
}

int64_t rpg_hip_session_len(int32_t session) {
  return Guard([&]() -> int64_t { return RequireSession(session)->s->len(); }, int64_t(-1));
}

int32_t rpg_hip_session_set_len(int32_t session, int64_t len) {
  return Guard([&]() -> int32_t {
    RequireSession(session)->s->SetLen(len);
    return 0;
  }, -1);
}

int32_t rpg_hip_prefill(int32_t session, const int32_t* ids, int64_t n, float* last_logits, float* all_logits) {
  return Guard([&]() -> int32_t {
    RequireSession(session)->s->Prefill(ids, n, last_logits, all_logits);
    return 0;
  }, -1);
}

int32_t rpg_hip_generate(int32_t session, const float* first_logits, int32_t max_tokens, float temperature,
                         int32_t top_k, float top_p, uint64_t seed, const int32_t* stop_ids, int32_t n_stop,
                         int32_t* out_ids, float* step_logits) {
  return Guard([&]() -> int32_t {
    auto e = RequireSession(session);
    SampleParams sp;
    sp.temperature = temperature;
    sp.top_k = top_k;
    sp.top_p = top_p;
    sp.seed = seed;
    std::vector<int32_t> stops(stop_ids, stop_ids + (n_stop > 0 ? n_stop : 0));
    const std::vector<int32_t> out = e->s->Generate(first_logits, max_tokens, sp, stops, step_logits);
    for (size_t i = 0; i < out.size(); ++i) out_ids[i] = out[i];
    return static_cast<int32_t>(out.size());
  }, -1);
}

int32_t rpg_hip_generate_batch(const int32_t* sessions, int32_t n, int32_t max_tokens, const float* temperature,
                               const int32_t* top_k, const float* top_p, const uint64_t* seed, int32_t* out_ids,
                               float* step_logits, double* decode_ms) {
  return Guard([&]() -> int32_t {
    RPG_CHECK(sessions != nullptr && out_ids != nullptr && temperature != nullptr && top_k != nullptr &&
                  top_p != nullptr && seed != nullptr,
              "generate_batch: null argument");
    RPG_CHECK(n >= 1 && n <= k::kMaxDecodeBatch, "generate_batch: %d sessions outside [1, %d]", n,
              k::kMaxDecodeBatch);
    std::vector<std::shared_ptr<SessEntry>> keep;
    std::vector<Session*> ss;
    std::vector<SampleParams> ps;
    for (int32_t i = 0; i < n; ++i) {
      keep.push_back(RequireSession(sessions[i]));
      RPG_CHECK(keep.back()->model == keep.front()->model, "generate_batch: sessions of different models");
      ss.push_back(keep.back()->s.get());
      SampleParams sp;
      sp.temperature = temperature[i];
      sp.top_k = top_k[i];
      sp.top_p = top_p[i];
      sp.seed = seed[i];
      ps.push_back(sp);
    }
    SessionBatch batch(*keep.front()->model, ss);
    batch.Generate(max_tokens, ps, out_ids, step_logits);
    if (decode_ms != nullptr) *decode_ms = batch.last_decode_ms();
    return max_tokens;
  }, -1);
}

int32_t rpg_hip_generate_forced(int32_t session, const float* first_logits, int32_t max_tokens, float temperature,
                                int32_t top_k, float top_p, uint64_t seed, const int32_t* force_ids,
                                int32_t* drawn_ids, float* step_logits) {
  return Guard([&]() -> int32_t {
    RPG_CHECK(force_ids != nullptr && drawn_ids != nullptr, "generate_forced: null argument");
    auto e = RequireSession(session);
    SampleParams sp;
    sp.temperature = temperature;
    sp.top_k = top_k;
    sp.top_p = top_p;
    sp.seed = seed;
    const std::vector<int32_t> out = e->s->Generate(first_logits, max_tokens, sp, {}, step_logits, force_ids);
    for (size_t i = 0; i < out.size(); ++i) drawn_ids[i] = out[i];
    return static_cast<int32_t>(out.size());
  }, -1);
}

int32_t rpg_hip_generate_batch_forced(const int32_t* sessions, int32_t n, int32_t max_tokens,
                                      const float* temperature, const int32_t* top_k, const float* top_p,
                                      const uint64_t* seed, const int32_t* force_ids, int32_t* drawn_ids,
                                      float* step_logits) {
  return Guard([&]() -> int32_t {
    RPG_CHECK(sessions != nullptr && force_ids != nullptr && drawn_ids != nullptr && temperature != nullptr &&
                  top_k != nullptr && top_p != nullptr && seed != nullptr,
              "generate_batch_forced: null argument");
    RPG_CHECK(n >= 1 && n <= k::kMaxDecodeBatch, "generate_batch_forced: %d sessions outside [1, %d]", n,
              k::kMaxDecodeBatch);
    std::vector<std::shared_ptr<SessEntry>> keep;
    std::vector<Session*> ss;
    std::vector<SampleParams> ps;
    for (int32_t i = 0; i < n; ++i) {
      keep.push_back(RequireSession(sessions[i]));
      RPG_CHECK(keep.back()->model == keep.front()->model, "generate_batch_forced: sessions of different models");
      ss.push_back(keep.back()->s.get());
      SampleParams sp;
      sp.temperature = temperature[i];
      sp.top_k = top_k[i];
      sp.top_p = top_p[i];
      sp.seed = seed[i];
      ps.push_back(sp);
    }
    SessionBatch batch(*keep.front()->model, ss);
    batch.Generate(max_tokens, ps, drawn_ids, step_logits, force_ids);
    return max_tokens;
  }, -1);
}

int32_t rpg_hip_fail_alloc_after(int64_t n) {
  FailDeviceAllocAfter(n);
  return 0;
}

int32_t rpg_hip_session_decode_path(int32_t session) {
  return Guard([&]() -> int32_t { return RequireSession(session)->s->uses_step() ? 1 : 0; }, -1);
}

int32_t rpg_hip_kv_read(int32_t session, int32_t which, int32_t layer, int32_t head, int64_t n, float* out) {
  return Guard([&]() -> int32_t {
    RequireSession(session)->s->ReadKv(which, layer, head, n, out);
    return 0;
  }, -1);
}

int32_t rpg_hip_session_timing(int32_t session, double* prefill_ms, double* decode_ms) {
  return Guard([&]() -> int32_t {
    auto e = RequireSession(session);
    if (prefill_ms) *prefill_ms = e->s->last_prefill_ms();
    if (decode_ms) *decode_ms = e->s->last_decode_ms();
    return 0;
  }, -1);
}

int32_t rpg_hip_bench_copy(int64_t bytes, int32_t iters, double* us) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(bytes >= 16 && bytes % 16 == 0 && iters > 0, "copy bench: bytes must be a positive multiple of 16");
    DevBuf a(static_cast<size_t>(bytes)), b(static_cast<size_t>(bytes));
    HIP_CHECK(hipMemset(a.p, 1, static_cast<size_t>(bytes)));
    const int64_t n = bytes / 16;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(CeilDiv(n, 256), 8192));
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    hipLaunchKernelGGL(CopyKernel, dim3(grid), dim3(256), 0, nullptr, a.as<uint4>(), b.as<uint4>(), n);
    HIP_CHECK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i)
      hipLaunchKernelGGL(CopyKernel, dim3(grid), dim3(256), 0, nullptr, (i & 1) ? b.as<uint4>() : a.as<uint4>(),
                         (i & 1) ? a.as<uint4>() : b.as<uint4>(), n);
    HIP_CHECK(hipEventRecord(e1, nullptr));
    HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    *us = 1e3 * static_cast<double>(ms) / iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
  }, -1);
}

int32_t rpg_hip_session_bench_gate_up(int32_t session, int32_t layer, int32_t iters, double* out) {
  return Guard([&]() -> int32_t {
    auto e = RequireSession(session);
    double bytes = 0.0;
    out[0] = e->s->BenchGateUp(layer, iters, &bytes);
    out[1] = bytes;
    return 0;
  }, -1);
}

int32_t rpg_hip_session_instep_gate_up(int32_t session, int32_t tokens, double* out) {
  return Guard([&]() -> int32_t {
    auto e = RequireSession(session);
    double bytes = 0.0;
    out[0] = e->s->InStepGateUp(tokens, &bytes);
    out[1] = bytes;
    return 0;
  }, -1);
}

int32_t rpg_hip_dequant(uint32_t type, const uint8_t* src, int64_t n, float* dst) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    const int64_t bytes = RowBytes(type, n);
    DevBuf s(static_cast<size_t>(bytes) + 256), d(static_cast<size_t>(n) * 4);
    HIP_CHECK(hipMemcpy(s.p, src, static_cast<size_t>(bytes), hipMemcpyHostToDevice));
    k::Dequant(type, s.as<uint8_t>(), n, d.as<float>(), nullptr);
    HIP_CHECK(hipMemcpy(dst, d.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost));
    return 0;
  }, -1);
}

int32_t rpg_hip_matmul(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const float* X, int64_t n,
                       float* Y) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(rows > 0 && cols > 0 && n > 0, "matmul: empty shape");
    const k::MatRef probe = HostMat(type, nullptr, rows, cols);
    const size_t wb = static_cast<size_t>(probe.row_bytes * rows);
    DevBuf dw(wb + 256), dx(static_cast<size_t>(n * cols) * 4), dy(static_cast<size_t>(n * rows) * 4);
    HIP_CHECK(hipMemcpy(dw.p, w, wb, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dx.p, X, static_cast<size_t>(n * cols) * 4, hipMemcpyHostToDevice));
    const k::MatRef m = HostMat(type, dw.as<uint8_t>(), rows, cols);
    DevBuf split(k::SplitXBytes(static_cast<int>(n), static_cast<int>(cols), static_cast<int>(rows)));
    const bool tile = n == 1 ? k::DecodeTileable(m) : n <= k::FewTokenLimit() && k::BatchTileable(m);
    DevBuf tiled(tile ? static_cast<size_t>(k::TileMajorBytes(m, false)) : 16);
    if (tile) k::TileMajor(m, nullptr, tiled.as<uint8_t>(), nullptr);
    Project(m, dx.as<float>(), static_cast<int>(n), dy.as<float>(), split.p, nullptr,
            tile ? tiled.as<uint8_t>() : nullptr);
    HIP_CHECK(hipMemcpy(Y, dy.p, static_cast<size_t>(n * rows) * 4, hipMemcpyDeviceToHost));
    return 0;
  }, -1);
}

int32_t rpg_hip_matvec_few(uint32_t type, const uint8_t* w, const uint8_t* up, int64_t rows, int64_t cols,
                           const float* X, int64_t n, const float* norm_w, float eps, int32_t add, float* Y) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(rows > 0 && cols > 0 && n >= 1 && n <= k::kMaxBatchTokens, "matvec_few: shape");
    RPG_CHECK(!(add && up), "matvec_few: a SwiGLU pair stores");
    const k::MatRef probe = HostMat(type, nullptr, rows, cols);
    RPG_CHECK(k::BatchTileable(probe), "matvec_few: no tile-major copy for this type and width");
    const size_t wb = static_cast<size_t>(probe.row_bytes * rows);
    const size_t yb = static_cast<size_t>(n * rows) * 4, xb = static_cast<size_t>(n * cols) * 4;
    DevBuf dw(wb + 256), du(up ? wb + 256 : 16), dx(xb), dy(yb), dn(norm_w ? static_cast<size_t>(cols) * 4 : 16);
    HIP_CHECK(hipMemcpy(dw.p, w, wb, hipMemcpyHostToDevice));
    if (up) HIP_CHECK(hipMemcpy(du.p, up, wb, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dx.p, X, xb, hipMemcpyHostToDevice));
    if (norm_w) HIP_CHECK(hipMemcpy(dn.p, norm_w, static_cast<size_t>(cols) * 4, hipMemcpyHostToDevice));
    if (add) HIP_CHECK(hipMemcpy(dy.p, Y, yb, hipMemcpyHostToDevice));
    const k::MatRef m = HostMat(type, dw.as<uint8_t>(), rows, cols);
    const k::MatRef mu = HostMat(type, du.as<uint8_t>(), rows, cols);
    DevBuf tiled(static_cast<size_t>(k::TileMajorBytes(m, up != nullptr)));
    k::TileMajor(m, up ? &mu : nullptr, tiled.as<uint8_t>(), nullptr);
    k::DecodeBatchArgs a;
    a.x = dx.as<float>();
    a.ldx = cols;
    a.T = static_cast<int32_t>(n);
    a.K = static_cast<int32_t>(cols);
    a.norm_w = norm_w ? dn.as<float>() : nullptr;
    a.eps = eps;
    a.epi = add ? k::kAdd : k::kStore;
    a.job[0].w = tiled.as<uint8_t>();
    a.job[0].tiled = 1;
    a.job[0].pair = up ? 1 : 0;
    a.job[0].row_bytes = m.row_bytes;
    a.job[0].type = type;
    a.job[0].rows = static_cast<int32_t>(rows);
    a.job[0].y = dy.as<float>();
    a.ldy[0] = rows;
    RPG_CHECK(k::DecodeMatvecBatch(a, nullptr), "matvec_few: the launch does not qualify");
    HIP_CHECK(hipMemcpy(Y, dy.p, yb, hipMemcpyDeviceToHost));
    return 0;
  }, -1);
}

int32_t rpg_hip_matmul_swiglu(uint32_t type, const uint8_t* gate, const uint8_t* up, int64_t rows, int64_t cols,
                              const float* X, int64_t n, float* Y) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(rows > 0 && cols > 0 && n >= 2, "matmul_swiglu: shape");
    const k::MatRef probe = HostMat(type, nullptr, rows, cols);
    RPG_CHECK(k::QGemmSupports(probe), "matmul_swiglu: no GEMM for this type and width");
    const size_t wb = static_cast<size_t>(probe.row_bytes * rows);
    DevBuf dg(wb + 256), du(wb + 256), dx(static_cast<size_t>(n * cols) * 4), dy(static_cast<size_t>(n * rows) * 4);
    HIP_CHECK(hipMemcpy(dg.p, gate, wb, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(du.p, up, wb, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dx.p, X, static_cast<size_t>(n * cols) * 4, hipMemcpyHostToDevice));
    DevBuf split(k::SplitXBytes(static_cast<int>(n), static_cast<int>(cols), static_cast<int>(2 * rows)));
    const k::SplitX sx = k::SplitXView(split.p, static_cast<int>(n), static_cast<int>(cols), static_cast<int>(2 * rows));
    k::SplitRows(dx.as<float>(), cols, static_cast<int>(n), static_cast<int>(cols), nullptr, 0.0f, sx, nullptr);
    k::GemmJob g, u;
    g.w = HostMat(type, dg.as<uint8_t>(), rows, cols);
    g.y = dy.as<float>();
    g.ldy = rows;
    u.w = HostMat(type, du.as<uint8_t>(), rows, cols);
    const bool fused = k::QGemmSwiGLU(sx, g, u, nullptr);
    if (!fused) {
      DevBuf gu(static_cast<size_t>(2 * n * rows) * 4);
      k::GemmJob both[2] = {g, u};
      both[0].y = gu.as<float>();
      both[1].y = gu.as<float>() + n * rows;
      both[1].ldy = rows;
      k::QGemm(sx, both, 2, nullptr);
      k::SwiGLURows(both[0].y, both[1].y, dy.as<float>(), n * rows, nullptr);
      HIP_CHECK(hipDeviceSynchronize());
    }
    HIP_CHECK(hipMemcpy(Y, dy.p, static_cast<size_t>(n * rows) * 4, hipMemcpyDeviceToHost));
    return fused ? 1 : 0;
  }, -1);
}

int32_t rpg_hip_sample(const float* logits, int32_t n, float temperature, int32_t top_k, float top_p, uint64_t seed,
                       int64_t counter, float* probs) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(n > 0, "sample: empty logits");
    DevBuf dl(static_cast<size_t>(n) * 4), dp(static_cast<size_t>(n) * 4), dt(4);
    HIP_CHECK(hipMemcpy(dl.p, logits, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice));
    Sampler sm(1, n);
    const SamplerParamsDev p{temperature, top_k, top_p, 0, seed};
    sm.SetParams(&p, 1, nullptr);
    sm.Enqueue(dl.as<float>(), n, nullptr, counter, dt.as<int32_t>(), probs ? dp.as<float>() : nullptr, nullptr);
    int32_t tok = -1;
    HIP_CHECK(hipMemcpy(&tok, dt.p, 4, hipMemcpyDeviceToHost));
    if (probs) HIP_CHECK(hipMemcpy(probs, dp.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost));
    g_sampler_fallbacks += sm.FallbackCount(nullptr, 0);
    g_sampler_tie_orders += sm.FallbackCount(nullptr, 1);
    RPG_CHECK(sm.FallbackCount(nullptr, 2) == 0, "sample: the top-p tie-order replay was refused");
    return tok;
  }, -1);
}

int64_t rpg_hip_sampler_fallbacks(void) { return g_sampler_fallbacks.load(); }

int64_t rpg_hip_sampler_tie_orders(void) { return g_sampler_tie_orders.load(); }

int32_t rpg_hip_attention(const float* q, const float* k, const float* v, int32_t seq, int32_t n_heads, int32_t n_kv,
                          int32_t pos0, float* out) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(seq > 0 && pos0 >= 0 && n_kv > 0 && n_heads > 0 && n_heads % n_kv == 0, "attention: bad shape");
    const int64_t n_pos = static_cast<int64_t>(pos0) + seq;
    const size_t qb = static_cast<size_t>(seq) * n_heads * 128 * 4, cb = static_cast<size_t>(n_kv) * n_pos * 128 * 4;
    DevBuf dq(qb), dk(cb), dv(cb), dout(qb);
    HIP_CHECK(hipMemcpy(dq.p, q, qb, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dk.p, k, cb, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dv.p, v, cb, hipMemcpyHostToDevice));
    k::AttnArgs a{};
    a.q = dq.as<float>();
    a.kcache = dk.as<float>();
    a.vcache = dv.as<float>();
    a.out = dout.as<float>();
    a.seq = seq;
    a.n_heads = n_heads;
    a.n_kv = n_kv;
    a.hd = 128;
    a.max_seq = n_pos;
    a.pos0_host = pos0;
    RPG_CHECK(seq > 1, "attention: the segment kernel takes seq >= 2");
    k::Attention(a, nullptr);
    HIP_CHECK(hipMemcpy(out, dout.p, qb, hipMemcpyDeviceToHost));
    return 0;
  }, -1);
}

int32_t rpg_hip_expf(const float* x, int64_t n, float* out) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    DevBuf dx(static_cast<size_t>(n) * 4), dy(static_cast<size_t>(n) * 4);
    HIP_CHECK(hipMemcpy(dx.p, x, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(ExpfKernel, dim3(static_cast<unsigned>(CeilDiv(n, 256))), dim3(256), 0, nullptr,
                       dx.as<float>(), n, dy.as<float>());
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipMemcpy(out, dy.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost));
    return 0;
  }, -1);
}

int32_t rpg_hip_bench_matmul(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const int32_t* ns,
                             int32_t n_count, int32_t copies, int32_t iters, double* out) {
  return Guard([&]() -> int32_t {
    RequireGpu();
    RPG_CHECK(copies > 0 && iters > 0 && n_count > 0, "bench: bad arguments");
    int32_t n_max = 0;
    for (int i = 0; i < n_count; ++i) {
      RPG_CHECK(ns[i] > 0, "bench: token count %d", ns[i]);
      n_max = std::max(n_max, ns[i]);
    }
    const k::MatRef probe = HostMat(type, nullptr, rows, cols);
    const size_t wb = static_cast<size_t>(probe.row_bytes * rows);
    const size_t stride = (wb + 255) / 256 * 256;
    DevBuf dw(stride * static_cast<size_t>(copies) + 256), dx(static_cast<size_t>(n_max * cols) * 4),
        dy(static_cast<size_t>(n_max * rows) * 4);
    hipStream_t s;
    HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    HIP_CHECK(hipMemcpy(dw.p, w, wb, hipMemcpyHostToDevice));
    for (int c = 1; c < copies; ++c)
      HIP_CHECK(hipMemcpyAsync(dw.as<uint8_t>() + stride * c, dw.p, wb, hipMemcpyDeviceToDevice, s));
    std::vector<float> xh(static_cast<size_t>(n_max * cols));
    for (size_t i = 0; i < xh.size(); ++i) xh[i] = static_cast<float>((i * 2654435761u) % 1000) * 1e-3f - 0.5f;
    HIP_CHECK(hipMemcpy(dx.p, xh.data(), xh.size() * 4, hipMemcpyHostToDevice));
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    DevBuf split(k::SplitXBytes(n_max, static_cast<int>(cols), static_cast<int>(rows)));
    // a few tokens: time the decode paths, on tile-major copies
    bool want_tile = false;
    for (int i = 0; i < n_count; ++i) want_tile = want_tile || ns[i] <= k::FewTokenLimit();
    const bool tile = want_tile && k::DecodeTileable(probe);
    const size_t tstride = tile ? (static_cast<size_t>(k::TileMajorBytes(probe, false)) + 255) / 256 * 256 : 0;
    DevBuf tiled(tile ? tstride * static_cast<size_t>(copies) : 16);
    for (int c = 0; tile && c < copies; ++c)
      k::TileMajor(HostMat(type, dw.as<uint8_t>() + stride * c, rows, cols), nullptr, tiled.as<uint8_t>() + tstride * c,
                   s);
    for (int q = 0; q < n_count; ++q) {
      const int n = ns[q];
      auto run = [&](int i) {
        const k::MatRef m = HostMat(type, dw.as<uint8_t>() + stride * (i % copies), rows, cols);
        const bool use_tile = tile && (n == 1 || (n <= k::FewTokenLimit() && k::BatchTileable(probe)));
        Project(m, dx.as<float>(), n, dy.as<float>(), split.p, s,
                use_tile ? tiled.as<uint8_t>() + tstride * (i % copies) : nullptr);
      };
      for (int i = 0; i < std::min(copies, 4); ++i) run(i);  // warm-up
      HIP_CHECK(hipEventRecord(e0, s));
      for (int i = 0; i < iters; ++i) run(i);
      HIP_CHECK(hipEventRecord(e1, s));
      HIP_CHECK(hipEventSynchronize(e1));
      float ms = 0.0f;
      HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
      out[q] = static_cast<double>(ms) / iters;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(s);
    return 0;
  }, -1);
}

}  // extern "C"
