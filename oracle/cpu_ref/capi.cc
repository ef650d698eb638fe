// C entry points of liboracle.so, for ctypes in tests/ and bench.py's CPU
// baseline leg. Test infrastructure only.

#include <chrono>
#include <cmath>

#include "oracle.h"

namespace {
thread_local std::string g_err;

template <typename F>
int32_t Guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}
}  // namespace

extern "C" {

const char* orc_last_error(void) { return g_err.c_str(); }

int32_t orc_dequant(uint32_t type, const uint8_t* src, int64_t n, float* dst) {
  return Guard([&] { orc::DequantizeRow(type, src, n, dst); });
}

int32_t orc_scale_min_k4(int32_t j, const uint8_t* q, uint8_t* sc, uint8_t* mn) {
  return Guard([&] { orc::ScaleMinK4(j, q, sc, mn); });
}

float orc_half_to_float(uint16_t h) { return orc::HalfToFloat(h); }

// One dot per row of `w` (rows x k) against the activation vector `a`.
// which: 0 = dispatched (AVX2 when available), 1 = scalar reference, 2 = AVX2.
int32_t orc_dot_rows(int32_t which, uint32_t type, const float* a, const uint8_t* w, int64_t k,
                     int64_t rows, float* out) {
  return Guard([&] {
    const int64_t rb = orc::RowBytes(type, k);
    for (int64_t r = 0; r < rows; ++r) {
      const uint8_t* wr = w + r * rb;
      out[r] = which == 1 ? orc::DotRowScalar(type, a, wr, k)
               : which == 2 ? orc::DotRowAvx2(type, a, wr, k)
                            : orc::DotRowQuant(type, a, wr, k);
    }
  });
}

int32_t orc_avx2_available(void) { return orc::Avx2Available() ? 1 : 0; }

// OUT[t*rows + r] = X[t] . W[r], dispatched as QuantMatrix::MatMulBatch.
int32_t orc_matmul_batch(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const float* X,
                         int64_t n, float* OUT, int32_t threads) {
  return Guard([&] {
    orc::Matrix m;
    m.data = w;
    m.type = type;
    m.rows = rows;
    m.cols = cols;
    orc::Pool pool(threads > 0 ? threads : 1);
    m.MatMulBatch(X, n, OUT, &pool);
  });
}

void orc_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* out) {
  orc::RmsNorm(x, w, n, eps, out);
}
void orc_softmax(float* x, int64_t n) { orc::SoftmaxInPlace(x, n); }
void orc_silu(float* x, int64_t n) { orc::SiluInPlace(x, n); }
void orc_rope(float* x, int32_t heads, int32_t hd, const float* c, const float* s) {
  orc::RopeInPlace(x, heads, hd, c, s);
}
int32_t orc_argmax(const float* x, int64_t n) { return orc::ArgMax(x, n); }
float orc_dot(const float* a, const float* b, int64_t n) { return orc::Dot(a, b, n); }
float orc_expf(float x) { return std::exp(x); }
// glibc expf over an array (the GPU expf parity test compares every output)
void orc_expf_n(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = std::exp(x[i]);
}
int32_t orc_attention(const float* q, const float* k, const float* v, int32_t seq, int32_t n_heads, int32_t n_kv,
                      int32_t hd, int32_t pos0, float* out) {
  return Guard([&] { orc::AttentionCache(n_heads, n_kv, hd, q, seq, pos0, k, v, out); });
}

uint64_t orc_splitmix64(uint64_t x) { return orc::SplitMix64(x); }
float orc_counter_uniform(uint64_t seed, uint64_t counter) { return orc::CounterUniform(seed, counter); }

int32_t orc_filter_to_probs(const float* logits, int64_t n, float temperature, int32_t top_k,
                            float top_p, float* probs) {
  return Guard([&] {
    orc::SampleOptions o;
    o.temperature = temperature;
    o.top_k = top_k;
    o.top_p = top_p;
    std::vector<float> p;
    orc::FilterToProbs(logits, n, o, &p);
    std::memcpy(probs, p.data(), static_cast<size_t>(n) * sizeof(float));
  });
}

int32_t orc_sample_token(const float* logits, int64_t n, float temperature, int32_t top_k,
                         float top_p, float u) {
  orc::SampleOptions o;
  o.temperature = temperature;
  o.top_k = top_k;
  o.top_p = top_p;
  try {
    return orc::SampleToken(logits, n, o, u);
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// ---- model / cache / forward / generate
// max_pos: the positions of the RoPE table (the reference's load option
// "max_pos", src/engine.cc config; at most the model's context length)
void* orc_model_load(const char* path, int32_t threads, int32_t max_pos) {
  try {
    return orc::Model::Load(path, threads, max_pos).release();
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}
void orc_model_free(void* m) { delete static_cast<orc::Model*>(m); }

// out: n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab,
//      context_length, eos_id
void orc_model_config(void* mp, int32_t* out) {
  const orc::Config& c = static_cast<orc::Model*>(mp)->config();
  out[0] = c.n_layers; out[1] = c.hidden; out[2] = c.n_heads; out[3] = c.n_kv_heads;
  out[4] = c.head_dim; out[5] = c.intermediate; out[6] = c.vocab; out[7] = c.context_length;
  out[8] = c.eos_id;
}

int32_t orc_rope_row(void* mp, int64_t pos, float* out) {
  return Guard([&] {
    const orc::Model& m = *static_cast<orc::Model*>(mp);
    ORC_CHECK(pos >= 0 && pos < m.rope_positions(), "pos out of range");
    std::memcpy(out, m.rope_cos(pos), static_cast<size_t>(m.config().head_dim) * sizeof(float));
  });
}

void* orc_kv_new(void* mp, int64_t max_seq) {
  try {
    return new orc::KvCache(static_cast<orc::Model*>(mp)->config(), max_seq);
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}
void orc_kv_free(void* kv) { delete static_cast<orc::KvCache*>(kv); }
// measurement only: K / V rounded to fp16 on write (KvCache::fp16)
void orc_kv_set_fp16(void* kv, int32_t on) { static_cast<orc::KvCache*>(kv)->fp16 = on != 0; }
void orc_round_half_n(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc::RoundToHalf(x[i]);
}
int64_t orc_kv_len(void* kv) { return static_cast<orc::KvCache*>(kv)->len; }
// Copy K (which=0) or V (which=1) of (layer, kv_head, positions [0, n)) out.
int32_t orc_kv_read(void* kvp, int32_t which, int32_t layer, int32_t head, int64_t n, float* out) {
  return Guard([&] {
    orc::KvCache& kv = *static_cast<orc::KvCache*>(kvp);
    ORC_CHECK(n <= kv.max_seq, "n beyond capacity");
    const float* src = which == 0 ? kv.K(layer, head, 0) : kv.V(layer, head, 0);
    std::memcpy(out, src, static_cast<size_t>(n * kv.hd) * sizeof(float));
  });
}

// logits: [n, vocab]; kv may be null.
int32_t orc_forward(void* mp, const int32_t* ids, int64_t n, void* kv, float* logits) {
  return Guard([&] {
    const orc::Model& m = *static_cast<orc::Model*>(mp);
    std::vector<float> out;
    orc::ForwardFull(m, ids, n, &out, static_cast<orc::KvCache*>(kv));
    std::memcpy(logits, out.data(), out.size() * sizeof(float));
  });
}

// Generate from `first_logits`; returns the number of ids written or -1.
// step_logits (optional) receives [returned, vocab].
int32_t orc_generate(void* mp, void* kv, const float* first_logits, int32_t max_tokens, float temperature,
                     int32_t top_k, float top_p, uint64_t seed, const int32_t* stop_ids, int32_t n_stop,
                     int32_t* out_ids, float* step_logits) {
  std::vector<int32_t> out;
  const int32_t rc = Guard([&] {
    const orc::Model& m = *static_cast<orc::Model*>(mp);
    orc::GenerateOptions g;
    g.max_tokens = max_tokens;
    g.sample.temperature = temperature;
    g.sample.top_k = top_k;
    g.sample.top_p = top_p;
    g.seed = seed;
    g.stop_ids.assign(stop_ids, stop_ids + n_stop);
    std::vector<float> steps;
    orc::Generate(m, static_cast<orc::KvCache*>(kv), first_logits, g, &out,
                  step_logits ? &steps : nullptr);
    std::memcpy(out_ids, out.data(), out.size() * sizeof(int32_t));
    if (step_logits) std::memcpy(step_logits, steps.data(), steps.size() * sizeof(float));
  });
  return rc < 0 ? -1 : static_cast<int32_t>(out.size());
}

// CPU baseline timing: prefill n ids then generate `gen` tokens; writes
// [prefill_ms, decode_ms, threads].
int32_t orc_time_run(void* mp, const int32_t* ids, int64_t n, int32_t gen, float temperature, int32_t top_k,
                     float top_p, uint64_t seed, double* out3) {
  return Guard([&] {
    const orc::Model& m = *static_cast<orc::Model*>(mp);
    orc::KvCache kv(m.config(), n + gen + 8);
    std::vector<float> logits;
    const auto t0 = std::chrono::steady_clock::now();
    orc::ForwardFull(m, ids, n, &logits, &kv);
    const auto t1 = std::chrono::steady_clock::now();
    orc::GenerateOptions g;
    g.max_tokens = gen;
    g.sample.temperature = temperature;
    g.sample.top_k = top_k;
    g.sample.top_p = top_p;
    g.seed = seed;
    std::vector<int32_t> out;
    if (gen > 0) orc::Generate(m, &kv, logits.data() + (n - 1) * m.config().vocab, g, &out, nullptr);
    const auto t2 = std::chrono::steady_clock::now();
    out3[0] = std::chrono::duration<double, std::milli>(t1 - t0).count();
    out3[1] = std::chrono::duration<double, std::milli>(t2 - t1).count();
    out3[2] = m.pool().size();
  });
}

}  // extern "C"
