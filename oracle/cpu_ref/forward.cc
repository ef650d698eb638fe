// Scalar kernels, attention, layer, full forward and generate loop --
// restates reference src/kernels.h:26-120 and src/qwen3.cc:44-363 with the
// same operation order. Non-AVX TU: products and sums round separately.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

#include "oracle.h"

namespace orc {

// reference src/kernels.h:26-38: four lane accumulators
float Dot(const float* a, const float* b, int64_t n) {
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  int64_t i = 0;
  for (; i < n - 3; i += 4) {
    s0 += a[i] * b[i];
    s1 += a[i + 1] * b[i + 1];
    s2 += a[i + 2] * b[i + 2];
    s3 += a[i + 3] * b[i + 3];
  }
  for (; i < n; ++i) s0 += a[i] * b[i];
  return (s0 + s1) + (s2 + s3);
}

// reference src/kernels.h:42-52: first index of the maximum (strict >)
int32_t ArgMax(const float* x, int64_t n) {
  int32_t best = 0;
  float bv = x[0];
  for (int64_t i = 1; i < n; ++i) {
    if (x[i] > bv) {
      bv = x[i];
      best = static_cast<int32_t>(i);
    }
  }
  return best;
}

// reference src/kernels.h:56-63: double sum of squares, float scale,
// out = (x * scale) * w
void RmsNorm(const float* x, const float* w, int64_t n, float eps, float* out) {
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) sum += static_cast<double>(x[i]) * x[i];
  const double mean = sum / static_cast<double>(n);
  const float scale = static_cast<float>(1.0 / std::sqrt(mean + eps));
  for (int64_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

// reference src/kernels.h:66-79: float max, expf, double sum, float 1/sum
void SoftmaxInPlace(float* x, int64_t n) {
  if (n <= 0) return;
  float mx = x[0];
  for (int64_t i = 1; i < n; ++i)
    if (x[i] > mx) mx = x[i];
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const float e = std::exp(x[i] - mx);
    x[i] = e;
    sum += e;
  }
  const float inv = static_cast<float>(1.0 / sum);
  for (int64_t i = 0; i < n; ++i) x[i] *= inv;
}

// reference src/kernels.h:82-87: v / (1 + expf(-v))
void SiluInPlace(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    x[i] = v / (1.0f + std::exp(-v));
  }
}

void MulInPlace(float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; ++i) a[i] *= b[i];
}

void VecAddInPlace(float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; ++i) a[i] += b[i];
}

// reference src/kernels.h:108-120: pairs (i, i + hd/2)
void RopeInPlace(float* x, int32_t n_heads, int32_t head_dim, const float* cos_t,
                 const float* sin_t) {
  const int32_t half = head_dim / 2;
  for (int32_t h = 0; h < n_heads; ++h) {
    float* xh = x + static_cast<int64_t>(h) * head_dim;
    for (int32_t i = 0; i < half; ++i) {
      const float c = cos_t[i], s = sin_t[i];
      const float a = xh[i], b = xh[i + half];
      xh[i] = a * c - b * s;
      xh[i + half] = b * c + a * s;
    }
  }
}

// The fp16 value nearest to x (ties to even), as a float: 11 significant
// bits for normal halves, the 2^-24 quantum below 2^-14, infinity from 65520
// on (the midpoint between the largest half, 65504, and 2^16).
float RoundToHalf(float x) {
  if (!std::isfinite(x) || x == 0.0f) return x;
  const float a = std::fabs(x);
  if (a >= 65520.0f) return std::copysign(std::numeric_limits<float>::infinity(), x);
  int e = 0;
  (void)std::frexp(a, &e);              // a = f * 2^e, f in [0.5, 1)
  const int q = std::max(e - 11, -24);  // exponent of the half's last bit
  return std::copysign(std::ldexp(std::nearbyint(std::ldexp(a, -q)), q), x);
}

KvCache::KvCache(const Config& c, int64_t ms)
    : n_layers(c.n_layers), n_kv(c.n_kv_heads), hd(c.head_dim), max_seq(ms) {
  ORC_CHECK(max_seq > 0, "max_seq must be positive");
  const size_t per = static_cast<size_t>(n_layers) * n_kv * max_seq * hd;
  k.assign(per, 0.0f);
  v.assign(per, 0.0f);
}

namespace {

struct Scratch {
  std::vector<float> x, h, q, k, v, attn, proj, gate, up, scores;
};

// reference src/qwen3.cc:44-77 (no cache) and :79-117 (from cache).
// kbase(kh) / vbase(kh) address position 0 of KV head kh; consecutive
// positions are `stride` floats apart.
template <typename KBase, typename VBase>
void Attention(const Config& c, const float* q, int64_t seq, int64_t pos0, KBase kbase, VBase vbase,
               int64_t stride, float* scores, float* out) {
  const int32_t hd = c.head_dim;
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  const int64_t qs = static_cast<int64_t>(c.n_heads) * hd;
  std::memset(out, 0, static_cast<size_t>(seq * qs) * sizeof(float));
  for (int32_t h = 0; h < c.n_heads; ++h) {
    const int32_t kh = h / c.group();
    const float* kb = kbase(kh);
    const float* vb = vbase(kh);
    for (int64_t t = 0; t < seq; ++t) {
      const int64_t pos = pos0 + t;
      const float* qt = q + t * qs + static_cast<int64_t>(h) * hd;
      for (int64_t s = 0; s <= pos; ++s) scores[s] = Dot(qt, kb + s * stride, hd) * scale;
      SoftmaxInPlace(scores, pos + 1);
      float* ot = out + t * qs + static_cast<int64_t>(h) * hd;
      for (int64_t s = 0; s <= pos; ++s) {
        const float* vs = vb + s * stride;
        const float p = scores[s];
        for (int32_t d = 0; d < hd; ++d) ot[d] += p * vs[d];
      }
    }
  }
}

// reference src/qwen3.cc:119-206
void Layer_(const Model& m, const Layer& w, int32_t layer, int64_t pos0, Scratch* s, int64_t seq,
            KvCache* kv) {
  const Config& c = m.config();
  Pool* pool = &m.pool();
  const int64_t H = c.hidden, F = c.intermediate, qd = c.q_dim(), kvd = c.kv_dim();
  const int32_t hd = c.head_dim;
  for (int64_t t = 0; t < seq; ++t)
    RmsNorm(s->x.data() + t * H, w.attn_norm.data(), H, c.rms_eps, s->h.data() + t * H);
  w.q.MatMulBatch(s->h.data(), seq, s->q.data(), pool);
  w.k.MatMulBatch(s->h.data(), seq, s->k.data(), pool);
  w.v.MatMulBatch(s->h.data(), seq, s->v.data(), pool);
  // per-head QK-norm before RoPE (reference :139-152)
  for (int64_t t = 0; t < seq; ++t) {
    for (int32_t h = 0; h < c.n_heads; ++h) {
      float* p = s->q.data() + t * qd + static_cast<int64_t>(h) * hd;
      RmsNorm(p, w.q_norm.data(), hd, c.rms_eps, p);
    }
    for (int32_t h = 0; h < c.n_kv_heads; ++h) {
      float* p = s->k.data() + t * kvd + static_cast<int64_t>(h) * hd;
      RmsNorm(p, w.k_norm.data(), hd, c.rms_eps, p);
    }
  }
  for (int64_t t = 0; t < seq; ++t) {
    RopeInPlace(s->q.data() + t * qd, c.n_heads, hd, m.rope_cos(pos0 + t), m.rope_sin(pos0 + t));
    RopeInPlace(s->k.data() + t * kvd, c.n_kv_heads, hd, m.rope_cos(pos0 + t), m.rope_sin(pos0 + t));
  }
  if (kv != nullptr) {
    for (int64_t t = 0; t < seq; ++t) {
      for (int32_t h = 0; h < c.n_kv_heads; ++h) {
        float* kd = kv->K(layer, h, pos0 + t);
        float* vd = kv->V(layer, h, pos0 + t);
        std::memcpy(kd, s->k.data() + t * kvd + static_cast<int64_t>(h) * hd, static_cast<size_t>(hd) * sizeof(float));
        std::memcpy(vd, s->v.data() + t * kvd + static_cast<int64_t>(h) * hd, static_cast<size_t>(hd) * sizeof(float));
        if (kv->fp16) {
          for (int32_t i = 0; i < hd; ++i) {
            kd[i] = RoundToHalf(kd[i]);
            vd[i] = RoundToHalf(vd[i]);
          }
        }
      }
    }
    Attention(c, s->q.data(), seq, pos0, [&](int32_t kh) { return kv->K(layer, kh, 0); },
              [&](int32_t kh) { return kv->V(layer, kh, 0); }, hd, s->scores.data(), s->attn.data());
  } else {
    Attention(c, s->q.data(), seq, 0,
              [&](int32_t kh) -> const float* { return s->k.data() + static_cast<int64_t>(kh) * hd; },
              [&](int32_t kh) -> const float* { return s->v.data() + static_cast<int64_t>(kh) * hd; }, kvd,
              s->scores.data(), s->attn.data());
  }
  w.o.MatMulBatch(s->attn.data(), seq, s->proj.data(), pool);
  for (int64_t t = 0; t < seq; ++t) VecAddInPlace(s->x.data() + t * H, s->proj.data() + t * H, H);
  for (int64_t t = 0; t < seq; ++t)
    RmsNorm(s->x.data() + t * H, w.ffn_norm.data(), H, c.rms_eps, s->h.data() + t * H);
  w.gate.MatMulBatch(s->h.data(), seq, s->gate.data(), pool);
  w.up.MatMulBatch(s->h.data(), seq, s->up.data(), pool);
  for (int64_t t = 0; t < seq; ++t) {
    SiluInPlace(s->gate.data() + t * F, F);
    MulInPlace(s->gate.data() + t * F, s->up.data() + t * F, F);
  }
  w.down.MatMulBatch(s->gate.data(), seq, s->proj.data(), pool);
  for (int64_t t = 0; t < seq; ++t) VecAddInPlace(s->x.data() + t * H, s->proj.data() + t * H, H);
}

}  // namespace

// Attention of a segment over a cache [n_kv][pos0 + seq][hd] (the C API's
// attention probe): the Attention above with the cache's head stride.
void AttentionCache(int32_t n_heads, int32_t n_kv, int32_t hd, const float* q, int64_t seq, int64_t pos0,
                    const float* k, const float* v, float* out) {
  Config c;
  c.n_heads = n_heads;
  c.n_kv_heads = n_kv;
  c.head_dim = hd;
  const int64_t n_pos = pos0 + seq;
  std::vector<float> scores(static_cast<size_t>(n_pos));
  Attention(
      c, q, seq, pos0, [&](int32_t kh) { return k + static_cast<int64_t>(kh) * n_pos * hd; },
      [&](int32_t kh) { return v + static_cast<int64_t>(kh) * n_pos * hd; }, hd, scores.data(), out);
}

// reference src/qwen3.cc:208-290
void ForwardFull(const Model& m, const int32_t* tokens, int64_t seq, std::vector<float>* logits,
                 KvCache* kv) {
  const Config& c = m.config();
  ORC_CHECK(seq > 0, "empty prompt");
  const int64_t pos0 = kv ? kv->len : 0;
  ORC_CHECK(pos0 + seq <= m.rope_positions(), "position %lld beyond the RoPE table (%lld)",
            (long long)(pos0 + seq), (long long)m.rope_positions());
  if (kv) ORC_CHECK(pos0 + seq <= kv->max_seq, "position %lld beyond the KV capacity", (long long)(pos0 + seq));
  const int64_t H = c.hidden;
  Scratch s;
  s.x.assign(seq * H, 0.0f);
  s.h.assign(seq * H, 0.0f);
  s.q.assign(seq * c.q_dim(), 0.0f);
  s.k.assign(seq * c.kv_dim(), 0.0f);
  s.v.assign(seq * c.kv_dim(), 0.0f);
  s.attn.assign(seq * c.q_dim(), 0.0f);
  s.proj.assign(seq * H, 0.0f);
  s.gate.assign(seq * c.intermediate, 0.0f);
  s.up.assign(seq * c.intermediate, 0.0f);
  s.scores.assign(pos0 + seq, 0.0f);
  for (int64_t t = 0; t < seq; ++t) {
    ORC_CHECK(tokens[t] >= 0 && tokens[t] < c.vocab, "token %d out of range", tokens[t]);
    m.embd().Row(tokens[t], s.x.data() + t * H);  // not scaled (Qwen3)
  }
  for (int32_t l = 0; l < c.n_layers; ++l) Layer_(m, m.layers()[static_cast<size_t>(l)], l, pos0, &s, seq, kv);
  if (kv) kv->len = pos0 + seq;  // committed after all layers (reference :272-274)
  for (int64_t t = 0; t < seq; ++t)
    RmsNorm(s.x.data() + t * H, m.output_norm().data(), H, c.rms_eps, s.h.data() + t * H);
  logits->assign(static_cast<size_t>(seq) * c.vocab, 0.0f);
  m.lm_head().MatMulBatch(s.h.data(), seq, logits->data(), &m.pool());
}

// reference src/qwen3.cc:302-355: pick (argmax, or CounterUniform(seed,
// kv.len) + SampleToken), append, stop check, capacity check, forward the
// returned token (including the last one).
void Generate(const Model& m, KvCache* kv, const float* first_logits, const GenerateOptions& opt,
              std::vector<int32_t>* out_ids, std::vector<float>* step_logits) {
  const Config& c = m.config();
  ORC_CHECK(kv != nullptr, "Generate needs a KV cache");
  ORC_CHECK(opt.max_tokens > 0, "max_tokens must be positive");
  std::vector<float> logits(first_logits, first_logits + c.vocab);
  const bool greedy = !(opt.sample.temperature > 0.0f);
  for (int32_t i = 0; i < opt.max_tokens; ++i) {
    int32_t next;
    if (greedy) {
      next = ArgMax(logits.data(), c.vocab);
    } else {
      const float u = CounterUniform(opt.seed, static_cast<uint64_t>(kv->len));
      next = SampleToken(logits.data(), c.vocab, opt.sample, u);
    }
    out_ids->push_back(next);
    bool stop = false;
    for (int32_t sid : opt.stop_ids) stop = stop || sid == next;
    ORC_CHECK(kv->len < kv->max_seq, "context full (%lld positions)", (long long)kv->max_seq);
    int32_t tok = next;
    ForwardFull(m, &tok, 1, &logits, kv);
    if (step_logits) step_logits->insert(step_logits->end(), logits.begin(), logits.end());
    if (stop) break;
  }
}

}  // namespace orc
