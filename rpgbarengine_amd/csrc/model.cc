#include "model.h"

#include <cmath>
#include <cstring>

#include "common.h"
#include "decode.h"
#include "kernels.h"

namespace rpg {

namespace {

constexpr int64_t kAlign = 256;
constexpr int64_t kTailPad = 256;  // block decoders may read a few bytes past a block

int64_t AlignUp(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

}  // namespace

DeviceModel::~DeviceModel() {
  if (arena_) (void)hipFree(arena_);
  if (tiled_) (void)hipFree(tiled_);
  if (rope_dev_) (void)hipFree(rope_dev_);
  if (norms_f32_) (void)hipFree(norms_f32_);
}

std::unique_ptr<DeviceModel> DeviceModel::Load(const std::string& path, int32_t max_pos) {
  std::unique_ptr<DeviceModel> m(new DeviceModel());
  m->gguf_.reset(GgufFile::Open(path));
  const GgufFile& g = *m->gguf_;
  ModelConfig& c = m->cfg_;
  c.arch = g.Str("general.architecture");
  RPG_CHECK(c.arch == "qwen3", "model architecture is %s; this engine implements qwen3", c.arch.c_str());
  c.name = g.Str("general.name", "(unnamed)");
  c.n_layers = static_cast<int32_t>(g.Int("qwen3.block_count", 0));
  c.hidden = static_cast<int32_t>(g.Int("qwen3.embedding_length", 0));
  c.n_heads = static_cast<int32_t>(g.Int("qwen3.attention.head_count", 0));
  c.n_kv_heads = static_cast<int32_t>(g.Int("qwen3.attention.head_count_kv", c.n_heads));
  c.intermediate = static_cast<int32_t>(g.Int("qwen3.feed_forward_length", 0));
  c.context_length = static_cast<int32_t>(g.Int("qwen3.context_length", 4096));
  // head_dim only from key_length: hidden / heads is wrong for the 4B shape
  // (reference src/model.cc:167-179).
  const int64_t key_len = g.Int("qwen3.attention.key_length", 0);
  if (key_len > 0) {
    c.head_dim = static_cast<int32_t>(key_len);
  } else {
    RPG_CHECK(c.n_heads > 0 && c.hidden % c.n_heads == 0,
              "attention.key_length missing and hidden %d not divisible by heads %d", c.hidden, c.n_heads);
    Log(kLogWarn, "GGUF has no attention.key_length; using hidden/heads = %d", c.hidden / c.n_heads);
    c.head_dim = c.hidden / c.n_heads;
  }
  c.value_dim = static_cast<int32_t>(g.Int("qwen3.attention.value_length", c.head_dim));
  c.rope_theta = static_cast<float>(g.Float("qwen3.rope.freq_base", 10000.0));
  c.rms_eps = static_cast<float>(g.Float("qwen3.attention.layer_norm_rms_epsilon", 1e-6));
  c.bos_id = static_cast<int32_t>(g.Int("tokenizer.ggml.bos_token_id", -1));
  c.eos_id = static_cast<int32_t>(g.Int("tokenizer.ggml.eos_token_id", -1));
  c.pad_id = static_cast<int32_t>(g.Int("tokenizer.ggml.padding_token_id", -1));
  c.add_bos = g.Int("tokenizer.ggml.add_bos_token", 0) != 0;
  RPG_CHECK(c.n_layers > 0 && c.hidden > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.head_dim > 0 &&
                c.intermediate > 0,
            "incomplete GGUF metadata: layers=%d hidden=%d heads=%d kv=%d head_dim=%d ffn=%d", c.n_layers, c.hidden,
            c.n_heads, c.n_kv_heads, c.head_dim, c.intermediate);
  RPG_CHECK(c.n_heads % c.n_kv_heads == 0, "%d query heads is not a multiple of %d KV heads", c.n_heads,
            c.n_kv_heads);
  RPG_CHECK(c.value_dim == c.head_dim, "value_length %d differs from key_length %d", c.value_dim, c.head_dim);
  if (c.context_length <= 0) c.context_length = 4096;
  const int64_t n_tok = g.ArrayLen("tokenizer.ggml.tokens");
  RPG_CHECK(n_tok > 0, "GGUF has no tokenizer.ggml.tokens");
  c.vocab = static_cast<int32_t>(n_tok);

  // ---- plan the arena: every tensor the forward pass reads
  struct Item {
    const GgufTensor* t;
    int64_t off;
  };
  std::vector<Item> items;
  int64_t off = 0;
  auto place = [&](const GgufTensor* t) {
    items.push_back({t, off});
    off = AlignUp(off + t->n_bytes, kAlign);
    return items.back().off;
  };
  auto require = [&](const std::string& name) -> const GgufTensor* {
    const GgufTensor* t = g.Find(name);
    if (!t) Throw("tensor %s not found in the GGUF (architecture %s)", name.c_str(), c.arch.c_str());
    return t;
  };
  auto check_mat = [&](const GgufTensor* t, int64_t rows, int64_t cols) {
    if (t->dims.size() != 2 || t->rows() != rows || t->cols() != cols)
      Throw("tensor %s has the wrong shape: want [%lld,%lld] (rows x cols)", t->name.c_str(), (long long)rows,
            (long long)cols);
  };
  auto check_norm = [&](const GgufTensor* t, int64_t n) {
    if (t->dims.size() != 1 || t->dims[0] != n)
      Throw("norm %s has the wrong shape (want %lld elements)", t->name.c_str(), (long long)n);
    if (BlockElems(t->type) <= 0 || n % BlockElems(t->type) != 0)
      Throw("norm %s: type %s cannot hold %lld elements", t->name.c_str(), TypeName(t->type), (long long)n);
  };
  struct MatPlan {
    const GgufTensor* t;
    int64_t off;
  };
  auto mat = [&](const std::string& name, int64_t rows, int64_t cols) {
    const GgufTensor* t = require(name);
    check_mat(t, rows, cols);
    RPG_CHECK(cols % 32 == 0, "tensor %s: %lld columns is not a multiple of 32", name.c_str(), (long long)cols);
    return MatPlan{t, place(t)};
  };
  auto norm = [&](const std::string& name, int64_t n) {
    const GgufTensor* t = require(name);
    check_norm(t, n);
    return MatPlan{t, place(t)};
  };
  const MatPlan emb = mat("token_embd.weight", c.vocab, c.hidden);
  MatPlan head = emb;
  if (const GgufTensor* out = g.Find("output.weight")) {
    check_mat(out, c.vocab, c.hidden);
    head = MatPlan{out, place(out)};
    c.tied_embeddings = false;
  } else {
    c.tied_embeddings = true;
  }
  const MatPlan onorm = norm("output_norm.weight", c.hidden);
  struct LayerPlan {
    MatPlan an, fn, qn, kn, q, k, v, o, gate, up, down;
  };
  std::vector<LayerPlan> lp(static_cast<size_t>(c.n_layers));
  for (int l = 0; l < c.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    LayerPlan& x = lp[static_cast<size_t>(l)];
    x.an = norm(p + "attn_norm.weight", c.hidden);
    x.fn = norm(p + "ffn_norm.weight", c.hidden);
    x.qn = norm(p + "attn_q_norm.weight", c.head_dim);
    x.kn = norm(p + "attn_k_norm.weight", c.head_dim);
    x.q = mat(p + "attn_q.weight", c.q_dim(), c.hidden);
    x.k = mat(p + "attn_k.weight", c.kv_dim(), c.hidden);
    x.v = mat(p + "attn_v.weight", c.kv_dim(), c.hidden);
    x.o = mat(p + "attn_output.weight", c.hidden, c.q_dim());
    x.gate = mat(p + "ffn_gate.weight", c.intermediate, c.hidden);
    x.up = mat(p + "ffn_up.weight", c.intermediate, c.hidden);
    x.down = mat(p + "ffn_down.weight", c.hidden, c.intermediate);
  }

  // ---- upload
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  m->device_ = dev;
  m->arena_bytes_ = off + kTailPad;
  DeviceAlloc(&m->arena_, static_cast<size_t>(m->arena_bytes_));
  HIP_CHECK(hipMemset(m->arena_ + off, 0, kTailPad));
  for (const Item& it : items) {
    HIP_CHECK(hipMemcpy(m->arena_ + it.off, g.TensorData(*it.t), static_cast<size_t>(it.t->n_bytes),
                        hipMemcpyHostToDevice));
  }
  // every tensor of the file, as the reference counts it (reference
  // src/model.h:139-143)
  m->weight_bytes_ = 0;
  for (const GgufTensor& t : g.tensors()) m->weight_bytes_ += t.n_bytes;
  auto mref = [&](const MatPlan& p) {
    k::MatRef r;
    r.w = m->arena_ + p.off;
    r.type = p.t->type;
    r.rows = static_cast<int32_t>(p.t->rows());
    r.cols = static_cast<int32_t>(p.t->cols());
    r.row_bytes = RowBytes(p.t->type, p.t->cols());
    return r;
  };
  // Norm gains stored in another type are dequantised once into their own
  // fp32 buffer, as the reference does at load (reference src/model.cc:99-120).
  std::vector<const GgufTensor*> odd_norms;
  for (const Item& it : items)
    if (it.t->dims.size() == 1 && it.t->type != kF32) odd_norms.push_back(it.t);
  std::vector<std::pair<int64_t, int64_t>> norm_at;  // (arena offset, fp32 offset)
  if (!odd_norms.empty()) {
    int64_t n_f = 0;
    for (const GgufTensor* t : odd_norms) n_f += t->n_elements;
    DeviceAlloc(&m->norms_f32_, sizeof(float) * static_cast<size_t>(n_f));
    int64_t at = 0;
    for (const Item& it : items) {
      if (it.t->dims.size() != 1 || it.t->type == kF32) continue;
      Log(kLogWarn, "norm %s is %s: dequantised at load", it.t->name.c_str(), TypeName(it.t->type));
      k::Dequant(it.t->type, m->arena_ + it.off, it.t->n_elements, m->norms_f32_ + at, nullptr);
      norm_at.push_back({it.off, at});
      at += it.t->n_elements;
    }
    HIP_CHECK(hipDeviceSynchronize());
  }
  auto fptr = [&](const MatPlan& p) -> const float* {
    for (const auto& na : norm_at)
      if (na.first == p.off) return m->norms_f32_ + na.second;
    return reinterpret_cast<const float*>(m->arena_ + p.off);
  };
  m->embd_ = mref(emb);
  m->lm_head_ = mref(head);
  m->output_norm_ = fptr(onorm);
  m->layers_.resize(static_cast<size_t>(c.n_layers));
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerPlan& x = lp[static_cast<size_t>(l)];
    LayerDev& d = m->layers_[static_cast<size_t>(l)];
    d.attn_norm = fptr(x.an);
    d.ffn_norm = fptr(x.fn);
    d.q_norm = fptr(x.qn);
    d.k_norm = fptr(x.kn);
    d.q = mref(x.q);
    d.k = mref(x.k);
    d.v = mref(x.v);
    d.o = mref(x.o);
    d.gate = mref(x.gate);
    d.up = mref(x.up);
    d.down = mref(x.down);
  }

  // ---- tile-major decode copies
  {
    struct Copy {
      const k::MatRef* a;
      const k::MatRef* b;
      k::MatRef* out;
    };
    std::vector<Copy> copies;
    for (LayerDev& d : m->layers_) {
      copies.push_back({&d.q, nullptr, &d.dq});
      copies.push_back({&d.k, nullptr, &d.dk});
      copies.push_back({&d.v, nullptr, &d.dv});
      copies.push_back({&d.o, nullptr, &d.dout});
      copies.push_back({&d.down, nullptr, &d.ddown});
      if (d.gate.type == d.up.type && d.gate.rows == d.up.rows && d.gate.cols == d.up.cols)
        copies.push_back({&d.gate, &d.up, &d.gate_up});
    }
    copies.push_back({&m->lm_head_, nullptr, &m->lm_head_t_});
    int64_t tb = 0;
    std::vector<int64_t> offs;
    for (const Copy& cp : copies) {
      offs.push_back(tb);
      if (k::DecodeTileable(*cp.a)) tb += AlignUp(k::TileMajorBytes(*cp.a, cp.b != nullptr), kAlign);
    }
    if (tb > 0) {
      m->tiled_bytes_ = tb + kTailPad;
      DeviceAlloc(&m->tiled_, static_cast<size_t>(m->tiled_bytes_));
      for (size_t i = 0; i < copies.size(); ++i) {
        const Copy& cp = copies[i];
        if (!k::DecodeTileable(*cp.a)) continue;
        k::TileMajor(*cp.a, cp.b, m->tiled_ + offs[i], nullptr);
        *cp.out = *cp.a;
        cp.out->w = m->tiled_ + offs[i];
      }
      HIP_CHECK(hipDeviceSynchronize());
    }
  }

  // ---- RoPE table: inv[i] = 1/theta^(2i/hd), angle p*inv[i] in double,
  // cos/sin rounded to float; row = [cos(hd/2) | sin(hd/2)].
  const int32_t half = c.head_dim / 2;
  m->n_rope_ = max_pos > c.context_length ? c.context_length : max_pos;
  if (m->n_rope_ <= 0) m->n_rope_ = 1;
  m->rope_host_.assign(static_cast<size_t>(m->n_rope_) * c.head_dim, 0.0f);
  std::vector<double> inv(static_cast<size_t>(half));
  for (int32_t i = 0; i < half; ++i) {
    inv[i] = 1.0 / std::pow(static_cast<double>(c.rope_theta),
                            static_cast<double>(2 * i) / static_cast<double>(c.head_dim));
  }
  for (int64_t p = 0; p < m->n_rope_; ++p) {
    float* row = m->rope_host_.data() + p * c.head_dim;
    for (int32_t i = 0; i < half; ++i) {
      const double ang = static_cast<double>(p) * inv[i];
      row[i] = static_cast<float>(std::cos(ang));
      row[half + i] = static_cast<float>(std::sin(ang));
    }
  }
  DeviceAlloc(&m->rope_dev_, m->rope_host_.size() * sizeof(float));
  HIP_CHECK(hipMemcpy(m->rope_dev_, m->rope_host_.data(), m->rope_host_.size() * sizeof(float),
                      hipMemcpyHostToDevice));
  Log(kLogInfo, "loaded %s: %d layers, hidden %d, %d/%d heads, head_dim %d, ffn %d, vocab %d, tied=%d, %.2f GB",
      c.name.c_str(), c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.intermediate, c.vocab,
      c.tied_embeddings ? 1 : 0, static_cast<double>(m->weight_bytes_) / 1e9);
  return m;
}

int64_t DeviceModel::decode_weight_bytes() const {
  const ModelConfig& c = cfg_;
  int64_t b = 0;
  for (const LayerDev& l : layers_) {
    for (const k::MatRef* r : {&l.q, &l.k, &l.v, &l.o, &l.gate, &l.up, &l.down}) b += r->row_bytes * r->rows;
    b += (2 * static_cast<int64_t>(c.hidden) + 2 * c.head_dim) * 4;
  }
  b += lm_head_.row_bytes * lm_head_.rows;
  b += embd_.row_bytes;  // one embedding row
  b += static_cast<int64_t>(c.hidden) * 4;
  return b;
}

}  // namespace rpg
