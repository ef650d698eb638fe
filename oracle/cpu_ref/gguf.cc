// Minimal GGUF v1-v3 reader + qwen3 model loader -- restates reference
// src/gguf.cc:169-260 (header, metadata, tensor table, data_start alignment,
// bounds checks) and src/model.cc:99-281 (config from metadata only, shape
// checks, F32 norms, tied lm_head, RoPE table in double).

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <map>

#include "oracle.h"

namespace orc {

struct TensorInfo {
  std::vector<int64_t> dims;  // dims[0] fastest
  uint32_t type = 0;
  uint64_t offset = 0;
  int64_t bytes = 0;
};

class GgufMap {
 public:
  explicit GgufMap(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    ORC_CHECK(fd_ >= 0, "cannot open %s", path.c_str());
    struct stat st;
    ORC_CHECK(::fstat(fd_, &st) == 0, "stat failed for %s", path.c_str());
    size_ = static_cast<size_t>(st.st_size);
    ORC_CHECK(size_ >= 24, "file too small to be GGUF: %s", path.c_str());
    void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    ORC_CHECK(p != MAP_FAILED, "mmap failed for %s", path.c_str());
    base_ = static_cast<const uint8_t*>(p);
    Parse();
  }
  ~GgufMap() {
    if (base_) ::munmap(const_cast<uint8_t*>(base_), size_);
    if (fd_ >= 0) ::close(fd_);
  }

  std::map<std::string, double> nums;
  std::map<std::string, std::string> strs;
  std::map<std::string, int64_t> array_len;
  std::map<std::string, TensorInfo> tensors;
  const uint8_t* data(const TensorInfo& t) const { return base_ + data_start_ + t.offset; }

 private:
  template <typename T>
  T Get() {
    ORC_CHECK(pos_ + sizeof(T) <= size_, "read past end of file at %zu", pos_);
    T v;
    std::memcpy(&v, base_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }
  std::string Str() {
    const uint64_t n = Get<uint64_t>();
    ORC_CHECK(pos_ + n <= size_, "string past end of file");
    std::string s(reinterpret_cast<const char*>(base_ + pos_), n);
    pos_ += n;
    return s;
  }
  // metadata value types (GGUF spec): 0 u8 1 i8 2 u16 3 i16 4 u32 5 i32 6 f32
  // 7 bool 8 string 9 array 10 u64 11 i64 12 f64
  void Value(const std::string& key, uint32_t type, bool top) {
    double v = 0.0;
    switch (type) {
      case 0: v = Get<uint8_t>(); break;
      case 1: v = Get<int8_t>(); break;
      case 2: v = Get<uint16_t>(); break;
      case 3: v = Get<int16_t>(); break;
      case 4: v = Get<uint32_t>(); break;
      case 5: v = Get<int32_t>(); break;
      case 6: v = Get<float>(); break;
      case 7: v = Get<uint8_t>(); break;
      case 8: {
        std::string s = Str();
        if (top) strs[key] = s;
        return;
      }
      case 9: {
        const uint32_t et = Get<uint32_t>();
        const uint64_t n = Get<uint64_t>();
        ORC_CHECK(n < (1ull << 32), "metadata array too long");
        if (top) array_len[key] = static_cast<int64_t>(n);
        for (uint64_t i = 0; i < n; ++i) Value(key, et, false);
        return;
      }
      case 10: v = static_cast<double>(Get<uint64_t>()); break;
      case 11: v = static_cast<double>(Get<int64_t>()); break;
      case 12: v = Get<double>(); break;
      default: Fail("unknown GGUF metadata type %u", type);
    }
    if (top) nums[key] = v;
  }
  void Parse() {
    ORC_CHECK(Get<uint32_t>() == 0x46554747u, "bad GGUF magic");
    const uint32_t version = Get<uint32_t>();
    ORC_CHECK(version >= 1 && version <= 3, "unsupported GGUF version %u", version);
    const uint64_t n_tensors = version == 1 ? Get<uint32_t>() : Get<uint64_t>();
    const uint64_t n_kv = version == 1 ? Get<uint32_t>() : Get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; ++i) {
      const std::string key = Str();
      Value(key, Get<uint32_t>(), true);
    }
    const uint64_t align = nums.count("general.alignment") ? static_cast<uint64_t>(nums["general.alignment"]) : 32;
    ORC_CHECK(align > 0 && align % 8 == 0, "bad alignment %llu", (unsigned long long)align);
    for (uint64_t i = 0; i < n_tensors; ++i) {
      const std::string name = Str();
      TensorInfo t;
      const uint32_t nd = Get<uint32_t>();
      ORC_CHECK(nd >= 1 && nd <= 4, "tensor %s has %u dims", name.c_str(), nd);
      int64_t elems = 1;
      for (uint32_t d = 0; d < nd; ++d) {
        const uint64_t v = Get<uint64_t>();
        ORC_CHECK(v > 0 && v < (1ull << 40), "tensor %s bad dim", name.c_str());
        t.dims.push_back(static_cast<int64_t>(v));
        elems *= static_cast<int64_t>(v);
      }
      t.type = Get<uint32_t>();
      t.offset = Get<uint64_t>();
      t.bytes = RowBytes(t.type, elems);
      ORC_CHECK(tensors.emplace(name, t).second, "duplicate tensor %s", name.c_str());
    }
    data_start_ = (pos_ + align - 1) / align * align;
    for (const auto& kv : tensors) {
      ORC_CHECK(data_start_ + kv.second.offset + static_cast<uint64_t>(kv.second.bytes) <= size_,
                "tensor %s runs past the end of the file", kv.first.c_str());
    }
  }

  int fd_ = -1;
  const uint8_t* base_ = nullptr;
  size_t size_ = 0;
  size_t pos_ = 0;
  uint64_t data_start_ = 0;
};

Model::~Model() = default;

std::unique_ptr<Model> Model::Load(const std::string& path, int threads, int32_t max_pos) {
  std::unique_ptr<Model> m(new Model());
  m->file_.reset(new GgufMap(path));
  GgufMap& g = *m->file_;
  ORC_CHECK(g.strs["general.architecture"] == "qwen3", "architecture is not qwen3");
  auto num = [&](const std::string& k, double def) {
    auto it = g.nums.find(k);
    return it == g.nums.end() ? def : it->second;
  };
  Config& c = m->cfg_;
  c.n_layers = static_cast<int32_t>(num("qwen3.block_count", 0));
  c.hidden = static_cast<int32_t>(num("qwen3.embedding_length", 0));
  c.n_heads = static_cast<int32_t>(num("qwen3.attention.head_count", 0));
  c.n_kv_heads = static_cast<int32_t>(num("qwen3.attention.head_count_kv", c.n_heads));
  c.intermediate = static_cast<int32_t>(num("qwen3.feed_forward_length", 0));
  c.context_length = static_cast<int32_t>(num("qwen3.context_length", 4096));
  c.head_dim = static_cast<int32_t>(num("qwen3.attention.key_length", 0));  // never hidden/heads
  ORC_CHECK(c.head_dim > 0, "missing attention.key_length");
  c.rope_theta = static_cast<float>(num("qwen3.rope.freq_base", 10000.0));
  c.rms_eps = static_cast<float>(num("qwen3.attention.layer_norm_rms_epsilon", 1e-6));
  c.eos_id = static_cast<int32_t>(num("tokenizer.ggml.eos_token_id", -1));
  ORC_CHECK(c.n_layers > 0 && c.hidden > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.intermediate > 0,
            "incomplete qwen3 metadata");
  ORC_CHECK(c.n_heads % c.n_kv_heads == 0, "heads %d not a multiple of kv heads %d", c.n_heads, c.n_kv_heads);
  if (c.context_length <= 0) c.context_length = 4096;
  ORC_CHECK(g.array_len.count("tokenizer.ggml.tokens"), "no tokenizer.ggml.tokens");
  c.vocab = static_cast<int32_t>(g.array_len["tokenizer.ggml.tokens"]);

  auto mat = [&](const std::string& name, int64_t rows, int64_t cols) {
    auto it = g.tensors.find(name);
    ORC_CHECK(it != g.tensors.end(), "tensor %s not found", name.c_str());
    const TensorInfo& t = it->second;
    ORC_CHECK(t.dims.size() == 2 && t.dims[1] == rows && t.dims[0] == cols,
              "tensor %s has the wrong shape", name.c_str());
    Matrix mx;
    mx.data = g.data(t);
    mx.type = t.type;
    mx.rows = rows;
    mx.cols = cols;
    return mx;
  };
  auto norm = [&](const std::string& name, int64_t n) {
    auto it = g.tensors.find(name);
    ORC_CHECK(it != g.tensors.end(), "tensor %s not found", name.c_str());
    const TensorInfo& t = it->second;
    ORC_CHECK(t.dims.size() == 1 && t.dims[0] == n, "norm %s has the wrong shape", name.c_str());
    std::vector<float> v(static_cast<size_t>(n));
    DequantizeRow(t.type, g.data(t), n, v.data());
    return v;
  };
  m->embd_ = mat("token_embd.weight", c.vocab, c.hidden);
  m->lm_head_ = g.tensors.count("output.weight") ? mat("output.weight", c.vocab, c.hidden) : m->embd_;
  m->output_norm_ = norm("output_norm.weight", c.hidden);
  m->layers_.resize(static_cast<size_t>(c.n_layers));
  for (int l = 0; l < c.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    Layer& w = m->layers_[static_cast<size_t>(l)];
    w.attn_norm = norm(p + "attn_norm.weight", c.hidden);
    w.ffn_norm = norm(p + "ffn_norm.weight", c.hidden);
    w.q_norm = norm(p + "attn_q_norm.weight", c.head_dim);
    w.k_norm = norm(p + "attn_k_norm.weight", c.head_dim);
    w.q = mat(p + "attn_q.weight", c.q_dim(), c.hidden);
    w.k = mat(p + "attn_k.weight", c.kv_dim(), c.hidden);
    w.v = mat(p + "attn_v.weight", c.kv_dim(), c.hidden);
    w.o = mat(p + "attn_output.weight", c.hidden, c.q_dim());
    w.gate = mat(p + "ffn_gate.weight", c.intermediate, c.hidden);
    w.up = mat(p + "ffn_up.weight", c.intermediate, c.hidden);
    w.down = mat(p + "ffn_down.weight", c.hidden, c.intermediate);
  }
  m->pool_.reset(new Pool(threads > 0 ? threads : PhysicalCores()));

  // RoPE table (reference src/model.cc:122-145): inv[i] = 1/theta^(2i/hd) in
  // double, angle p*inv[i] in double, cos/sin rounded to float.
  const int32_t half = c.head_dim / 2;
  m->n_rope_ = max_pos > c.context_length ? c.context_length : max_pos;
  if (m->n_rope_ <= 0) m->n_rope_ = 1;
  m->rope_.assign(static_cast<size_t>(m->n_rope_) * half * 2, 0.0f);
  std::vector<double> inv(static_cast<size_t>(half));
  for (int32_t i = 0; i < half; ++i) {
    inv[i] = 1.0 / std::pow(static_cast<double>(c.rope_theta),
                            static_cast<double>(2 * i) / static_cast<double>(c.head_dim));
  }
  for (int64_t p = 0; p < m->n_rope_; ++p) {
    float* row = m->rope_.data() + p * half * 2;
    for (int32_t i = 0; i < half; ++i) {
      const double ang = static_cast<double>(p) * inv[i];
      row[i] = static_cast<float>(std::cos(ang));
      row[half + i] = static_cast<float>(std::sin(ang));
    }
  }
  return m;
}

}  // namespace orc
