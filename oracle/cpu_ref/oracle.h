// oracle.h -- CPU restatement of the reference Qwen3 token loop.
//
// TEST INFRASTRUCTURE, NOT PRODUCT. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load liboracle.so, and only to check or time
// the engine against it.
// The HIP engine never links or calls it.
//
// Every function restates one reference function (file:line given beside it)
// with the same floating-point operation order, so that -- compiled with the
// reference's flags (oracle/Makefile) -- it returns the same bits. Parity
// pins (tests/test_oracle.py): bitwise against the reference built from its
// own sources (oracle/_ref/ref_golden) on committed golden vectors, plus
// closed forms (Q8_0 KAT, exhaustive 6-bit scale unpack, sampler KATs of
// reference tools/selftest.cc:546-645, brute-force float64 dots).

#ifndef RPG_ORACLE_H
#define RPG_ORACLE_H

#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace orc {

// ggml type ids (reference src/quant.h)
enum : uint32_t {
  kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ8_1 = 9, kQ2_K = 10,
  kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kQ8_K = 15, kBF16 = 30,
};

[[noreturn]] void Fail(const char* fmt, ...);
#define ORC_CHECK(cond, ...) \
  do {                       \
    if (!(cond)) ::orc::Fail(__VA_ARGS__); \
  } while (0)

// f16 -> f32, bit-exact including NaN payloads (reference src/dtypes.h:21-47).
inline float HalfToFloat(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      // normalise the subnormal: shift until the implicit bit appears
      int shift = 0;
      while ((m & 0x400u) == 0) {
        m <<= 1;
        ++shift;
      }
      bits = sign | (static_cast<uint32_t>(113 - shift) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

inline uint16_t Load16(const uint8_t* p) {
  uint16_t v;
  std::memcpy(&v, p, 2);
  return v;
}

int64_t BlockElems(uint32_t type);
int64_t BlockBytes(uint32_t type);
int64_t RowBytes(uint32_t type, int64_t n);

// ---- quant.cc: DequantizeRow (reference src/quant.cc:416-436)
void DequantizeRow(uint32_t type, const uint8_t* src, int64_t n, float* dst);
// 6-bit (scale, min) unpack (reference src/quant.cc:159-167)
void ScaleMinK4(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn);

// ---- dot_scalar.cc: DotRowQuantRef (reference src/matmul.cc:73-102)
float DotRowScalar(uint32_t type, const float* a, const uint8_t* w, int64_t k);

// ---- dot_avx2.cc (reference src/matmul_avx2.cc)
bool Avx2Available();
float DotRowAvx2(uint32_t type, const float* a, const uint8_t* w, int64_t k);
class Pool;
// false when the type has no blocked kernel or n_tokens < 8 (reference :482-507)
bool MatMulBlockedAvx2(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols,
                       const float* X, int64_t n_tokens, float* OUT, Pool* pool);

// Dispatch as reference src/matmul.cc:49-67,106-124 (RPGBAR_NO_SIMD honoured).
float DotRowQuant(uint32_t type, const float* a, const uint8_t* w, int64_t k);

// ---- pool.cc: row-partitioned thread pool (reference src/threads.cc:200-234)
class Pool {
 public:
  explicit Pool(int n_threads);
  ~Pool();
  int size() const;
  // body(begin, end) on equal chunks ceil(n / threads); caller runs chunk 0.
  void ParallelForRange(int64_t n, const std::function<void(int64_t, int64_t)>& body);

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};
int PhysicalCores();  // reference src/threads.cc:70-123

// ---- scalar kernels (reference src/kernels.h:26-120)
float Dot(const float* a, const float* b, int64_t n);
int32_t ArgMax(const float* x, int64_t n);
void RmsNorm(const float* x, const float* w, int64_t n, float eps, float* out);
void SoftmaxInPlace(float* x, int64_t n);
void SiluInPlace(float* x, int64_t n);
void MulInPlace(float* a, const float* b, int64_t n);
void VecAddInPlace(float* a, const float* b, int64_t n);
void RopeInPlace(float* x, int32_t n_heads, int32_t head_dim, const float* cos_t,
                 const float* sin_t);
// causal GQA attention of a segment from a cache (reference src/qwen3.cc:79-117)
void AttentionCache(int32_t n_heads, int32_t n_kv, int32_t hd, const float* q, int64_t seq, int64_t pos0,
                    const float* k, const float* v, float* out);

// ---- sampler.cc (reference src/sampler.cc:16-112)
uint64_t SplitMix64(uint64_t x);
uint64_t CounterRng(uint64_t seed, uint64_t counter);
float CounterUniform(uint64_t seed, uint64_t counter);
struct SampleOptions {
  float temperature = 1.0f;
  int32_t top_k = 0;
  float top_p = 1.0f;
};
void FilterToProbs(const float* logits, int64_t n, const SampleOptions& opt,
                   std::vector<float>* probs);
int32_t SampleToken(const float* logits, int64_t n, const SampleOptions& opt, float u);

// ---- gguf.cc / model.cc (reference src/gguf.cc:169-260, src/model.cc:122-281)
struct Matrix {
  const uint8_t* data = nullptr;
  uint32_t type = kF32;
  int64_t rows = 0;
  int64_t cols = 0;
  // reference src/model.cc:32-37
  void Row(int64_t r, float* out) const;
  // reference src/model.cc:39-69
  void MatMulBatch(const float* X, int64_t n, float* OUT, Pool* pool) const;
};

struct Config {
  int32_t n_layers = 0, hidden = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0;
  int32_t intermediate = 0, vocab = 0, context_length = 0;
  float rope_theta = 10000.0f, rms_eps = 1e-6f;
  int32_t eos_id = -1;
  int32_t q_dim() const { return n_heads * head_dim; }
  int32_t kv_dim() const { return n_kv_heads * head_dim; }
  int32_t group() const { return n_heads / n_kv_heads; }
};

struct Layer {
  std::vector<float> attn_norm, ffn_norm, q_norm, k_norm;
  Matrix q, k, v, o, gate, up, down;
};

class GgufMap;  // read-only mapping + parsed header

class Model {
 public:
  static std::unique_ptr<Model> Load(const std::string& path, int threads, int32_t max_pos);
  ~Model();
  const Config& config() const { return cfg_; }
  Pool& pool() const { return *pool_; }
  const Matrix& embd() const { return embd_; }
  const Matrix& lm_head() const { return lm_head_; }
  const std::vector<float>& output_norm() const { return output_norm_; }
  const std::vector<Layer>& layers() const { return layers_; }
  int64_t rope_positions() const { return n_rope_; }
  const float* rope_cos(int64_t p) const { return rope_.data() + p * cfg_.head_dim; }
  const float* rope_sin(int64_t p) const { return rope_.data() + p * cfg_.head_dim + cfg_.head_dim / 2; }

 private:
  Model() = default;
  std::unique_ptr<GgufMap> file_;
  Config cfg_;
  std::unique_ptr<Pool> pool_;
  Matrix embd_, lm_head_;
  std::vector<float> output_norm_;
  std::vector<Layer> layers_;
  std::vector<float> rope_;
  int64_t n_rope_ = 0;
};

// fp32 [L, n_kv, max_seq, hd], K and V separate (reference src/kv_cache.cc:7-83)
struct KvCache {
  KvCache(const Config& c, int64_t max_seq);
  int32_t n_layers, n_kv, hd;
  int64_t max_seq, len = 0;
  // Measurement only (the reference keeps fp32): round every K / V value
  // written to the nearest fp16 (ties to even, as a GPU fp16 cache would
  // store it) and keep it as that float.
  bool fp16 = false;
  std::vector<float> k, v;
  float* K(int32_t l, int32_t h, int64_t p) { return k.data() + ((int64_t(l) * n_kv + h) * max_seq + p) * hd; }
  float* V(int32_t l, int32_t h, int64_t p) { return v.data() + ((int64_t(l) * n_kv + h) * max_seq + p) * hd; }
};

// The nearest fp16 value (ties to even) as a float (the fp16-cache measurement).
float RoundToHalf(float x);

// ---- forward.cc (reference src/qwen3.cc:44-363)
// logits: [seq, vocab]; kv may be null (no-cache full-sequence path).
void ForwardFull(const Model& m, const int32_t* tokens, int64_t seq,
                 std::vector<float>* logits, KvCache* kv);
struct GenerateOptions {
  int32_t max_tokens = 64;
  std::vector<int32_t> stop_ids;
  SampleOptions sample;
  uint64_t seed = 0;
};
// step_logits (optional): logits after each generated token ([n_out, vocab]).
void Generate(const Model& m, KvCache* kv, const float* first_logits,
              const GenerateOptions& opt, std::vector<int32_t>* out_ids,
              std::vector<float>* step_logits);

}  // namespace orc

#endif  // RPG_ORACLE_H
