// Qwen3 model resident on one GPU.
//
// Load follows reference src/model.cc:147-281: every shape comes from GGUF
// metadata (head_dim only from attention.key_length), each tensor is shape-
// checked, norms are F32 vectors, lm_head is token_embd when output.weight is
// absent (tied). Raw GGUF blocks are copied once into one device arena, each
// tensor at a 256-byte aligned offset, layout unchanged (row-major rows of
// blocks); the prefill GEMMs, the embedding gather and the fallback matvecs
// read it. Every projection the matrix-core decode matvec runs also gets a
// tile-major copy in a second allocation (k::TileMajor, gate and up
// interleaved as one pair), read by the decode step only. The RoPE table is built on the host in double exactly as the
// reference does (src/model.cc:122-145) and uploaded.

#ifndef RPG_HIP_MODEL_H_
#define RPG_HIP_MODEL_H_

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "gguf.h"
#include "kernels.h"

namespace rpg {

struct ModelConfig {
  std::string arch, name;
  int32_t n_layers = 0, hidden = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, value_dim = 0;
  int32_t intermediate = 0, vocab = 0, context_length = 0;
  float rope_theta = 10000.0f, rms_eps = 1e-6f;
  bool tied_embeddings = false;
  int32_t bos_id = -1, eos_id = -1, pad_id = -1;
  bool add_bos = false;
  int32_t q_dim() const { return n_heads * head_dim; }
  int32_t kv_dim() const { return n_kv_heads * head_dim; }
  int32_t group() const { return n_kv_heads > 0 ? n_heads / n_kv_heads : 0; }
};

struct LayerDev {
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
  k::MatRef q, k, v, o, gate, up, down;
  // tile-major decode copies (w == nullptr: none; gate_up is the pair)
  k::MatRef dq, dk, dv, dout, gate_up, ddown;
};

class DeviceModel {
 public:
  // max_pos: RoPE positions (clipped to context_length, reference src/model.cc:124).
  static std::unique_ptr<DeviceModel> Load(const std::string& path, int32_t max_pos);
  ~DeviceModel();

  const ModelConfig& config() const { return cfg_; }
  const GgufFile& gguf() const { return *gguf_; }
  const std::vector<LayerDev>& layers() const { return layers_; }
  const k::MatRef& embd() const { return embd_; }
  const k::MatRef& lm_head() const { return lm_head_; }
  const k::MatRef& lm_head_tiled() const { return lm_head_t_; }
  const float* output_norm() const { return output_norm_; }
  const float* rope() const { return rope_dev_; }
  const std::vector<float>& rope_host() const { return rope_host_; }
  int64_t rope_positions() const { return n_rope_; }
  int64_t weight_bytes() const { return weight_bytes_; }
  int device() const { return device_; }
  // Bytes streamed from HBM per decode token for weights (every matrix once,
  // lm_head included, one embedding row, all norm vectors).
  int64_t decode_weight_bytes() const;

 private:
  DeviceModel() = default;
  std::unique_ptr<GgufFile> gguf_;
  ModelConfig cfg_;
  int device_ = 0;
  uint8_t* arena_ = nullptr;  // device
  int64_t arena_bytes_ = 0;
  uint8_t* tiled_ = nullptr;  // device: the tile-major decode copies
  int64_t tiled_bytes_ = 0;
  int64_t weight_bytes_ = 0;
  std::vector<LayerDev> layers_;
  k::MatRef embd_, lm_head_, lm_head_t_;
  const float* output_norm_ = nullptr;
  float* rope_dev_ = nullptr;
  float* norms_f32_ = nullptr;  // device: norm gains stored in another type, dequantised
  std::vector<float> rope_host_;
  int64_t n_rope_ = 0;
};

}  // namespace rpg

#endif  // RPG_HIP_MODEL_H_
