/* rpg_synth.h -- synthetic Qwen3 GGUF models and block quantizers.
 *
 * Test and benchmark input generator. CPU only; no GPU calls. The reference
 * engine ships no quantizer and no model files, so every parity test and every
 * benchmark in this repository reads GGUF files written by this library:
 * the CPU oracle and the HIP engine then read the very same bytes.
 *
 * Weights are N(0, weight_std) per tensor from a counter-based generator
 * (SplitMix64 -> Box-Muller in double -> float), seeded by (seed, tensor name,
 * row), so the output does not depend on the thread count. Norm gains are
 * 1 + N(0, norm_std). The GGUF layout follows the GGUF v3 format that the
 * reference reads (reference src/gguf.cc:169-260): little-endian header,
 * metadata key/values, tensor infos, data aligned to general.alignment = 32.
 */
#ifndef RPG_SYNTH_H
#define RPG_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (reference src/quant.h:22-38). */
#define RPG_GGML_F32 0
#define RPG_GGML_F16 1
#define RPG_GGML_Q4_0 2
#define RPG_GGML_Q4_1 3
#define RPG_GGML_Q5_0 6
#define RPG_GGML_Q5_1 7
#define RPG_GGML_Q8_0 8
#define RPG_GGML_Q8_1 9
#define RPG_GGML_Q2_K 10
#define RPG_GGML_Q3_K 11
#define RPG_GGML_Q4_K 12
#define RPG_GGML_Q5_K 13
#define RPG_GGML_Q6_K 14
#define RPG_GGML_Q8_K 15
#define RPG_GGML_BF16 30

/* Quantisation mixes for the 2-D weights. */
#define RPG_MIX_Q8_0 0   /* every matrix Q8_0, token_embd included */
#define RPG_MIX_Q4_K_M 1 /* Q4_K; attn_v, ffn_down of even layers, token_embd: Q6_K */
#define RPG_MIX_F32 2    /* every matrix F32 (tiny exact tests) */
#define RPG_MIX_Q4_K 3   /* every matrix Q4_K */
#define RPG_MIX_Q6_K 4   /* every matrix Q6_K */
#define RPG_MIX_OTHER 5  /* the matrices cycle through Q4_0, Q4_1, Q5_0, Q5_1,
                            Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, F16, BF16 (token_embd
                            Q5_K); attn_norm F16 and ffn_norm BF16 gains */

typedef struct rpg_synth_spec {
  int32_t n_layers;
  int32_t hidden;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t ffn;
  int32_t vocab;
  int32_t context_length;
  float rope_theta;
  float rms_eps;
  int32_t mix;
  uint64_t seed;
  float weight_std;
  float norm_std;
  /* 0: placeholder vocabulary ("<tN>" tokens, one merge); 1: a byte-level
   * BPE vocabulary -- the 256 byte tokens, merges learned from a built-in
   * multilingual corpus, Qwen's 26 added tokens (<|endoftext|>, <|im_start|>,
   * <|im_end|>, ..., <tool_call>, <think>, ...; bos / pad <|endoftext|>, eos
   * <|im_end|>) and unused [PADn] entries up to the vocabulary size. */
  int32_t tokenizer;
} rpg_synth_spec;

/* Fill *spec with the defaults (theta 1e6, eps 1e-6, std 0.02 / 0.01,
 * context 4096, mix Q8_0, seed 1) -- shape fields are zeroed. */
void rpg_synth_default_spec(rpg_synth_spec* spec);

/* Write a complete qwen3 GGUF to `path`. Returns 0 on success, -1 on failure
 * (message in rpg_synth_last_error()). n_threads <= 0: hardware threads. */
int32_t rpg_synth_write_gguf(const char* path, const rpg_synth_spec* spec,
                             int32_t n_threads);

/* Quantise n floats (n a multiple of the type's block size) into dst.
 * Returns the number of bytes written, or -1. Every type above. */
int64_t rpg_synth_quantize(uint32_t type, const float* src, int64_t n,
                           uint8_t* dst);

/* Bytes of one row of n elements of `type` (-1 if n is not a block multiple). */
int64_t rpg_synth_row_bytes(uint32_t type, int64_t n);

/* n samples of N(0, std) from stream (seed, stream), element i depends only
 * on (seed, stream, i). */
void rpg_synth_gaussian(uint64_t seed, uint64_t stream, int64_t n, float std,
                        float* out);

/* n uniform token ids in [0, vocab) from (seed, i). */
void rpg_synth_token_ids(uint64_t seed, int64_t n, int32_t vocab, int32_t* out);

const char* rpg_synth_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* RPG_SYNTH_H */
