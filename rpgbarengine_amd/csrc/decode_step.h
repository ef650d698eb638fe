// The whole decode forward of one token as one persistent launch.
//
// A decode token runs, per layer, six dependent steps (norm + QKV, attention
// split, attention merge, O + residual, norm + gate/up + SwiGLU, down +
// residual), then norm + lm_head (reference src/qwen3.cc:119-206,276-289).
// As separate launches each step pays a kernel boundary plus the ramp of
// its first weight loads; here one workgroup per compute unit walks all the
// steps ("phases") in order. Between phases the activations travel as
// epoch-tagged 64-bit words (value | tag << 32, tag = epoch * kTagSpan +
// phase), stored and loaded at device coherence: a consumer issues its own
// weight loads for the phase first, then reads its input and checks the
// tags -- the read itself is the wait, retried with a back-off until every
// word carries the phase's tag. Every wait is bounded: past the limit the
// workgroup sets an error flag and leaves, so the launch always drains.
// The arithmetic is that of the per-launch kernels (mfma_dot.h, decode.hip).

#ifndef RPG_HIP_DECODE_STEP_H_
#define RPG_HIP_DECODE_STEP_H_

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace rpg {
namespace k {

constexpr int kStepWaves = 8;
constexpr int kStepThreads = 64 * kStepWaves;
constexpr int kTagSpan = 1024;  // phases per token: 1 + 6 * layers + 1 must fit

// Weights and cache of one layer (tile-major copies, decode.h).
struct StepLayer {
  const uint8_t* w[6];  // q, k, v, o, gate/up pair, down
  int32_t type[6];      // kQ4_K or kQ6_K
  int32_t kwl[6];       // log2 waves per tile of each projection (q, k, v share kwl[0])
  const float* attn_norm;
  const float* ffn_norm;
  const float* q_norm;
  const float* k_norm;
  float* kcache;  // [n_kv][max_seq][128]
  float* vcache;
};

struct StepArgs {
  const StepLayer* layers;  // device [n_layers]
  int32_t n_layers, H, qd, kvd, F, V, n_heads, n_kv;
  int64_t max_seq;
  float eps;
  const float* rope;  // [max_pos][128]
  MatRef embd;        // row-major token embedding (the gather)
  const uint8_t* lm_head;  // tile-major
  int32_t lm_type, lm_kwl;
  const float* output_norm;
  // tagged activations (uint2: value bits, tag)
  uint2 *x, *q, *k, *v, *attn, *act, *part;  // part: [n_heads][splits of max_seq][2 + 128]
  float* logits;
  const int32_t* token;  // device scalars
  const int32_t* pos;    // pos[0] position, pos[1] epoch
  int32_t* out_ids;      // token record: out_ids[*step] = token
  const int32_t* step;
  int32_t* err;          // set when a bounded wait gives up
};

// Bytes of LDS the launch takes (one workgroup per compute unit).
size_t DecodeStepLds(const StepArgs& a);
// True when the model fits the persistent step: Q4_K / Q6_K tile-major
// projections, K <= 10240, GQA group <= 7, head_dim 128, and a workgroup per
// compute unit fits. groups: the launch width (compute units).
bool DecodeStepSupported(const StepArgs& a, int groups);
void DecodeStep(const StepArgs& a, int groups, hipStream_t s);

}  // namespace k
}  // namespace rpg

#endif  // RPG_HIP_DECODE_STEP_H_
