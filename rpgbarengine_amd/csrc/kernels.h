// Host launchers of the gfx950 kernels (implemented in kernels.hip,
// attention.hip, sampler.hip). All pointers are device pointers; every
// launcher enqueues on `stream` and returns without synchronising.

#ifndef RPG_HIP_KERNELS_H_
#define RPG_HIP_KERNELS_H_

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rpg {
namespace k {

// A quantised weight matrix in device memory: raw GGUF rows, row-major.
struct MatRef {
  const uint8_t* w = nullptr;
  uint32_t type = 0;
  int32_t rows = 0;
  int32_t cols = 0;
  int64_t row_bytes = 0;
};

enum Epilogue : int32_t {
  kStore = 0,  // Y = W.X
  kAdd = 1,    // Y += W.X   (residual add, reference src/qwen3.cc:186-188,203-205)
};

// Y[m*ldy + r] (=|+=) sum_c W[r][c] * X[m*ldx + c] for m < M, r < rows.
// Fused dequant, fp32 accumulation; any M >= 1 (processed 8 tokens at a time).
void Matvec(const MatRef& W, const float* X, int64_t ldx, int M, float* Y, int64_t ldy, Epilogue epi,
            hipStream_t s);

// Y[m*ldy + r] = silu(G[r].X_m) * (U[r].X_m) -- SwiGLU with glibc-exact expf
// (reference src/kernels.h:82-92).
void MatvecSwiGLU(const MatRef& G, const MatRef& U, const float* X, int64_t ldx, int M, float* Y, int64_t ldy,
                  hipStream_t s);

// out[i*ldo + c] = dequant(W row ids[i])[c], bit-exact (reference src/model.cc:32-37).
// ids is a device array of n token ids; ids outside [0, rows) set *err = 1.
// With rec_ids set the launch also records the tokens: for one id (decode)
// rec_ids[*rec_step] = ids[0], (*rec_step)++; with rec_ld > 0 (a decode
// batch) rec_ids[i * rec_ld + *rec_step] = ids[i] and the step is left to
// AdvancePositions.
void GatherRows(const MatRef& W, const int32_t* ids, int n, float* out, int64_t ldo, int32_t* err,
                hipStream_t s, int32_t* rec_ids = nullptr, int32_t* rec_step = nullptr, int64_t rec_ld = 0);

// pos[i]++ for i < n and, when step is set, (*step)++: the end of a batched
// decode step.
void AdvancePositions(int32_t* pos, int n, int32_t* step, hipStream_t s);

// Teacher forcing (parity tests): at the step *step, drawn[i * ld + *step] =
// tokens[i] (the id the sampler drew), then tokens[i] = force[i * ld + *step]
// (the id forwarded instead), for i < n.
void ForceTokens(int32_t* tokens, int n, const int32_t* force, int32_t* drawn, const int32_t* step, int64_t ld,
                 hipStream_t s);

// Bit-exact dequantisation of n elements of one tensor (reference src/quant.cc:416-436).
void Dequant(uint32_t type, const uint8_t* src, int64_t n, float* dst, hipStream_t s);

// out[r] = x[r] * scale_r * w (double sum of squares; reference src/kernels.h:56-63).
void RmsNormRows(const float* x, int64_t ldx, const float* w, int n, int rows, float eps, float* out,
                 int64_t ldo, hipStream_t s);

// Per token t of a segment starting at absolute position pos0 (device scalar
// when pos0_dev != nullptr, else pos0_host): RMSNorm every Q and K head with
// q_norm / k_norm, RoPE with the table row of position pos0+t, write K and V
// into the cache at that position (reference src/qwen3.cc:139-177).
struct QkvArgs {
  float* q;            // [seq, n_heads*hd]   in/out
  const float* k;      // [seq, n_kv*hd]      in
  const float* v;      // [seq, n_kv*hd]      in
  const float* q_norm; // [hd]
  const float* k_norm; // [hd]
  const float* rope;   // [max_pos, hd]: cos | sin halves
  float* kcache;       // this layer: [n_kv, max_seq, hd]
  float* vcache;
  int32_t seq, n_heads, n_kv, hd;
  int64_t max_seq;
  float eps;
  const int32_t* pos0_dev;
  int32_t pos0_host;
};
void QkNormRopeCache(const QkvArgs& a, hipStream_t s);

// Attention of `seq` queries at positions pos0..pos0+seq-1 over the cache
// (causal; reference src/qwen3.cc:79-117). out: [seq, n_heads*hd].
struct AttnArgs {
  const float* q;
  const float* kcache;  // this layer: [n_kv, max_seq, hd]
  const float* vcache;
  float* out;
  float* work;          // split-K partials (decode): see AttnWorkFloats
  int32_t seq, n_heads, n_kv, hd;
  int64_t max_seq;
  const int32_t* pos0_dev;
  int32_t pos0_host;
};
int64_t AttnWorkFloats(int n_heads, int64_t max_seq);
void Attention(const AttnArgs& a, hipStream_t s);

// First index of the maximum of each row (reference src/kernels.h:42-52).
// Index of the first maximum of each row (NaN never wins; a NaN first
// element gives 0). With `pair` (two 64-bit words of device memory, zero
// before the first call, left zero by every call) a single row is picked by
// many workgroups at once.
void ArgMaxRows(const float* x, int64_t ldx, int n, int rows, int32_t* out, hipStream_t s, uint64_t* pair = nullptr);

}  // namespace k
}  // namespace rpg

#endif  // RPG_HIP_KERNELS_H_
