// One-token (decode) kernels: fused norm + matvec tiles, fused QK-norm /
// RoPE / cache-write / split-K attention. Device pointers throughout.

#ifndef RPG_HIP_DECODE_H_
#define RPG_HIP_DECODE_H_

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace rpg {
namespace k {

// One matrix of a decode matvec launch. w2 != nullptr makes it a SwiGLU pair:
// y[r] = silu(W[r].x) * (W2[r].x).
struct DecodeJob {
  const uint8_t* w = nullptr;
  int64_t row_bytes = 0;
  uint32_t type = 0;
  int32_t rows = 0;
  const uint8_t* w2 = nullptr;
  int64_t row_bytes2 = 0;
  uint32_t type2 = 0;
  float* y = nullptr;
  int32_t rows_per_tile = 1;  // virtual rows per wave tile, chosen by DecodeMatvec
  int32_t tiles = 0;          // filled by DecodeMatvec
  // w is a tile-major copy (TileMajor); row_bytes stays the row-major row
  // length. With pair set, tile rows 0..7 are rows of the first matrix of a
  // SwiGLU pair and rows 8..15 those of the second (w2 unused).
  int32_t tiled = 0;
  int32_t pair = 0;
};

struct DecodeMatvecArgs {
  DecodeJob job[3];
  int32_t n_jobs = 1;
  const float* x = nullptr;       // input vector [K]
  int32_t K = 0;
  const float* norm_w = nullptr;  // RMSNorm gain: stage RMSNorm(x) instead of x
  float eps = 1e-6f;
  int32_t epi = kStore;           // kStore / kAdd for single jobs
  int32_t* inc = nullptr;         // when set, the launch also adds 1 to *inc
};

void DecodeMatvec(DecodeMatvecArgs a, hipStream_t s);

// Widest input whose RMSNorm a decode matvec folds into its staging
// (norm_w); callers norm wider inputs first (RmsNormRows).
constexpr int kDecodeNormMaxK = 4096;

// The matrix-core path for launches whose jobs are all Q4_K / Q6_K with
// K % 256 == 0 (matvec_mfma.hip); returns false, launching nothing, when the
// launch does not qualify. DecodeMatvec tries it first.
bool DecodeMatvecMfma(const DecodeMatvecArgs& a, hipStream_t s);

// The matrix-core matvec for a few tokens at once (matvec_batch.hip): the
// decode step of a batch of sessions, prefill segments of a few tokens.
// y of job j is [T][ldy[j]]; a job with `pair` set writes silu(gate) * up.
// Every job must read a tile-major copy of a Q4_K / Q6_K matrix (w2 unused);
// returns false, launching nothing, when the launch does not qualify. Up to
// kMaxBatchTokens tokens per launch, in groups of 8 (or 4) tokens whose
// workgroups of one tile share an XCD (the weights are read from HBM once).
constexpr int kMaxBatchTokens = 64;
// Segments of at most this many tokens run their projections on the
// few-token matvec; longer ones on the matrix-core GEMMs (the crossover
// measured on the 1.7B / 4B projection shapes). RPG_FEW_TOKENS overrides it
// for tuning sweeps (1 .. kMaxBatchTokens).
int FewTokenLimit();
struct DecodeBatchArgs {
  DecodeJob job[3];
  int64_t ldy[3] = {0, 0, 0};
  int32_t n_jobs = 1;
  const float* x = nullptr;  // [T][ldx]
  int64_t ldx = 0;
  int32_t T = 1;
  int32_t K = 0;
  const float* norm_w = nullptr;  // RMSNorm gain: stage RMSNorm(x_t) instead of x_t
  float eps = 1e-6f;
  int32_t epi = kStore;
};
bool DecodeMatvecBatch(const DecodeBatchArgs& a, hipStream_t s);

// Tile-major decode copies. The matrix-core matvec reads a tile of 16 rows
// per wave; stored row-major, one wave load touches 16 pieces a row apart.
// The copy stores the GGUF blocks tile by tile and within a tile super-block
// by super-block: the chunk of (tile t, super-block b) at
// (t * n_sb + b) * 16 * block_bytes holds the 16 rows' blocks, rows past the
// end zero. Q4_K blocks are stored unchanged, one after another; a Q6_K
// chunk holds the same bytes grouped by field -- the 16 rows' ql (128 bytes
// each), then their qh (64), scales (16) and d (2) -- so that every lane
// load is aligned (the blocks are 210 bytes long). A SwiGLU pair interleaves
// its two matrices 8 + 8 rows per tile.
bool DecodeTileable(const MatRef& m);  // Q4_K / Q6_K / Q8_0 with cols % 256 == 0, cols <= 10240
bool BatchTileable(const MatRef& m);   // DecodeTileable and read by the few-token launches (all three types)
int64_t TileMajorBytes(const MatRef& m, bool pair);
void TileMajor(const MatRef& a, const MatRef* b, uint8_t* dst, hipStream_t s);

struct DecodeAttnArgs {
  const float* q;       // [n_heads * 128] raw projection
  const float* k;       // [n_kv * 128]
  const float* v;       // [n_kv * 128]
  const float* q_norm;  // [128]
  const float* k_norm;
  const float* rope;    // [max_pos][128]
  float* kcache;        // this layer: [n_kv][max_seq][128]
  float* vcache;
  float* out;           // [n_heads * 128]
  float* work;          // DecodeAttnWorkFloats(n_heads, n_kv, max_seq), the
                        // trailing n_kv counters zeroed once at allocation
  int32_t n_heads, n_kv;
  int64_t max_seq;
  float eps;
  const int32_t* pos_dev;
};
int64_t DecodeAttnWorkFloats(int n_heads, int n_kv, int64_t max_seq);
void DecodeAttention(const DecodeAttnArgs& a, hipStream_t s);

// DecodeAttention for a batch of sessions, one token each, in one pair of
// launches: session z reads its rows of q, k, v (base pointers + z * stride),
// its own cache and position (base.pos_dev[z]) and writes its rows of out
// and work. base.kcache / vcache / max_seq are unused.
constexpr int kMaxDecodeBatch = 8;
struct DecodeAttnBatchArgs {
  DecodeAttnArgs base;
  float* kcache[kMaxDecodeBatch];  // this layer of session z: [n_kv][max_seq[z]][128]
  float* vcache[kMaxDecodeBatch];
  int64_t max_seq[kMaxDecodeBatch];
  int64_t q_stride = 0, kv_stride = 0;  // floats between sessions' rows of q / out and of k / v
  int64_t work_stride = 0;              // >= DecodeAttnBatchWorkFloats(n_heads, max_seq_all)
};
int64_t DecodeAttnBatchWorkFloats(int n_heads, int64_t max_seq);
void DecodeAttentionBatch(const DecodeAttnBatchArgs& b, int sessions, int64_t max_seq_all, hipStream_t s);

}  // namespace k
}  // namespace rpg

#endif  // RPG_HIP_DECODE_H_
