// Multi-token (prefill) projections on the bf16/f16 matrix cores of gfx950.
//
// Y[t][n] = sum_k X[t][k] * W[n][k] for a segment of M tokens and a raw GGUF
// weight matrix W (Q4_K, Q6_K or Q8_0). The product runs on
// v_mfma_f32_16x16x32_f16 with operands that make it exact up to fp32
// accumulation:
//  * W side: the integer quants times their integer sub-block scales, which
//    are small enough to be exact in f16 (Q4_K: q*sc <= 945; Q6_K: (q-32)*sc
//    split into 16*(q-32)*floor(sc/16) and (q-32)*(sc mod 16); Q8_0: q);
//    the fp16 block scales d (and dmin) are applied in fp32 once per block.
//  * X side: each token row scaled by a power of two s so that max|x*s| lies
//    in [2^14, 2^15), then split x*s = hi + lo into two f16 (22 significant
//    bits), both multiplied into the same accumulator.
// SplitRows prepares the X side once per segment (optionally fused with the
// RMSNorm that produces it); QGemm runs up to three weight matrices over it.
// Results satisfy the matvec row bound max|d|/sum|a*w| <= 1e-6 of the
// reference's own dot kernels (reference src/matmul.cc:73-124).

#ifndef RPG_HIP_PREFILL_H_
#define RPG_HIP_PREFILL_H_

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace rpg {
namespace k {

// Device buffers of a split segment (M tokens, K inputs). Within every 8
// consecutive inputs the f16 copies are stored in the order 0,2,1,3,4,6,5,7
// (the order in which the weight operand is assembled from packed quants).
struct SplitX {
  void* hi = nullptr;      // f16 [M][K]
  void* lo = nullptr;      // f16 [M][K]
  void* sum_hi = nullptr;  // f16 [M][K/32]: sum of each 32 inputs * s/32, split
  void* sum_lo = nullptr;
  float* inv_s = nullptr;  // [M] 1/s
  float* part = nullptr;   // split-K partial products of QGemm
  int64_t part_floats = 0;
  int32_t M = 0, K = 0;
};
// Bytes of a SplitX for up to M x K whose QGemm launches produce at most
// n_max output columns in total (sizes the split-K partials).
size_t SplitXBytes(int M, int K, int n_max);
// Carve a SplitX out of `base` (SplitXBytes(M, K, n_max) bytes).
SplitX SplitXView(void* base, int M, int K, int n_max);

// x = X rows (stride ldx), or RMSNorm(x) * norm_w when norm_w != nullptr
// (double sum of squares, float scale, (x * scale) * w, reference
// src/kernels.h:56-63).
void SplitRows(const float* X, int64_t ldx, int M, int K, const float* norm_w, float eps, const SplitX& out,
               hipStream_t s);

// Split-K partial sums of a kAdd projection not yet added to its output:
// y[t][c] += sum over z < ksplit of part[(z * M + t) * part_ld + pcol + c].
struct SplitPending {
  const float* part = nullptr;
  int64_t part_ld = 0;
  int32_t pcol = 0, ksplit = 1, M = 0;
};
// SplitRows over X after adding the pending sums to X (written back: X is
// the residual stream), the bits of the reduce launch followed by SplitRows.
void SplitRowsAdd(float* X, int64_t ldx, int M, int K, const float* norm_w, float eps, const SplitX& out,
                  const SplitPending& pend, hipStream_t s);
// The reduce launch of a pending sum, into y (row stride ldy, N columns).
void ApplyPending(const SplitPending& pend, float* y, int64_t ldy, int N, hipStream_t s);

struct GemmJob {
  MatRef w;
  float* y = nullptr;
  int64_t ldy = 0;
  Epilogue epi = kStore;
};
// True when W can run on QGemm (K-quants need K a multiple of 256).
bool QGemmSupports(const MatRef& w);
void QGemm(const SplitX& x, const GemmJob* jobs, int n_jobs, hipStream_t s, SplitPending* defer = nullptr);
// (defer: for one kAdd job, a K split's sums are left to the caller -- to
// SplitRowsAdd or ApplyPending before y is read; defer->ksplit stays 1 when
// nothing is pending)
// gate.y[t][r] = silu(gate row r . x_t) * (up row r . x_t) in one launch,
// the same bits as two QGemm products and SwiGLURows -- except where a tiled
// launch runs its last round's tiles in K halves (more tiles than compute
// units, that round at most half full): those rows' sums are the halves'
// sums added, within the products' row bound. Q4_K gate and up of one shape
// only, and only where QGemm would not split K; false (nothing launched)
// otherwise.
bool QGemmSwiGLU(const SplitX& x, const GemmJob& gate, const GemmJob& up, hipStream_t s);

// y[i] = silu(g[i]) * u[i] (reference src/kernels.h:82-92), n elements.
void SwiGLURows(const float* g, const float* u, float* y, int64_t n, hipStream_t s);

// Tiled Q4_K / Q6_K GEMM (gemm_tiled.hip): 128 tokens x 128 weight rows per
// workgroup, each step's weights unpacked once into LDS. QGemm and QGemmSwiGLU
// take it for segments of at least kTiledMinTokens tokens.
constexpr int kTiledTokens = 128;
constexpr int kTiledRows = 128;
constexpr int kTiledMinTokens = 96;

struct TiledArgs {
  SplitX x;
  GemmJob job[3];
  int32_t tiles[3];  // 128-row tiles per job (pair: 64-row tiles of gate and up)
  int32_t n_jobs;
  int32_t tiles_m;   // 128-token tiles; workgroup i takes token tile i % tiles_m
  int32_t ksplit;    // blockIdx.y takes super-blocks [y * n / ksplit, (y + 1) * n / ksplit)
  int64_t part_ld;   // partials: x.part[(z * M + token) * part_ld + pcol[job] + row]
  int32_t pcol[3];
  int32_t pair;      // job 0 gate, job 1 up: y = silu(gate.x) * (up.x), no K split
  // pair only, 0 = none: workgroups from tail_wg on take the tiles from
  // tail_wg on in halves (the two super-block halves of each, raw sums to
  // x.part, kTiledTailFloats per half), finished by a second launch
  int32_t tail_wg = 0;
};
constexpr int kTiledTailFloats = kTiledTokens * kTiledRows;
void LaunchTiled(const TiledArgs& a, hipStream_t s);

}  // namespace k
}  // namespace rpg

#endif  // RPG_HIP_PREFILL_H_
