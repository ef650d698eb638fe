// The transformer layers of a multi-token forward, shared by a session's
// prefill segment and a batch of sessions' decode step (reference
// src/qwen3.cc:119-206: per layer RMSNorm -> QKV -> QK-norm/RoPE/cache ->
// attention -> O + residual -> RMSNorm -> gate/up -> SwiGLU -> down +
// residual). The projections run on the matrix-core GEMMs where the weight
// type has one, else on the fused dequant matvec; only the attention step
// differs between the callers.

#ifndef RPG_HIP_FORWARD_H_
#define RPG_HIP_FORWARD_H_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>
#include <utility>

#include "common.h"
#include "kernels.h"
#include "model.h"
#include "prefill.h"

namespace rpg {

// Device buffers (N tokens) and streams of one forward. split: SplitXBytes(N,
// max K, split_cols) bytes; gu: [2][N][intermediate]; h: [N][max K].
struct FwdBufs {
  float *x, *h, *q, *k, *v, *attn, *act, *gu;
  void* split;
  int split_cols;
  hipStream_t stream, side;
  hipEvent_t ev_fork, ev_join;
};

// Output columns of the widest GEMM launch that may split its K range (the
// QKV projections; the gate+up pair never needs to): sizes the partials.
inline int SplitColumns(const ModelConfig& c) { return std::max(c.hidden, c.q_dim() + 2 * c.kv_dim()); }

// Every layer for N tokens whose embeddings are in b.x (row stride hidden).
// attend(l, w) computes layer l's attention from the raw projections b.q,
// b.k, b.v into b.attn (and writes the cache). On return b.x holds the final
// residual stream, every pending split-K sum applied.
template <typename Attend>
void ForwardLayers(const DeviceModel& m, const FwdBufs& b, int N, Attend attend) {
  const ModelConfig& c = m.config();
  const int H = c.hidden, F = c.intermediate, qd = c.q_dim(), kvd = c.kv_dim();
  float* const x = b.x;
  const hipStream_t stream = b.stream;
  // Projections of several tokens run on the matrix cores where the weight
  // type has a GEMM (the input split once per input vector set), the rest on
  // the fused dequant matvec.
  const bool mma = N >= 2;
  // With norm_w set, the projections take RMSNorm(in): folded into the
  // operand split when every job has a GEMM, else normed into b.h first.
  // Split-K sums of the last residual projection (O or down) not yet added
  // to x: the next split of x adds them (SplitRowsAdd), any other reader
  // gets them applied first.
  k::SplitPending pend;
  auto settle = [&]() {
    k::ApplyPending(pend, x, H, H, stream);
    pend = k::SplitPending{};
  };
  // A few tokens (the decode step of a batch of sessions) run on the
  // multi-token matrix-core matvec over the tile-major copies, the RMSNorm
  // folded into its staging; returns false when a job has no such copy.
  const bool few = N <= k::FewTokenLimit();
  auto batch = [&](const float* in, int K, const float* norm_w, bool pair,
                   std::initializer_list<std::pair<const k::MatRef*, k::GemmJob>> jobs) {
    if (!few) return false;
    k::DecodeBatchArgs a;
    a.n_jobs = 0;
    for (const auto& jb : jobs) {
      if (jb.first == nullptr || jb.first->w == nullptr) return false;
      k::DecodeJob& J = a.job[a.n_jobs];
      J.w = jb.first->w;
      J.row_bytes = jb.first->row_bytes;
      J.type = jb.first->type;
      J.rows = jb.first->rows;
      J.y = jb.second.y;
      J.tiled = 1;
      J.pair = pair ? 1 : 0;
      a.ldy[a.n_jobs] = jb.second.ldy;
      a.epi = jb.second.epi;
      ++a.n_jobs;
    }
    settle();
    a.x = in;
    a.ldx = K;
    a.T = N;
    a.K = K;
    a.norm_w = norm_w;
    a.eps = c.rms_eps;
    return k::DecodeMatvecBatch(a, stream);
  };
  auto project = [&](const float* in, int K, const float* norm_w,
                     std::initializer_list<std::pair<const k::MatRef*, k::GemmJob>> jobs) {
    bool all_gemm = mma;
    for (const auto& jb : jobs) all_gemm = all_gemm && k::QGemmSupports(*jb.first);
    if (in != x || !all_gemm) settle();
    if (norm_w != nullptr && !all_gemm) {
      k::RmsNormRows(in, K, norm_w, K, N, c.rms_eps, b.h, K, stream);
      in = b.h;
      norm_w = nullptr;
    }
    k::GemmJob g[3];
    int ng = 0;
    for (const auto& jb : jobs) {
      if (mma && k::QGemmSupports(*jb.first)) {
        g[ng++] = jb.second;
      } else {
        k::Matvec(*jb.first, in, K, N, jb.second.y, jb.second.ldy, jb.second.epi, stream);
      }
    }
    if (ng == 0) return;
    const k::SplitX sx = k::SplitXView(b.split, N, K, b.split_cols);
    k::SplitRowsAdd(const_cast<float*>(in), K, N, K, norm_w, c.rms_eps, sx, pend, stream);
    pend = k::SplitPending{};
    // one launch per weight type; a second type runs on the side stream
    // beside the first, each with half of the split-K partial buffer
    k::GemmJob grp[3][3];
    int gn[3] = {0, 0, 0}, n_grp = 0;
    bool done[3] = {false, false, false};
    for (int i = 0; i < ng; ++i) {
      if (done[i]) continue;
      for (int j = i; j < ng; ++j) {
        if (!done[j] && g[j].w.type == g[i].w.type) {
          grp[n_grp][gn[n_grp]++] = g[j];
          done[j] = true;
        }
      }
      ++n_grp;
    }
    if (n_grp == 2) {
      k::SplitX sa = sx, sb = sx;
      sa.part_floats = sx.part_floats / 2;
      sb.part_floats = sx.part_floats / 2;
      sb.part = sx.part + sa.part_floats;
      HIP_CHECK(hipEventRecord(b.ev_fork, stream));
      HIP_CHECK(hipStreamWaitEvent(b.side, b.ev_fork, 0));
      k::QGemm(sb, grp[1], gn[1], b.side);
      HIP_CHECK(hipEventRecord(b.ev_join, b.side));
      k::QGemm(sa, grp[0], gn[0], stream);
      HIP_CHECK(hipStreamWaitEvent(stream, b.ev_join, 0));
    } else if (n_grp == 1 && gn[0] == 1 && grp[0][0].y == x && grp[0][0].epi == k::kAdd) {
      k::QGemm(sx, grp[0], 1, stream, &pend);  // a K split's sums stay pending
    } else {
      for (int i = 0; i < n_grp; ++i) k::QGemm(sx, grp[i], gn[i], stream);
    }
  };
  auto gj = [](const k::MatRef& w, float* y, int64_t ldy, k::Epilogue epi) {
    k::GemmJob j;
    j.w = w;
    j.y = y;
    j.ldy = ldy;
    j.epi = epi;
    return std::make_pair(&w, j);
  };
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerDev& w = m.layers()[static_cast<size_t>(l)];
    if (!batch(x, H, w.attn_norm, false,
               {gj(w.dq, b.q, qd, k::kStore), gj(w.dk, b.k, kvd, k::kStore), gj(w.dv, b.v, kvd, k::kStore)}))
      project(x, H, w.attn_norm,
              {gj(w.q, b.q, qd, k::kStore), gj(w.k, b.k, kvd, k::kStore), gj(w.v, b.v, kvd, k::kStore)});
    attend(l, w);
    if (!batch(b.attn, qd, nullptr, false, {gj(w.dout, x, H, k::kAdd)}))
      project(b.attn, qd, nullptr, {gj(w.o, x, H, k::kAdd)});
    if (batch(x, H, w.ffn_norm, true, {gj(w.gate_up, b.act, F, k::kStore)})) {
      // silu(gate) * up in the one launch
    } else if (mma && k::QGemmSupports(w.gate) && k::QGemmSupports(w.up) && w.gate.type == w.up.type) {
      // one launch computes silu(gate) * up where the kernel allows, else
      // both products and the SwiGLU pass
      const k::SplitX sx = k::SplitXView(b.split, N, H, b.split_cols);
      k::SplitRowsAdd(x, H, N, H, w.ffn_norm, c.rms_eps, sx, pend, stream);
      pend = k::SplitPending{};
      if (!k::QGemmSwiGLU(sx, gj(w.gate, b.act, F, k::kStore).second, gj(w.up, nullptr, F, k::kStore).second,
                          stream)) {
        float* g = b.gu;
        float* u = b.gu + static_cast<int64_t>(N) * F;
        const k::GemmJob both[2] = {gj(w.gate, g, F, k::kStore).second, gj(w.up, u, F, k::kStore).second};
        k::QGemm(sx, both, 2, stream);
        k::SwiGLURows(g, u, b.act, static_cast<int64_t>(N) * F, stream);
      }
    } else {
      settle();
      k::RmsNormRows(x, H, w.ffn_norm, H, N, c.rms_eps, b.h, H, stream);
      k::MatvecSwiGLU(w.gate, w.up, b.h, H, N, b.act, F, stream);
    }
    if (!batch(b.act, F, nullptr, false, {gj(w.ddown, x, H, k::kAdd)}))
      project(b.act, F, nullptr, {gj(w.down, x, H, k::kAdd)});
  }
  settle();
}

}  // namespace rpg

#endif  // RPG_HIP_FORWARD_H_
