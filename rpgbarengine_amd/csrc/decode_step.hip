// The persistent decode step (decode_step.h): one launch walks every phase of
// one token's forward, one workgroup of 8 waves per compute unit.
//
// Phases, in order (global index p; tag of its outputs = epoch * kTagSpan + p):
//   p = 0            embedding row -> x (each workgroup its slice); the token
//                    is recorded in out_ids
//   p = 1 + 6 l + 0  RMSNorm(x) . [Wq | Wk | Wv] -> q, k, v
//               + 1  QK-norm + RoPE + cache write + attention partials per
//                    (KV head, 32 positions) -> part
//               + 2  merge of the partials per query head -> attn
//               + 3  x += Wo . attn
//               + 4  act = silu(Wg . RMSNorm(x)) * (Wu . RMSNorm(x))
//               + 5  x += Wd . act
//   p = 1 + 6 L      RMSNorm(x) . Wlm -> logits (plain stores: read after
//                    the launch)
// A matrix phase hands out "slots" of 8 / kw tiles (16 output rows each, kw
// waves per tile splitting its super-blocks and adding in a fixed order):
// workgroup b takes slots b, b + groups, ... Each wave issues its first
// weight batch, then the workgroup reads its tagged input until every word
// is current (the wait), stages it once per phase (mfma_dot.h), and streams
// the rest. Dependencies only point to earlier phases, and every workgroup of
// the launch is resident (one per compute unit), so every wait ends; a
// spin limit turns a wait that does not end into an error flag instead.
//
// Write-after-read: a buffer is rewritten only by a phase whose inputs
// needed every reader of its previous contents to have finished (x by O and
// down, whose inputs come from phases that read all of x), so one copy of
// each activation suffices.

#include "decode_step.h"

#include <hip/hip_runtime.h>

#include "common.h"
#include "decode.h"
#include "expf_glibc.h"
#include "lanes.h"
#include "soft_exp.h"
#include "mfma_dot.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

using namespace mfma;
using lanes::WaveMaxF;
using lanes::WaveSumD;
using lanes::WaveSumF;

constexpr int NW = kStepWaves, NT = kStepThreads;
constexpr int kMaxLayers = 64;
constexpr int kSpinLimit = 1 << 20;  // ~1-2 s of polling before a wait gives up
constexpr int kHdS = 128;
constexpr int kSplitS = 32;          // cache positions per attention item
constexpr int kPartS = 2 + kHdS;     // partial record: max, sum, 128 outputs
constexpr int kKStrideS = kHdS + 4;  // padded K rows in LDS
constexpr int kMaxSplitsS = 256;     // up to 8192 positions
constexpr int kCpolSc1 = 16;         // buffer-load cache policy: device-coherent (sc1)

typedef float F2v __attribute__((ext_vector_type(2)));

// A field of the layer table in LDS, made wave-uniform (scalar registers).
template <typename T>
__device__ __forceinline__ T LdsField(const T& f) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t v = __builtin_bit_cast(uint64_t, f);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
    return __builtin_bit_cast(T, lo | (hi << 32));
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, f)));
  }
}

__device__ __forceinline__ uint32_t Tag(uint32_t epoch, int phase) {
  return epoch * static_cast<uint32_t>(kTagSpan) + static_cast<uint32_t>(phase);
}

// A tagged word stored at device coherence.
__device__ __forceinline__ void TagStore(uint2* p, float v, uint32_t tag) {
  const unsigned long long w = (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(v);
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ Rsrc WordsRsrc(const uint2* base, int64_t words) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(base), 0, static_cast<int>(words * 8), 0x00020000);
}
// Two tagged words (16 bytes at byte offset off) read at device coherence;
// the loads carry no ordering, the tags validate them.
__device__ __forceinline__ U4 Load2(Rsrc r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1);
}
__device__ __forceinline__ U2 Load1(Rsrc r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCpolSc1);
}

// Workgroup barriers that order LDS only. Waves of one workgroup exchange
// nothing through global memory here, and a full barrier's release fence
// would wait for the workgroup's coherent stores to be acknowledged (a
// memory round trip per barrier).
__device__ __forceinline__ void Bar() { LdsBarrier(); }

// AND / OR of a per-thread flag over the workgroup, through LDS.
__device__ __forceinline__ bool BarAnd(bool v) {
  __shared__ int votes[NW];
  const int wave = threadIdx.x >> 6;
  const bool w = __ballot(!v) == 0;
  if ((threadIdx.x & 63) == 0) votes[wave] = w ? 1 : 0;
  Bar();
  int all = 1;
#pragma unroll
  for (int i = 0; i < NW; ++i) all &= votes[i];
  Bar();  // the votes are read before the next vote writes them
  return all != 0;
}
__device__ __forceinline__ bool BarOr(bool v) { return !BarAnd(!v); }

// Repeats probe() -- which issues this thread's loads and returns whether
// every word it read is current -- until the whole workgroup reads current
// words. False (error flag set) after the spin limit.
// Also false, at once, when another workgroup has already given up. Polls
// back off (up to ~0.9 us apart): a workgroup with nothing to do in one phase
// reaches the next early, and its reads must not crowd the weight streams of
// the busy ones.
template <typename Probe>
__device__ __forceinline__ bool WaitCurrent(Probe probe, int32_t* err) {
  for (int spin = 0;; ++spin) {
    if (BarAnd(probe())) return true;
    if (spin >= kSpinLimit) {
      if (threadIdx.x == 0) atomicExch(err, 1);
      return false;
    }
    if ((spin & 63) == 63 &&
        BarOr(__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
      return false;
    if (spin < 4)
      __builtin_amdgcn_s_sleep(2);
    else if (spin < 16)
      __builtin_amdgcn_s_sleep(8);
    else
      __builtin_amdgcn_s_sleep(32);
    asm volatile("" ::: "memory");
  }
}

// ---------------------------------------------------------------- matrix phases

// One matrix phase over one input vector: the scalars every job shares, and
// up to three jobs (tile-major weights of one type each), passed as separate
// values -- an aggregate holding all three would be kept in scratch memory
// once a job is picked from it per wave.
struct MvPhase {
  const uint2* in;  // tagged input [K]
  int32_t K;
  const float* norm_w;
  uint32_t in_tag, out_tag, res_tag;
  int32_t epi;  // kStore / kAdd (x += W . in, reading x tagged res_tag)
  int32_t kwl;
  int32_t n_jobs;
  float* y_plain;  // set: job 0 stores plain floats here instead
};

// One wave's share of one tile: its super-block range [lo, hi), a two-batch
// load ring.
template <uint32_t T>
struct WaveTile {
  static constexpr int BB = MUnit<T>::kBytes;
  MUnit<T> ua[kNB], ub[kNB];
  Rsrc rsrc;
  typename MUnit<T>::Off off;
  int lo, hi;
  __device__ __forceinline__ int Sb(int i) const { return min(lo + i, hi - 1); }
  __device__ __forceinline__ void Load(MUnit<T>* u, int bt) {
#pragma unroll
    for (int b = 0; b < kNB; ++b) u[b].LoadT(rsrc, 16 * BB * Sb(bt * kNB + b), off);
  }
  // the first batch, before the input exists
  __device__ __forceinline__ void Begin(const uint8_t* w, int tile, int n_sb, int part, int kwl, int g, int col) {
    rsrc = TileRsrc(w + static_cast<int64_t>(tile) * n_sb * 16 * BB, n_sb * 16 * BB);
    off = MUnit<T>::MakeOff(g, col);
    lo = (part * n_sb) >> kwl;
    hi = ((part + 1) * n_sb) >> kwl;
    Load(ua, 0);
  }
  __device__ __forceinline__ float Finish(const uint8_t* lds, int abase, int astep, const float2* xg, int g) {
    const int n_part = hi - lo;
    float acc = 0.0f;
    auto comp = [&](const MUnit<T>* u, int bt) {
#pragma unroll
      for (int b = 0; b < kNB; ++b) {
        const int i = bt * kNB + b, sb = Sb(i);
        const float r = UnitDot(u[b], lds + abase + astep * sb, xg + 16 * sb, g);
        acc += i < n_part ? r : 0.0f;
      }
    };
    const int nb = (n_part + kNB - 1) / kNB;
    for (int bt = 0; bt < nb; bt += 2) {
      Load(ub, bt + 1);
      comp(ua, bt);
      if (bt + 1 >= nb) break;
      Load(ua, bt + 2);
      comp(ub, bt + 1);
    }
    return acc;
  }
};

// The workgroup reads its tagged input until current, then stages the digits.
__device__ __forceinline__ bool StageInput(const MvPhase& P, const Hdr& h, uint8_t* lds, double* redd,
                                           int32_t* err) {
  XChunks<NW> xc;
  const int tid = threadIdx.x, K = P.K, n8 = K >> 3;
  const uint32_t in_tag = P.in_tag;
  constexpr int NC = XChunks<NW>::NC, NNC = XChunks<NW>::NNC;
  xc.nc = (n8 + NT - 1) / NT;
  const Rsrc r = WordsRsrc(P.in, K);
  // first a sparse probe, one word per 8 (every producer writes whole
  // groups of 8 or 16 rows at once), then the full read, validated again
  auto sample = [&]() {
    bool ok = true;
    U2 w[(kMaxK / 8 + NT - 1) / NT];
#pragma unroll
    for (int c = 0; c < (kMaxK / 8 + NT - 1) / NT; ++c) {
      const int i = tid + c * NT;
      w[c] = Load1(r, 64 * min(i, n8 - 1));
    }
#pragma unroll
    for (int c = 0; c < (kMaxK / 8 + NT - 1) / NT; ++c)
      ok = ok && (tid + c * NT >= n8 || w[c].y == in_tag);
    return ok;
  };
  auto probe = [&]() {
    U4 w[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c >= xc.nc) break;
      const int ch = min(tid + c * NT, n8 - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) w[c][q] = Load2(r, 64 * ch + 16 * q);
    }
    bool ok = true;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c >= xc.nc) break;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xc.v[c][2 * q] = __uint_as_float(w[c][q].x);
        xc.v[c][2 * q + 1] = __uint_as_float(w[c][q].z);
        ok = ok && w[c][q].y == in_tag && w[c][q].w == in_tag;
      }
    }
    return ok;
  };
  // the RMSNorm gains first: they depend on no producer
  if (P.norm_w != nullptr) {
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(P.norm_w);
#pragma unroll
    for (int c = 0; c < NNC; ++c) {
      if (c >= xc.nc) break;
      const int ch = min(tid + c * NT, n8 - 1);
      const F4 p = GLoad<F4>(wb + 32 * ch), q = GLoad<F4>(wb + 32 * ch + 16);
      xc.wv[c][0] = p.x, xc.wv[c][1] = p.y, xc.wv[c][2] = p.z, xc.wv[c][3] = p.w;
      xc.wv[c][4] = q.x, xc.wv[c][5] = q.y, xc.wv[c][6] = q.z, xc.wv[c][7] = q.w;
    }
  }
  // the full read first (current at once when the producers are done);
  // while stale, the cheap sampled wait, then the full read again
  for (int tries = 0;; ++tries) {
    if (BarAnd(probe())) break;
    if (tries >= kSpinLimit) {
      if (tid == 0) atomicExch(err, 1);
      return false;
    }
    if (!WaitCurrent(sample, err)) return false;
  }
  StageDigits<NW>(h, xc, lds, redd, []() {});
  return true;
}

// One job of a phase.
struct MvJob {
  const uint8_t* w;
  int32_t type, rows, pair;  // pair: a SwiGLU pair, 8 + 8 rows per tile
  uint2* y;                  // tagged output (kAdd: also the residual)
};
__device__ __forceinline__ MvJob Pick(int j, MvJob a, MvJob b, MvJob c) {
  MvJob r;
  r.w = j == 0 ? a.w : j == 1 ? b.w : c.w;
  r.type = j == 0 ? a.type : j == 1 ? b.type : c.type;
  r.rows = j == 0 ? a.rows : j == 1 ? b.rows : c.rows;
  r.pair = j == 0 ? a.pair : j == 1 ? b.pair : c.pair;
  r.y = j == 0 ? a.y : j == 1 ? b.y : c.y;
  return r;
}

// One slot of a matrix phase for one weight type: this wave's (tile, part).
template <uint32_t T>
__device__ __forceinline__ bool RunSlot(const MvPhase& P, const MvJob& J, const Hdr& h, int tile, bool active,
                                        int part, bool stage, uint8_t* lds, double* redd, int32_t* err) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int n_sb = P.K >> 8, kw = 1 << P.kwl;
  WaveTile<T> wt;
  if (active) wt.Begin(J.w, tile, n_sb, part, P.kwl, g, col);
  if (stage && !StageInput(P, h, lds, redd, err)) return false;
  float acc = 0.0f;
  if (active) {
    const int gb = MUnit<T>::GroupBase(g);
    const bool diag = (col >> 2) == g;
    const int abase = diag ? gb * 64 + 16 * (col & 3) : h.zero_off + 64 * g;
    const int astep = diag ? 16 * 64 : 0;
    const float2* xg = reinterpret_cast<const float2*>(lds + h.xg_off) + gb;
    acc = wt.Finish(lds, abase, astep, xg, g);
  }
  acc = AddXor16(acc);
  acc = AddXor32(acc);
  if (kw > 1) {
    float* red = reinterpret_cast<float*>(lds + h.red_off);
    if (lane < 16) red[16 * wave + lane] = acc;
    LdsBarrier();
    if (part == 0) {
      float sum = red[16 * wave + col];
      for (int p = 1; p < kw; ++p) sum += red[16 * (wave + p) + col];
      acc = sum;
    }
  }
  if (!active || part != 0) return true;
  const bool pair = J.pair != 0;
  const int R = pair ? 8 : 16;
  const bool second = pair && col >= 8;
  const int row = tile * R + (second ? col - 8 : col);
  const bool valid = row < J.rows;
  if (pair) {
    const float up = __uint_as_float(Dpp<kRowRor8>(__float_as_uint(acc)));  // lanes 0..7 <- 8..15
    if (lane < 8 && valid) {
      // silu(g) * up with glibc-exact expf (reference src/kernels.h:82-92)
      const float sg = acc / __fadd_rn(1.0f, GlibcExpf(-acc));
      TagStore(J.y + row, __fmul_rn(sg, up), P.out_tag);
    }
  } else if (lane < 16 && valid) {
    if (P.y_plain != nullptr) {
      P.y_plain[row] = acc;
    } else if (P.epi == kAdd) {
      // x += proj: the old x[row] is current since this phase's input was
      // computed from all of it
      const U2 old = Load1(WordsRsrc(J.y, J.rows), 8 * row);
      if (old.y != P.res_tag) atomicExch(err, 2);
      TagStore(J.y + row, __uint_as_float(old.x) + acc, P.out_tag);
    } else {
      TagStore(J.y + row, acc, P.out_tag);
    }
  }
  return true;
}

__device__ __forceinline__ bool MatrixPhase(const MvPhase P, const MvJob J0, const MvJob J1, const MvJob J2,
                                            const Hdr& h, uint8_t* lds, double* redd, int32_t* err) {
  // wave-uniform: tile, part and job live in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = 1 << P.kwl, tps = NW >> P.kwl;
  const int t0 = J0.pair ? (J0.rows + 7) / 8 : (J0.rows + 15) / 16;
  const int t1 = P.n_jobs > 1 ? (J1.rows + 15) / 16 : 0;
  const int t2 = P.n_jobs > 2 ? (J2.rows + 15) / 16 : 0;
  const int n_slots = (t0 + t1 + t2 + tps - 1) / tps;
  bool staged = false;
  for (int slot = blockIdx.x; slot < n_slots; slot += gridDim.x) {
    if (staged) LdsBarrier();  // the previous slot's cross-wave sums are read
    int tile = __builtin_amdgcn_readfirstlane(slot * tps + (wave >> P.kwl));
    const int part = __builtin_amdgcn_readfirstlane(wave & (kw - 1));
    int j = 0, tj = t0;
    if (P.n_jobs > 1 && tile >= t0) {
      tile -= t0;
      j = 1;
      tj = t1;
      if (P.n_jobs > 2 && tile >= t1) {
        tile -= t1;
        j = 2;
        tj = t2;
      }
    }
    j = __builtin_amdgcn_readfirstlane(j);
    tile = __builtin_amdgcn_readfirstlane(tile);
    const bool active = tile < tj;
    const MvJob J = Pick(j, J0, J1, J2);
    const bool ok = J.type == kQ6_K ? RunSlot<kQ6T>(P, J, h, tile, active, part, !staged, lds, redd, err)
                                    : RunSlot<kQ4_K>(P, J, h, tile, active, part, !staged, lds, redd, err);
    if (!ok) return false;
    staged = true;
  }
  return true;
}

// ---------------------------------------------------------------- attention phases

// QK-norm + RoPE of one head vector held as lane pairs (i, i + 64)
// (reference src/qwen3.cc:141-152, src/kernels.h:56-63,108-120).
__device__ __forceinline__ void NormRope(float x0, float x1, float w0, float w1, float c, float sn, float eps,
                                         float* o0, float* o1) {
  double s = static_cast<double>(x0) * x0 + static_cast<double>(x1) * x1;
  s = WaveSumD(s);
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(s / static_cast<double>(kHdS) + static_cast<double>(eps)));
  const float na = __fmul_rn(__fmul_rn(x0, scale), w0);
  const float nb = __fmul_rn(__fmul_rn(x1, scale), w1);
  *o0 = __fsub_rn(__fmul_rn(na, c), __fmul_rn(nb, sn));
  *o1 = __fadd_rn(__fmul_rn(nb, c), __fmul_rn(na, sn));
}

struct AttnLds {
  float ks[kSplitS][kKStrideS];
  float vs[kSplitS][kHdS];
  float qs[NW][kHdS];
};

// Items (KV head, 32-position split) of 0..pos: the G query heads of the KV
// head against the split's cached keys and values; the split holding pos
// normalises, rotates and caches the new key and value. Leaves the
// flash-decoding partial (max, sum of exp, unnormalised output) per query
// head (the arithmetic of decode.hip's split kernel).
__device__ __forceinline__ bool AttnPhase(const StepArgs& a, const float* q_norm, const float* k_norm, float* kcache,
                                          float* vcache, int pos, uint32_t qkv_tag, uint32_t out_tag, int n_splits_all,
                                          uint8_t* lds, int32_t* err) {
  AttnLds& S = *reinterpret_cast<AttnLds*>(lds);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int G = a.n_heads / a.n_kv, n_keys = pos + 1;
  const int ns = (n_keys + kSplitS - 1) / kSplitS;
  const int64_t max_seq = a.max_seq;
  const Rsrc rq = WordsRsrc(a.q, a.qd), rk = WordsRsrc(a.k, a.kvd), rv = WordsRsrc(a.v, a.kvd);
  const float* rope_row = a.rope + static_cast<int64_t>(pos) * kHdS;
  const float rc = rope_row[lane], rs = rope_row[64 + lane];
  bool first = true;
  for (int item = blockIdx.x; item < a.n_kv * ns; item += gridDim.x) {
    if (!first) Bar();  // the previous item's LDS reads are done
    first = false;
    const int kh = item / ns, split = item - kh * ns;
    const int s0 = split * kSplitS;
    const int n = min(kSplitS, n_keys - s0);
    const bool has_new = s0 + n == n_keys;
    // 1. the cached tile (rows clamped into the cache; rows from n on, and
    // row n - 1 of the split holding pos, are replaced below)
    const float* kg = kcache + static_cast<int64_t>(kh) * max_seq * kHdS;
    const float* vg = vcache + static_cast<int64_t>(kh) * max_seq * kHdS;
    constexpr int kPer = kSplitS * (kHdS / 4) / NT;
    F4 kr[kPer], vr[kPer];
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int idx = tid + c * NT;
      const int64_t row = min(static_cast<int64_t>(s0 + (idx >> 5)), max_seq - 1);
      kr[c] = *reinterpret_cast<const F4*>(kg + row * kHdS + 4 * (idx & 31));
      vr[c] = *reinterpret_cast<const F4*>(vg + row * kHdS + 4 * (idx & 31));
    }
    // 2. the raw projections this item needs: wave jb < G query head
    // kh * G + jb, wave G the new key and value (tagged, written by QKV)
    const int jb = wave;
    const bool is_k = jb == G, is_q = jb < G;
    const float* nw = is_k ? k_norm : q_norm;
    const float w0 = nw[lane], w1 = nw[lane + 64];
    float x0 = 0.f, x1 = 0.f, nv0 = 0.f, nv1 = 0.f;
    auto probe = [&]() {
      bool ok = true;
      if (is_q || is_k) {
        const Rsrc r = is_k ? rk : rq;
        const int base = is_k ? kh * kHdS : (kh * G + jb) * kHdS;
        const U2 a0 = Load1(r, 8 * (base + lane)), a1 = Load1(r, 8 * (base + lane + 64));
        x0 = __uint_as_float(a0.x);
        x1 = __uint_as_float(a1.x);
        ok = a0.y == qkv_tag && a1.y == qkv_tag;
        if (is_k) {
          const U2 b0 = Load1(rv, 8 * (kh * kHdS + lane)), b1 = Load1(rv, 8 * (kh * kHdS + lane + 64));
          nv0 = __uint_as_float(b0.x);
          nv1 = __uint_as_float(b1.x);
          ok = ok && b0.y == qkv_tag && b1.y == qkv_tag;
        }
      }
      return ok;
    };
    if (!WaitCurrent(probe, err)) return false;
    // 3. QK-norm + RoPE; the new key and value into the cache and the tile
    if (is_q || is_k) {
      float o0, o1;
      NormRope(x0, x1, w0, w1, rc, rs, a.eps, &o0, &o1);
      if (is_q) {
        S.qs[jb][lane] = o0;
        S.qs[jb][lane + 64] = o1;
      } else if (has_new) {
        float* kd = kcache + (static_cast<int64_t>(kh) * max_seq + pos) * kHdS;
        float* vd = vcache + (static_cast<int64_t>(kh) * max_seq + pos) * kHdS;
        kd[lane] = o0;
        kd[lane + 64] = o1;
        vd[lane] = nv0;
        vd[lane + 64] = nv1;
        S.ks[n - 1][lane] = o0;
        S.ks[n - 1][lane + 64] = o1;
        S.vs[n - 1][lane] = nv0;
        S.vs[n - 1][lane + 64] = nv1;
      }
    }
    // 4. the tile into LDS (rows from n on zero: P.V runs over all 32 rows)
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int idx = tid + c * NT, r = idx >> 5, c4 = idx & 31;
      if (has_new && r == n - 1) continue;
      const F4 z = {0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<F4*>(&S.ks[r][4 * c4]) = r < n ? kr[c] : z;
      *reinterpret_cast<F4*>(&S.vs[r][4 * c4]) = r < n ? vr[c] : z;
    }
    Bar();
    // 5. wave h < G: head kh * G + h -- lane (key j, half) scores 64 dims,
    // softmax over the split, unnormalised P.V
    if (wave < G) {
      const int h = wave;
      const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHdS));
      const int j = lane & 31, half = lane >> 5;
      const F4* q4 = reinterpret_cast<const F4*>(&S.qs[h][64 * half]);
      const F4* k4 = reinterpret_cast<const F4*>(&S.ks[j][64 * half]);
      float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const F4 qq = q4[i], kk = k4[i];
        d0 = __builtin_fmaf(qq.x, kk.x, d0);
        d1 = __builtin_fmaf(qq.y, kk.y, d1);
        d2 = __builtin_fmaf(qq.z, kk.z, d2);
        d3 = __builtin_fmaf(qq.w, kk.w, d3);
      }
      const float sc = lanes::AddXor32((d0 + d1) + (d2 + d3)) * scale;
      const float v = j < n ? sc : -__builtin_inff();
      const float m = WaveMaxF(v);
      const float p = j < n ? ExpSoft(v - m) : 0.0f;
      const float l = WaveSumF(half == 0 ? p : 0.0f);
      float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
      for (int jj = 0; jj < kSplitS; ++jj) {
        const float pj = lanes::ReadLaneF(p, jj);
        const F2v vv = *reinterpret_cast<const F2v*>(&S.vs[jj][2 * lane]);
        acc0 = __builtin_fmaf(pj, vv.x, acc0);
        acc1 = __builtin_fmaf(pj, vv.y, acc1);
      }
      uint2* w = a.part + (static_cast<int64_t>(kh * G + h) * n_splits_all + split) * kPartS;
      if (lane == 0) {
        TagStore(w, m, out_tag);
        TagStore(w + 1, l, out_tag);
      }
      TagStore(w + 2 + 2 * lane, acc0, out_tag);
      TagStore(w + 3 + 2 * lane, acc1, out_tag);
    }
  }
  return true;
}

// Query head h = blockIdx.x (first n_heads workgroups): out[h] = sum_s o_s *
// exp(m_s - M) / sum_s l_s * exp(m_s - M). Wave w takes dimensions
// 16 w .. 16 w + 15, lane (d, g) the splits s = g (mod 4) of dimension d.
__device__ __forceinline__ bool MergePhase(const StepArgs& a, int pos, uint32_t in_tag, uint32_t out_tag, int n_splits_all,
                           uint8_t* lds, int32_t* err) {
  const int h = blockIdx.x;
  if (h >= a.n_heads) return true;
  float* fs = reinterpret_cast<float*>(lds);  // [kMaxSplitsS] split weights
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ns = (pos + 1 + kSplitS - 1) / kSplitS;
  const Rsrc r = WordsRsrc(a.part, static_cast<int64_t>(a.n_heads) * n_splits_all * kPartS);
  const int64_t rec0 = static_cast<int64_t>(h) * n_splits_all * kPartS;
  const int d = 16 * wave + (lane & 15), sg = lane >> 4;
  constexpr int kPerLane = kMaxSplitsS / 4;  // splits per lane at most
  float mv[kMaxSplitsS / NT > 0 ? kMaxSplitsS / NT : 1];
  float lv[kMaxSplitsS / NT > 0 ? kMaxSplitsS / NT : 1];
  (void)kPerLane;
  // (max, sum) of the splits: thread t holds split t (ns <= 256 <= NT)
  auto probe_ml = [&]() {
    if (tid >= ns) return true;
    const U4 w = Load2(r, static_cast<int>(8 * (rec0 + static_cast<int64_t>(tid) * kPartS)));
    mv[0] = __uint_as_float(w.x);
    lv[0] = __uint_as_float(w.z);
    return w.y == in_tag && w.w == in_tag;
  };
  if (!WaitCurrent(probe_ml, err)) return false;
  // M and the weights, by wave 0 through LDS
  float M = tid < ns ? mv[0] : -__builtin_inff();
  M = WaveMaxF(M);
  __shared__ float wmax[NW], wsum[NW];
  if (lane == 0) wmax[wave] = M;
  Bar();
  M = wmax[0];
  for (int w = 1; w < NW; ++w) M = fmaxf(M, wmax[w]);
  float L = 0.0f;
  if (tid < ns) {
    const float f = ExpSoft(mv[0] - M);
    fs[tid] = f;
    L = lv[0] * f;
  }
  // the weighted sum of the l_s in split order (as the per-launch merge:
  // fma in index order within a lane, then the wave sum) -- here thread s
  // holds split s, so the lane sums are single terms
  L = WaveSumF(L);
  if (lane == 0) wsum[wave] = L;
  Bar();
  L = 0.0f;
  for (int w = 0; w < NW; ++w) L += wsum[w];
  // the outputs of dimension d over the splits s = sg, sg + 4, ...
  float o = 0.0f;
  auto probe_o = [&]() {
    bool ok = true;
    float acc = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += 4 * 16) {
      U2 wv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int s = min(s0 + 4 * u + sg, ns - 1);
        wv[u] = Load1(r, static_cast<int>(8 * (rec0 + static_cast<int64_t>(s) * kPartS + 2 + d)));
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int s = s0 + 4 * u + sg;
        if (s < ns) {
          ok = ok && wv[u].y == in_tag;
          acc = __builtin_fmaf(__uint_as_float(wv[u].x), fs[s], acc);
        }
      }
    }
    o = acc;
    return ok;
  };
  if (!WaitCurrent(probe_o, err)) return false;
  o = AddXor16(o);
  o = AddXor32(o);
  if (sg == 0) TagStore(a.attn + static_cast<int64_t>(h) * kHdS + d, o / L, out_tag);
  Bar();  // fs is reused by the next phase's staging
  return true;
}

// ---------------------------------------------------------------- the kernel

__global__ __launch_bounds__(NT) void DecodeStepKernel(StepArgs a) {
  extern __shared__ __align__(256) uint8_t lds[];
  __shared__ double redd[NW];
  // the layer table, read once per launch: the weight streams evict it from
  // the caches between phases, and a descriptor read from memory would cost
  // a round trip per phase
  __shared__ StepLayer layers[kMaxLayers];
  const int tid = threadIdx.x;
  for (int i = tid; i < a.n_layers * static_cast<int>(sizeof(StepLayer) / 4); i += NT)
    reinterpret_cast<uint32_t*>(layers)[i] = reinterpret_cast<const uint32_t*>(a.layers)[i];
  const int pos = lanes::UniformRead(a.pos);
  const uint32_t epoch = static_cast<uint32_t>(lanes::UniformRead(a.pos + 1));
  const int token = lanes::UniformRead(a.token);
  int32_t* err = a.err;
  // an earlier step gave up: its outputs are incomplete, leave at once
  if (lanes::UniformRead(err) != 0) return;
  // phase 0: the token's embedding row, each workgroup its slice of x
  if (blockIdx.x == 0 && tid == 0) {
    const int st = *a.step;
    a.out_ids[st] = token;
  }
  {
    const int tok = token >= 0 && token < a.embd.rows ? token : 0;
    if (tok != token && blockIdx.x == 0 && tid == 0) atomicExch(err, 3);
    const uint8_t* row = a.embd.w + static_cast<int64_t>(tok) * a.embd.row_bytes;
    const int per = (a.H + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    for (int c = blockIdx.x * per + tid; c < min(a.H, (static_cast<int>(blockIdx.x) + 1) * per); c += NT)
      TagStore(a.x + c, dev::DequantExact(a.embd.type, row, c), Tag(epoch, 0));
  }
  Bar();  // the layer table
  const int n_splits_all = static_cast<int>((a.max_seq + kSplitS - 1) / kSplitS);
  const int kmax = max(max(a.H, a.qd), a.F);
  Hdr h;
  h.eps = a.eps;
  h.epi = kStore;
  h.kwl = 0;
  h.zero_off = 4 * kmax;  // digit records: 64 bytes per 16 inputs
  h.xg_off = h.zero_off + kZeroBytes;
  h.red_off = h.xg_off + kmax / 2;
  uint32_t x_tag = Tag(epoch, 0);  // the tag of x's current contents
  // One loop over the phases, each kind of phase inlined once (no calls: a
  // call would spill the live registers to scratch memory).
  const int n_phases = 6 * a.n_layers + 1;
  // Each wave computes the phase's descriptor itself, from the layer's
  // descriptor read by scalar loads: uniform values in scalar registers, no
  // barrier, no LDS round trips. (The next phase's first LDS write follows
  // its input wait, a workgroup barrier that every wave reaches only after
  // finishing this phase.)
  for (int p = 1; p <= n_phases; ++p) {
    const int l = min((p - 1) / 6, a.n_layers - 1), lp = p == n_phases ? 6 : (p - 1) % 6;
    const StepLayer* Ly = layers + l;  // fields read from LDS below
    const int kind = lp == 1 ? 1 : lp == 2 ? 2 : 0;  // 0 matrix, 1 attention split, 2 merge
    MvPhase P{};
    MvJob J0{}, J1{}, J2{};
    P.out_tag = Tag(epoch, p);
    P.n_jobs = 1;
    P.epi = kStore;
    switch (lp) {
      case 0:  // norm + QKV
        P.in = a.x;
        P.K = a.H;
        P.norm_w = LdsField(Ly->attn_norm);
        P.in_tag = x_tag;
        P.kwl = LdsField(Ly->kwl[0]);
        P.n_jobs = 3;
        J0 = MvJob{LdsField(Ly->w[0]), LdsField(Ly->type[0]), a.qd, 0, a.q};
        J1 = MvJob{LdsField(Ly->w[1]), LdsField(Ly->type[1]), a.kvd, 0, a.k};
        J2 = MvJob{LdsField(Ly->w[2]), LdsField(Ly->type[2]), a.kvd, 0, a.v};
        break;
      case 1:
      case 2:
        break;
      case 3:  // O + residual
        P.in = a.attn;
        P.K = a.qd;
        P.in_tag = Tag(epoch, p - 1);
        P.res_tag = x_tag;
        P.epi = kAdd;
        P.kwl = LdsField(Ly->kwl[3]);
        J0 = MvJob{LdsField(Ly->w[3]), LdsField(Ly->type[3]), a.H, 0, a.x};
        break;
      case 4:  // norm + gate/up + SwiGLU
        P.in = a.x;
        P.K = a.H;
        P.norm_w = LdsField(Ly->ffn_norm);
        P.in_tag = x_tag;
        P.kwl = LdsField(Ly->kwl[4]);
        J0 = MvJob{LdsField(Ly->w[4]), LdsField(Ly->type[4]), a.F, 1, a.act};
        break;
      case 5:  // down + residual
        P.in = a.act;
        P.K = a.F;
        P.in_tag = Tag(epoch, p - 1);
        P.res_tag = x_tag;
        P.epi = kAdd;
        P.kwl = LdsField(Ly->kwl[5]);
        J0 = MvJob{LdsField(Ly->w[5]), LdsField(Ly->type[5]), a.H, 0, a.x};
        break;
      default:  // final norm + lm_head
        P.in = a.x;
        P.K = a.H;
        P.norm_w = a.output_norm;
        P.in_tag = x_tag;
        P.kwl = a.lm_kwl;
        P.y_plain = a.logits;
        J0 = MvJob{a.lm_head, a.lm_type, a.V, 0, nullptr};
        break;
    }
    bool ok;
    if (kind == 0) {
      h.K = P.K;
      h.norm_w = P.norm_w;
      ok = MatrixPhase(P, J0, J1, J2, h, lds, redd, err);
      if (P.epi == kAdd) x_tag = P.out_tag;
    } else if (kind == 1) {
      ok = AttnPhase(a, LdsField(Ly->q_norm), LdsField(Ly->k_norm),
                     LdsField(Ly->kcache), LdsField(Ly->vcache), pos, Tag(epoch, p - 1),
                     P.out_tag, n_splits_all, lds, err);
      Bar();  // the merge reuses the LDS
    } else {
      ok = MergePhase(a, pos, Tag(epoch, p - 1), P.out_tag, n_splits_all, lds, err);
    }
    if (!ok) return;
  }
}

}  // namespace

size_t DecodeStepLds(const StepArgs& a) {
  const int kmax = std::max({a.H, a.qd, a.F});
  const size_t stage = static_cast<size_t>(4 * kmax + kZeroBytes + kmax / 2 + NW * 16 * 4);
  const size_t attn = sizeof(AttnLds);
  const size_t merge = sizeof(float) * kMaxSplitsS;
  // at least 96 KiB: one workgroup per compute unit
  return std::max({stage, attn, merge, static_cast<size_t>(96 << 10)});
}

bool DecodeStepSupported(const StepArgs& a, int groups) {
  if (a.n_layers <= 0 || a.n_layers > kMaxLayers || 2 + 6 * a.n_layers > kTagSpan) return false;
  if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0 || a.n_heads / a.n_kv > NW - 1) return false;
  if (a.H % 256 || a.qd % 256 || a.F % 256 || std::max({a.H, a.qd, a.F}) > kMaxK || a.H > kMaxNormK) return false;
  if (a.max_seq > static_cast<int64_t>(kMaxSplitsS) * kSplitS || a.n_heads > groups) return false;
  if (a.lm_type != kQ4_K && a.lm_type != kQ6_K) return false;
  int per_cu = 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(DecodeStepKernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(DecodeStepLds(a))) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, DecodeStepKernel, NT, DecodeStepLds(a)) != hipSuccess ||
      per_cu < 1) {
    (void)hipGetLastError();
    return false;
  }
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return groups <= cus * per_cu;  // every workgroup resident at once
}

void DecodeStep(const StepArgs& a, int groups, hipStream_t s) {
  const size_t lds = DecodeStepLds(a);
  HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(DecodeStepKernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  hipLaunchKernelGGL(DecodeStepKernel, dim3(static_cast<unsigned>(groups)), dim3(NT), lds, s, a);
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
