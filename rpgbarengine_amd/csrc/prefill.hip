// Prefill projections on the gfx950 matrix cores (v_mfma_f32_16x16x32_f16);
// the operand construction that keeps them exact is described in prefill.h.
//
// Kernels: QGemm4Kernel (Q4_K) and QGemm6Kernel (Q6_K), 4 waves over 32
// tokens x 256 weight rows with per-super-block scale tables in LDS, and
// QGemm8Kernel (Q8_0), 2 waves over 64 tokens x 128 rows. In all of them the
// token operands of a 64-input step (both f16 parts) are staged in LDS once
// for the workgroup, every lane assembles its weight operand from the raw
// quant bytes, and the next step's loads are in flight while the current one
// is multiplied.
//
// MFMA operand layout (16x16x32 f16): lane l holds A[i = l % 16][8*(l/16) ..
// +8), B[8*(l/16) .. +8][j = l % 16]; the result C[4*(l/16) + e][l % 16],
// e < 4. In the 16x16x16 form used for the Q4_K min term, 4 k per lane.

#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "common.h"
#include "lanes.h"
#include "expf_glibc.h"
#include "prefill.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

typedef _Float16 H2 __attribute__((ext_vector_type(2)));
typedef _Float16 H4 __attribute__((ext_vector_type(4)));
typedef _Float16 H8 __attribute__((ext_vector_type(8)));
typedef float F4 __attribute__((ext_vector_type(4)));
typedef uint32_t U2 __attribute__((ext_vector_type(2)));
typedef uint32_t U4 __attribute__((ext_vector_type(4)));
// 8 bytes at an address that is only 2-byte aligned (Q6_K and Q8_0 blocks
// are 210 and 34 bytes long): one dwordx2 load, which global memory serves
// at any byte alignment.
typedef U2 U2A2 __attribute__((aligned(2)));

template <typename T>
__device__ __forceinline__ T GLoad(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

__device__ __forceinline__ H2 AsH2(uint32_t v) { return __builtin_bit_cast(H2, v); }
__device__ __forceinline__ uint32_t AsU(H2 v) { return __builtin_bit_cast(uint32_t, v); }

// ---------------------------------------------------------------- SplitRows

constexpr int kSplitThreads = 256;      // rows of up to 10240 inputs
constexpr int kSplitThreadsWide = 1024;  // wider rows, up to 40960 inputs
constexpr int kSplitChunks = 5;          // 8-input chunks per thread at most
constexpr int kSplitPendMax = 4;         // pending split-K partials a row may carry

template <int NW>
__device__ __forceinline__ float BlockMax(float v, float* red) {
  v = lanes::WaveMaxF(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) m = fmaxf(m, red[i]);
  return m;
}
// the waves' partial sums added pairwise: ((r0 + r1) + (r2 + r3)) for four
template <int NW>
__device__ __forceinline__ double PairSum(const double* r) {
  if constexpr (NW == 1)
    return r[0];
  else
    return PairSum<NW / 2>(r) + PairSum<NW / 2>(r + NW / 2);
}

// One workgroup of NT threads per token row; NC 8-input chunks per thread
// (K <= 8 NT NC). kNorm: RMSNorm with gain norm_w; kPend: the pending
// split-K partials are added first. The prologue's loads (inputs, gains,
// partials) carry no branches, so all of them are in flight before the
// first is used.
template <int NT, int NC, bool kNorm, bool kPend>
__global__ __launch_bounds__(NT) void SplitRowsKernel(float* X, int64_t ldx, int K, const float* __restrict__ norm_w,
                                                      float eps, SplitX o, SplitPending pend) {
  constexpr int NW = NT / 64;
  const int t = blockIdx.x, tid = threadIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(X + t * ldx);
  const int n8 = K >> 3;
  __shared__ double redd[NW];
  __shared__ float redf[NW];
  float v[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = min(tid + c * NT, n8 - 1);
    const float4 a = x4[2 * ch], b = x4[2 * ch + 1];
    v[c][0] = a.x, v[c][1] = a.y, v[c][2] = a.z, v[c][3] = a.w;
    v[c][4] = b.x, v[c][5] = b.y, v[c][6] = b.z, v[c][7] = b.w;
  }
  // the RMSNorm gain chunks load with the inputs (used after the sum of
  // squares)
  float wv[NC][8];
  if constexpr (kNorm) {
    const float4* w4 = reinterpret_cast<const float4*>(norm_w);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = min(tid + c * NT, n8 - 1);
      const float4 a = w4[2 * ch], b = w4[2 * ch + 1];
      wv[c][0] = a.x, wv[c][1] = a.y, wv[c][2] = a.z, wv[c][3] = a.w;
      wv[c][4] = b.x, wv[c][5] = b.y, wv[c][6] = b.z, wv[c][7] = b.w;
    }
  }
  if constexpr (kPend) {
    // x += the sum of the split partials in split order (SplitKReduceKernel's
    // arithmetic), written back as the residual. Every partial of a chunk
    // (of every chunk, up to two per thread) is requested before any is
    // added: one round trip, not one per split. Split z >= ksplit reloads the
    // last one (an address in bounds) and is not added.
    constexpr int kGroup = NC <= 2 ? NC : 1;  // chunks whose partials are in flight together
    const int nz = pend.ksplit;
#pragma unroll
    for (int c0 = 0; c0 < NC; c0 += kGroup) {
      float4 pp[kGroup][kSplitPendMax][2];
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        const int ch = min(tid + (c0 + g) * NT, n8 - 1);
#pragma unroll
        for (int z = 0; z < kSplitPendMax; ++z) {
          const int zz = min(z, nz - 1);
          const float4* p4 = reinterpret_cast<const float4*>(
              pend.part + (static_cast<int64_t>(zz) * pend.M + t) * pend.part_ld + pend.pcol + 8 * ch);
          pp[g][z][0] = p4[0];
          pp[g][z][1] = p4[1];
        }
      }
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        const int c = c0 + g, ch = tid + c * NT;
        float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int z = 0; z < kSplitPendMax; ++z) {
          if (z == 0 || z < nz) {  // nz >= 1
            const float4 a = pp[g][z][0], b = pp[g][z][1];
            sum[0] += a.x, sum[1] += a.y, sum[2] += a.z, sum[3] += a.w;
            sum[4] += b.x, sum[5] += b.y, sum[6] += b.z, sum[7] += b.w;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] + sum[i];
        if (ch < n8) {
          float4* xo = reinterpret_cast<float4*>(X + t * ldx) + 2 * ch;
          xo[0] = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
          xo[1] = make_float4(v[c][4], v[c][5], v[c][6], v[c][7]);
        }
      }
    }
  }
  if constexpr (kNorm) {
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (tid + c * NT < n8)
#pragma unroll
        for (int i = 0; i < 8; ++i) s += static_cast<double>(v[c][i]) * v[c][i];
    s = lanes::WaveSumD(s);
    if ((tid & 63) == 0) redd[tid >> 6] = s;
    __syncthreads();
    const double total = PairSum<NW>(redd);
    const float scale =
        static_cast<float>(1.0 / __builtin_sqrt(total / static_cast<double>(K) + static_cast<double>(eps)));
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = __fmul_rn(__fmul_rn(v[c][i], scale), wv[c][i]);
  }
  float mx = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (tid + c * NT < n8)
#pragma unroll
      for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[c][i]));
  mx = BlockMax<NW>(mx, redf);
  // s = 2^(15 - E) for max = f * 2^E, f in [0.5, 1): max * s in [2^14, 2^15)
  int e = 0;
  (void)frexpf(mx, &e);
  const int se = mx > 0.0f ? min(max(15 - e, -100), 100) : 0;
  const float s = ldexpf(1.0f, se), s32 = ldexpf(1.0f, se - 5);
  if (tid == 0) o.inv_s[t] = ldexpf(1.0f, -se);
  _Float16* hi = static_cast<_Float16*>(o.hi) + static_cast<int64_t>(t) * K;
  _Float16* lo = static_cast<_Float16*>(o.lo) + static_cast<int64_t>(t) * K;
  _Float16* shi = static_cast<_Float16*>(o.sum_hi) + static_cast<int64_t>(t) * (K >> 5);
  _Float16* slo = static_cast<_Float16*>(o.sum_lo) + static_cast<int64_t>(t) * (K >> 5);
  constexpr int kPerm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = tid + c * NT;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) sum += v[c][i];
    // sum of the 32 inputs of this chunk's sub-block: chunks 4j..4j+3 sit
    // on 4 consecutive lanes
    sum += lanes::DppF<lanes::kQuadXor1>(sum);
    sum += lanes::DppF<lanes::kQuadXor2>(sum);
    if (ch < n8) {
      H8 h, l;
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const float xs = v[c][kPerm[p]] * s;
        const _Float16 xh = static_cast<_Float16>(xs);
        h[p] = xh;
        l[p] = static_cast<_Float16>(xs - static_cast<float>(xh));
      }
      *reinterpret_cast<H8*>(hi + 8 * ch) = h;
      *reinterpret_cast<H8*>(lo + 8 * ch) = l;
      if ((ch & 3) == 0) {
        const float ss = sum * s32;
        const _Float16 sh = static_cast<_Float16>(ss);
        shi[ch >> 2] = sh;
        slo[ch >> 2] = static_cast<_Float16>(ss - static_cast<float>(sh));
      }
    }
  }
}

// ---------------------------------------------------------------- QGemm

constexpr int kGT = 128;             // threads per workgroup (2 waves)
constexpr int kTM = 64;              // tokens per workgroup
constexpr int kWN = 64;              // weight rows per wave
constexpr int kTN = 2 * kWN;         // weight rows per workgroup
constexpr int kStep = 64;            // inputs per pipeline step
constexpr int kARow = kStep + 8;     // LDS row of one token's step (f16, padded)

constexpr int kGemmSplitMax = 4;     // K splits of one product (partials summed in order)
static_assert(kGemmSplitMax <= kSplitPendMax, "SplitRows holds every pending partial of a chunk in flight");

struct GemmArgs {
  SplitX x;
  GemmJob job[3];
  int32_t tiles[3];  // N tiles per job
  int32_t n_jobs;
  int32_t ksplit;    // blockIdx.z takes super-blocks [z * n / ksplit, (z + 1) * n / ksplit)
  int64_t part_ld;   // partials: x.part[(z * M + token) * part_ld + pcol[job] + row]
  int32_t pcol[3];
};

// The SplitX of the super-blocks [o0, ...): the same rows, pointers moved.
__device__ __forceinline__ SplitX ShiftSplit(const SplitX& x, int k0) {
  SplitX r = x;
  r.hi = static_cast<_Float16*>(x.hi) + k0;
  r.lo = static_cast<_Float16*>(x.lo) + k0;
  r.sum_hi = static_cast<_Float16*>(x.sum_hi) + (k0 >> 5);
  r.sum_lo = static_cast<_Float16*>(x.sum_lo) + (k0 >> 5);
  return r;
}

// Result of one output element: to y (with the job's epilogue), or to the
// split-K partials.
__device__ __forceinline__ void PutOut(const GemmJob& J, const SplitX& x, float* part, int64_t part_ld, int pcol,
                                       int ksplit, int z, int tok, int row, float v) {
  if (ksplit > 1) {
    part[(static_cast<int64_t>(z) * x.M + tok) * part_ld + pcol + row] = v;
  } else {
    float* y = J.y + static_cast<int64_t>(tok) * J.ldy + row;
    *y = J.epi == kAdd ? *y + v : v;
  }
}

// Staged token operands of one step: [part][token][2 segments of 32 inputs]
// f16, 16-byte chunks: 2 parts x 64 tokens x 8 chunks = 1024 chunks, 8 per
// thread. Segment s starts at input k[s] (the two 32-input K-steps of a step
// need not be adjacent).
struct AStage {
  U4 c[8];
};

__device__ __forceinline__ void LoadA(AStage& st, const SplitX& x, int m0, int k0, int k1) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * kGT;              // 0..1023
    const int part = idx >> 9, r = (idx >> 3) & 63, ch = idx & 7;
    const int tok = min(m0 + r, x.M - 1);
    const _Float16* src = static_cast<const _Float16*>(part ? x.lo : x.hi) + static_cast<int64_t>(tok) * x.K +
                          (ch < 4 ? k0 : k1);
    st.c[i] = GLoad<U4>(src + 8 * (ch & 3));
  }
}

__device__ __forceinline__ void StoreA(const AStage& st, _Float16 (*As)[kTM][kARow], int m0, int M) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * kGT;
    const int part = idx >> 9, r = (idx >> 3) & 63, ch = idx & 7;
    const U4 v = m0 + r < M ? st.c[i] : U4{0u, 0u, 0u, 0u};
    *reinterpret_cast<U4*>(&As[part][r][8 * ch]) = v;
  }
}

// Byte-wise values v (0..255) of a dword as the f16 pairs (1024 + v0, 1024 +
// v2) and (1024 + v1, 1024 + v3), in the operand order of 4 inputs.
__device__ __forceinline__ void BytePairs(uint32_t v, H2* p02, H2* p13) {
  *p02 = AsH2((v & 0x00FF00FFu) | 0x64006400u);
  *p13 = AsH2(((v >> 8) & 0x00FF00FFu) | 0x64006400u);
}

__device__ __forceinline__ H8 Pack(H2 a, H2 b, H2 c, H2 d) {
  return __builtin_bit_cast(H8, U4{AsU(a), AsU(b), AsU(c), AsU(d)});
}

// Q8_0 weight operand of 8 int8 quants: (1024 + (q ^ 0x80)) - 1152 = q.
__device__ __forceinline__ H8 Q8Operand(U2 q) {
  const H2 off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
  H2 p[4];
  BytePairs(q.x ^ 0x80808080u, &p[0], &p[1]);
  BytePairs(q.y ^ 0x80808080u, &p[2], &p[3]);
  return Pack(p[0] + off, p[1] + off, p[2] + off, p[3] + off);
}

__device__ __forceinline__ F4 Mfma32(H8 a, H8 b, F4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
// A fresh (zero-C) product: the empty asm keeps both sources live until the
// result exists, so the result is never allocated over a source -- an MFMA
// whose destination aliases its A or B registers returned wrong sums on
// gfx950 (measured), and the compiler allows it when a source dies there.
__device__ __forceinline__ F4 Mfma16Fresh(H4 a, H4 b) {
  const F4 r = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, F4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(r));
  return r;
}
// The same for a product accumulated onto c (c kept live too, so the result
// cannot partly overlap it either).
__device__ __forceinline__ F4 Mfma16Keep(H4 a, H4 b, F4 c) {
  const F4 r = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(c), "v"(r));
  return r;
}

// Q8_0 projections: a workgroup of 2 waves owns 64 tokens x 128 rows, each
// wave 64 x 64 = 4 x 4 MFMA tiles; a step covers one pair of 32-input blocks
// (K-step h = block h of the pair, scaled by its d once per K-step). The
// token operands of a step are staged in LDS for both waves; every lane
// assembles its weight operand from the raw quants; the next step's loads are
// in flight while the current one is multiplied.
__global__ __launch_bounds__(kGT) void QGemm8Kernel(GemmArgs a) {
  int nt = blockIdx.x, j = 0;
  while (j + 1 < a.n_jobs && nt >= a.tiles[j]) {
    nt -= a.tiles[j];
    ++j;
  }
  const GemmJob& J = a.job[j];
  // this split's block pairs [o0, o1)
  const int z = blockIdx.z, nall = a.x.K / 64;
  const int o0 = z * nall / a.ksplit, o1 = (z + 1) * nall / a.ksplit;
  const SplitX x = ShiftSplit(a.x, o0 * 64);
  const int m0 = blockIdx.y * kTM;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int jr = lane & 15, kq = lane >> 4;
  const int n0 = nt * kTN + wave * kWN;
  const int rows = J.w.rows;
  __shared__ __align__(16) _Float16 As[2][kTM][kARow];
  const uint8_t* wr[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    wr[t] = J.w.w + static_cast<int64_t>(min(n0 + 16 * t + jr, rows - 1)) * J.w.row_bytes +
            static_cast<int64_t>(o0) * 68;
  struct Raw {
    U2 q0, q1;
    uint32_t d;
  };
  auto load_raw = [&](Raw& r, const uint8_t* pair) {
    r.q0 = GLoad<U2A2>(pair + 2 + 8 * kq);
    r.q1 = GLoad<U2A2>(pair + 36 + 8 * kq);
    r.d = static_cast<uint32_t>(GLoad<uint16_t>(pair)) | (static_cast<uint32_t>(GLoad<uint16_t>(pair + 34)) << 16);
  };
  const int nout = o1 - o0;
  F4 T[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int t = 0; t < 4; ++t) T[mt][t] = F4{0.f, 0.f, 0.f, 0.f};
  AStage st;
  LoadA(st, x, m0, 0, 32);
  Raw raw[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) load_raw(raw[t], wr[t]);
  for (int o = 0; o < nout; ++o) {
    __syncthreads();
    StoreA(st, As, m0, x.M);
    __syncthreads();
    // the next pair's operands in flight during this one's products
    const int on = o + 1 < nout ? o + 1 : o;
    LoadA(st, x, m0, 64 * on, 64 * on + 32);
    Raw rn[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) load_raw(rn[t], wr[t] + 68 * on);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      H8 ah[4], al[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        ah[mt] = *reinterpret_cast<const H8*>(&As[0][16 * mt + jr][32 * h + 8 * kq]);
        al[mt] = *reinterpret_cast<const H8*>(&As[1][16 * mt + jr][32 * h + 8 * kq]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const H8 bf = Q8Operand(h ? raw[t].q1 : raw[t].q0);
        const float d = dev::HalfToFloatFast(h ? raw[t].d >> 16 : raw[t].d & 0xFFFFu);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const F4 c = Mfma32(al[mt], bf, Mfma32(ah[mt], bf, F4{0.f, 0.f, 0.f, 0.f}));
#pragma unroll
          for (int e = 0; e < 4; ++e) T[mt][t][e] = __builtin_fmaf(d, c[e], T[mt][t][e]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) raw[t] = rn[t];
  }
  // epilogue: C[4*kq + e][jr] of each tile
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tok = m0 + 16 * mt + 4 * kq + e;
      if (tok >= x.M) continue;
      const float is = x.inv_s[tok];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = n0 + 16 * t + jr;
        if (row >= rows) continue;
        PutOut(J, x, x.part, a.part_ld, a.pcol[j], a.ksplit, z, tok, row, T[mt][t][e] * is);
      }
    }
  }
}

// ---------------------------------------------------------------- QGemm, Q4_K pipeline
//
// Q4_K projections: a workgroup owns 16 MTW WM tokens x 256 weight rows; its
// waves form a WM x 4 grid, each wave 16 MTW tokens x 64 rows (MTW x 4 MFMA
// tiles). The token operands of a step are staged in LDS once for all waves;
// the loads of a step are issued RD steps ahead into a register ring; the
// scale table and the min-term sums of the next super-block are staged in LDS
// once per block.
// One barrier per step. Workgroup i takes token tile i % tiles_m, so the
// workgroups of one XCD (i % 8) share their token operands in its L2. With
// MTW = 2 a wave needs half the accumulators and two waves share a SIMD, so
// one wave's operand assembly overlaps the other's products.

constexpr int kG4Rows = 4 * kWN;  // weight rows per workgroup
constexpr int kG4Mtw = 2;         // 16-token MFMA tiles per wave
constexpr int kG4Wm = 1;          // waves along the tokens
constexpr int kG6Tokens = 32;     // tokens per Q6_K workgroup
constexpr int kG4Rd = 2;          // steps in flight

struct G4Args {
  SplitX x;
  GemmJob job[3];
  int32_t tiles[3];  // 256-row tiles per job
  int32_t n_jobs;
  int32_t tiles_m;   // token tiles
  int32_t ksplit;    // blockIdx.y takes super-blocks [y * n / ksplit, (y + 1) * n / ksplit)
  int64_t part_ld;   // partials as in GemmArgs
  int32_t pcol[3];
  // SwiGLU pair (Q4_K kernel, no K split): job 0 is gate (y = the product
  // silu(gate.x) * (up.x)), job 1 up; a 256-row tile holds rows
  // [128 tile, +128) of both, each wave 32 of gate (its 16-row subtiles 0,
  // 1) and the same 32 of up (subtiles 2, 3)
  int32_t pair;
};

// Workgroup shape: WM x 4 waves, each 16 * MTW tokens x 64 rows.
template <int MTW, int WM>
struct G4Shape {
  static constexpr int kThreads = 256 * WM;
  static constexpr int kTokens = 16 * MTW * WM;
};

// Per super-block scale table of the workgroup's weight rows, unpacked once
// from the raw headers and read by every wave.
struct G4Table {
  U4 sc[4][kG4Rows];   // [s][row]: f16 pairs {sc, sc}, {-1024 sc, ..} of sub-block 2s, {sc/16, ..}, {-64 sc, ..} of 2s + 1
  U4 mn[kG4Rows][2];   // f16 mins of sub-blocks 0..7, then 8 zeros
  float2 dd[kG4Rows];  // d, -32 dmin
};

__device__ __forceinline__ uint32_t HalfPair(float v) {
  const _Float16 h = static_cast<_Float16>(v);
  return AsU(H2{h, h});
}

// Entries of `row` for sub-blocks 4 * hf .. 4 * hf + 3 from its raw Q4_K
// header h (d, dmin | 12 scale bytes); hf 0 also writes d and -32 dmin, hf 1
// the mins. Every entry is exact in f16 (sc, m <= 63).
__device__ __forceinline__ void FillG4Table(G4Table& tb, int row, int hf, U4 h) {
  uint32_t sc[4], mn[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) dev::ScaleMinK4(4 * hf + e, h.y, h.z, h.w, &sc[e], &mn[e]);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float f0 = static_cast<float>(sc[2 * p]), f1 = static_cast<float>(sc[2 * p + 1]);
    tb.sc[2 * hf + p][row] = U4{HalfPair(f0), HalfPair(-1024.0f * f0), HalfPair(0.0625f * f1), HalfPair(-64.0f * f1)};
  }
  if (hf == 0) {
    tb.dd[row] = float2{dev::HalfToFloatFast(h.x & 0xFFFFu), -32.0f * dev::HalfToFloatFast(h.x >> 16)};
  } else {
    uint32_t unused;
#pragma unroll
    for (int e = 0; e < 4; ++e) dev::ScaleMinK4(e, h.y, h.z, h.w, &unused, &mn[4 + e]);
    // mn[0..3] are the mins of sub-blocks 4..7, mn[4..7] those of 0..3
    U4 v;
    v.x = AsU(H2{static_cast<_Float16>(static_cast<float>(mn[4])), static_cast<_Float16>(static_cast<float>(mn[5]))});
    v.y = AsU(H2{static_cast<_Float16>(static_cast<float>(mn[6])), static_cast<_Float16>(static_cast<float>(mn[7]))});
    v.z = AsU(H2{static_cast<_Float16>(static_cast<float>(mn[0])), static_cast<_Float16>(static_cast<float>(mn[1]))});
    v.w = AsU(H2{static_cast<_Float16>(static_cast<float>(mn[2])), static_cast<_Float16>(static_cast<float>(mn[3]))});
    tb.mn[row][0] = v;
    tb.mn[row][1] = U4{0u, 0u, 0u, 0u};
  }
}

// Q4_K weight operand of one sub-block from the lane's 8 raw bytes w (w8 =
// w >> 8 per dword): the nibbles selected by `mask` (0x000F000F: low
// nibbles, read as the f16 1024 + q; 0x00F000F0: high nibbles, 1024 + 16 q)
// OR-ed into the f16 pair magic, then one fused f16 FMA per pair with the
// table pair (scv, neg): (1024 + q) sc - 1024 sc = (1024 + 16 q) sc/16 - 64 sc
// = q sc, exact (the product never rounds: q sc <= 945). `magic` lives in a
// VGPR and `mask` in an SGPR so that each nibble pair costs one v_and_or_b32
// (VOP3 takes no literal on gfx9).
__device__ __forceinline__ H8 Q4OperandT(U2 w, U2 w8, uint32_t mask, uint32_t magic, uint32_t scv, uint32_t neg) {
  const H2 s = AsH2(scv), n = AsH2(neg);
  const H2 r0 = __builtin_elementwise_fma(AsH2((w.x & mask) | magic), s, n);   // inputs 0, 2
  const H2 r1 = __builtin_elementwise_fma(AsH2((w8.x & mask) | magic), s, n);  // inputs 1, 3
  const H2 r2 = __builtin_elementwise_fma(AsH2((w.y & mask) | magic), s, n);   // inputs 4, 6
  const H2 r3 = __builtin_elementwise_fma(AsH2((w8.y & mask) | magic), s, n);  // inputs 5, 7
  return __builtin_bit_cast(H8, U4{AsU(r0), AsU(r1), AsU(r2), AsU(r3)});
}

// RD: steps in flight in the register ring (2 or 4); the loads of step g are
// issued at step g - RD and its token chunks are stored into LDS at the end
// of step g - 1.
template <int RD, int MTW, int WM>
__global__ __launch_bounds__((G4Shape<MTW, WM>::kThreads)) void QGemm4Kernel(G4Args a) {
  constexpr int NT = G4Shape<MTW, WM>::kThreads;
  constexpr int TM = G4Shape<MTW, WM>::kTokens;
  constexpr int NA = 16 * TM / NT;  // token chunks of a step per thread
  const int tm = static_cast<int>(blockIdx.x) % a.tiles_m;
  int nt = static_cast<int>(blockIdx.x) / a.tiles_m, j = 0;
  while (j + 1 < a.n_jobs && nt >= a.tiles[j]) {
    nt -= a.tiles[j];
    ++j;
  }
  const GemmJob& J = a.job[j];
  // this split's super-blocks [o0, o1)
  const int z = blockIdx.y, nall = a.x.K / 256;
  const int o0 = z * nall / a.ksplit, o1 = (z + 1) * nall / a.ksplit;
  const SplitX x = ShiftSplit(a.x, 256 * o0);
  const int m0 = tm * TM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 3, wm = wave >> 2;  // row quarter, token block
  const int jr = lane & 15, kq = lane >> 4;
  const int nb = nt * kG4Rows;  // first row of the workgroup
  const int n0 = nb + wn * kWN;  // first row of the wave
  const int mb = 16 * MTW * wm;  // first token (within the tile) of the wave
  const int rows = J.w.rows;
  const int64_t rb = J.w.row_bytes;
  __shared__ __align__(16) _Float16 As[2][2][TM][kARow];
  __shared__ __align__(16) _Float16 Xs[2][2][TM][8];
  __shared__ __align__(16) G4Table Tb[2];
  // row r = 64 w + 16 t + j of the workgroup (0..255): row nb + r of the
  // job, or for a SwiGLU pair row 128 nt + 32 w + 16 (t % 2) + j of gate
  // (t < 2) or up (t >= 2)
  const bool pair = a.pair != 0;
  const int pb = nt * (kG4Rows / 2);
  auto row_ptr = [&](int r) {
    if (pair) {
      const int t = (r >> 4) & 3;
      const uint8_t* m = t < 2 ? J.w.w : a.job[1].w.w;
      return m + static_cast<int64_t>(min(pb + 32 * (r >> 6) + 16 * (t & 1) + (r & 15), rows - 1)) * rb;
    }
    return J.w.w + static_cast<int64_t>(min(nb + r, rows - 1)) * rb;
  };
  const uint8_t* wr[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) wr[t] = row_ptr(wn * kWN + 16 * t + jr) + static_cast<int64_t>(144) * o0;
  // header row of threads 0..255
  const uint8_t* hrow = row_ptr(tid & 255) + static_cast<int64_t>(144) * o0;
  const int nout = o1 - o0;
  // token chunks of a step: 2 parts x TM tokens x 8 chunks of 16 bytes
  auto issue_a = [&](U4* ra, int o, int s) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = tid + i * NT;
      const int part = idx / (8 * TM), r = (idx >> 3) % TM, ch = idx & 7;
      const int tok = min(m0 + r, x.M - 1);
      const _Float16* src =
          static_cast<const _Float16*>(part ? x.lo : x.hi) + static_cast<int64_t>(tok) * x.K + 256 * o + 64 * s;
      ra[i] = GLoad<U4>(src + 8 * ch);
    }
  };
  auto store_a = [&](const U4* ra, int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = tid + i * NT;
      const int part = idx / (8 * TM), r = (idx >> 3) % TM, ch = idx & 7;
      *reinterpret_cast<U4*>(&As[buf][part][r][8 * ch]) = m0 + r < x.M ? ra[i] : U4{0u, 0u, 0u, 0u};
    }
  };
  auto issue_raw = [&](U2* rw, int o, int s) {
#pragma unroll
    for (int t = 0; t < 4; ++t) rw[t] = GLoad<U2>(wr[t] + 144 * o + 16 + 32 * s + 8 * kq);
  };
  // per super-block: headers (threads 0..255, one row each) and the
  // sub-block sums of the token rows (threads 0..2 TM - 1: part x token)
  const int xs_part = (tid / TM) & 1, xs_r = tid % TM;
  const int xs_tok = min(m0 + xs_r, x.M - 1);
  const _Float16* xs_src =
      static_cast<const _Float16*>(xs_part ? x.sum_lo : x.sum_hi) + static_cast<int64_t>(xs_tok) * (x.K >> 5);
  U4 hreg, xreg;
  auto issue_block = [&](int o) {
    hreg = GLoad<U4>(hrow + 144 * o);
    xreg = GLoad<U4>(xs_src + 8 * o);
  };
  auto store_block = [&](int buf) {
    for (int hf = tid >> 8; hf < 2; hf += NT / 256) FillG4Table(Tb[buf], tid & 255, hf, hreg);
    if (tid < 2 * TM) *reinterpret_cast<U4*>(&Xs[buf][xs_part][xs_r][0]) = m0 + xs_r < x.M ? xreg : U4{0u, 0u, 0u, 0u};
  };
  // nibble masks and the f16 pair magic as opaque registers (see Q4OperandT)
  uint32_t mask_lo, mask_hi, magic;
  asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(mask_lo));
  asm volatile("s_mov_b32 %0, 0xf000f0" : "=s"(mask_hi));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));

  F4 C1[MTW][4], T[MTW][4];
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int t = 0; t < 4; ++t) C1[mt][t] = T[mt][t] = F4{0.f, 0.f, 0.f, 0.f};
  U4 ra[RD][NA];
  U2 rw[RD][4];
  // step g = 4 * o + s lives in ring slot g % RD (s % RD: 4 is a multiple of RD)
  auto clamp_o = [&](int o) { return o < nout ? o : nout - 1; };
#pragma unroll
  for (int g = 0; g < RD; ++g) {
    issue_a(ra[g], clamp_o(g / 4), g % 4);
    issue_raw(rw[g], clamp_o(g / 4), g % 4);
  }
  issue_block(0);
  store_a(ra[0], 0);
  store_block(0);
  __syncthreads();

  for (int o = 0; o < nout; ++o) {
    const int ob = o & 1, on = o + 1 < nout ? o + 1 : o;
    const G4Table& tb = Tb[ob];
    const int wrow = wn * kWN + jr;  // the lane's row within the workgroup (+ 16 t)
    issue_block(on);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int buf = s & 1;
      U4 sct[4];
      U2 w8[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sct[t] = tb.sc[s][wrow + 16 * t];
        const U2 r = rw[s % RD][t];
        w8[t] = U2{r.x >> 8, r.y >> 8};
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        H8 ah[MTW], al[MTW];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
          ah[mt] = *reinterpret_cast<const H8*>(&As[buf][0][mb + 16 * mt + jr][32 * h + 8 * kq]);
          al[mt] = *reinterpret_cast<const H8*>(&As[buf][1][mb + 16 * mt + jr][32 * h + 8 * kq]);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // sub-block 2s + h
          const H8 bf = h ? Q4OperandT(rw[s % RD][t], w8[t], mask_hi, magic, sct[t].z, sct[t].w)
                          : Q4OperandT(rw[s % RD][t], w8[t], mask_lo, magic, sct[t].x, sct[t].y);
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt) {
            const F4 c0 = (s == 0 && h == 0) ? F4{0.f, 0.f, 0.f, 0.f} : C1[mt][t];
            C1[mt][t] = Mfma32(al[mt], bf, Mfma32(ah[mt], bf, c0));
          }
        }
      }
      if (s == 3) {
        // block end: T += d * C1 - 32 * dmin * sum_sb m_sb * sums_sb; the
        // 16x16x16 operand's k = 4 * kq + e is sub-block k (k < 8), zero
        // beyond (the table's zero padding)
        const int kqc = kq & 1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const H4 bm = *reinterpret_cast<const H4*>(reinterpret_cast<const char*>(&tb.mn[wrow + 16 * t][0]) + 8 * kq);
          const float2 dd = tb.dd[wrow + 16 * t];
          const float d = dd.x, dmin32 = dd.y;
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt) {
            const H4 xh = *reinterpret_cast<const H4*>(&Xs[ob][0][mb + 16 * mt + jr][4 * kqc]);
            const H4 xl = *reinterpret_cast<const H4*>(&Xs[ob][1][mb + 16 * mt + jr][4 * kqc]);
            const F4 c2 = Mfma16Keep(xl, bm, Mfma16Fresh(xh, bm));
#pragma unroll
            for (int e = 0; e < 4; ++e)
              T[mt][t][e] = __builtin_fmaf(dmin32, c2[e], __builtin_fmaf(d, C1[mt][t][e], T[mt][t][e]));
          }
        }
      }
      // stage the next step's token chunks; refill this step's ring slot
      // with step 4 * o + s + RD
      store_a(ra[(s + 1) % RD], buf ^ 1);
      if (s == 3) store_block(ob ^ 1);
      issue_a(ra[s % RD], clamp_o(o + (s + RD) / 4), (s + RD) % 4);
      issue_raw(rw[s % RD], clamp_o(o + (s + RD) / 4), (s + RD) % 4);
      __syncthreads();
    }
  }
  // epilogue: C[4*kq + e][jr] of each tile
  if (pair) {
    // each lane holds gate (subtiles 0, 1) and up (2, 3) of the same rows:
    // silu(g) * u (reference src/kernels.h:82-92), the bits of the unfused
    // stores followed by SwiGLURows
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = m0 + mb + 16 * mt + 4 * kq + e;
        if (tok >= x.M) continue;
        const float is = x.inv_s[tok];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int row = pb + 32 * wn + 16 * t + jr;
          if (row >= rows) continue;
          const float g = T[mt][t][e] * is, u = T[mt][t + 2][e] * is;
          const float sg = g / __fadd_rn(1.0f, GlibcExpf(-g));
          J.y[static_cast<int64_t>(tok) * J.ldy + row] = __fmul_rn(sg, u);
        }
      }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tok = m0 + mb + 16 * mt + 4 * kq + e;
      if (tok >= x.M) continue;
      const float is = x.inv_s[tok];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = n0 + 16 * t + jr;
        if (row >= rows) continue;
        PutOut(J, x, x.part, a.part_ld, a.pcol[j], a.ksplit, z, tok, row, T[mt][t][e] * is);
      }
    }
  }
}

// ---------------------------------------------------------------- QGemm, Q6_K pipeline
//
// Q6_K projections on the Q4_K pipeline's shape: 4 waves own 32 tokens x 256
// rows (each wave 32 x 64), two workgroups per CU, loads two steps ahead, one
// barrier per step. Step s covers groups m = s % 2 and m + 2 of half s / 2 of
// a super-block -- inputs 128 (s / 2) + 32 m + [0, 32) (K-step 0, low
// nibbles) and + 64 (K-step 1, high nibbles) of the same ql bytes. A weight
// is held as the f16 1 + q/64 (q in mantissa bits 4..9, put together from
// its ql nibble and qh bits with two v_and_or per pair); one packed FMA per
// operand then gives, exactly, for sc = 16 sh + sl,
//   hi = 16 sh (q - 32) = (1 + q/64) 1024 sh - 1536 sh   (|hi| <= 4096, a multiple of 16)
//   lo =    sl (q - 32) = (1 + q/64)   64 sl -   96 sl   (|lo| <= 480),
// and both meet both token parts (4 products per K-step). The table holds
// per super-block and row the 16 pairs {1024 sh, 64 sl} and d.

struct G6Table {
  uint32_t sc[16][kG4Rows];  // [sub-block][row]: f16 pair {1024 sh, 64 sl}
  float d[kG4Rows];
};

// f16 pairs (1 + q/64) of inputs (0, 2) and (1, 3) of a ql dword (nibbles
// selected and placed at bits 4..7 by the caller) and its qh dword (the two
// bits placed at 8..9 by the caller).
__device__ __forceinline__ uint32_t AndOr(uint32_t a, uint32_t mask, uint32_t c) {  // (a & mask) | c
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t Q6Pair(uint32_t nib, uint32_t qh, uint32_t one) {
  return AndOr(nib, 0x00F000F0u, AndOr(qh, 0x03000300u, one));
}

__global__ __launch_bounds__(256) void QGemm6Kernel(G4Args a) {
  constexpr int NT = 256, TM = kG6Tokens, NA = 16 * TM / NT, MTW = TM / 16;
  const int tm = static_cast<int>(blockIdx.x) % a.tiles_m;
  int nt = static_cast<int>(blockIdx.x) / a.tiles_m, j = 0;
  while (j + 1 < a.n_jobs && nt >= a.tiles[j]) {
    nt -= a.tiles[j];
    ++j;
  }
  const GemmJob& J = a.job[j];
  const int z = blockIdx.y, nall = a.x.K / 256;
  const int o0 = z * nall / a.ksplit, o1 = (z + 1) * nall / a.ksplit;
  const SplitX x = ShiftSplit(a.x, 256 * o0);
  const int m0 = tm * TM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);  // row quarter
  const int jr = lane & 15, kq = lane >> 4;
  const int nb = nt * kG4Rows;
  const int n0 = nb + wn * kWN;
  const int rows = J.w.rows;
  const int64_t rb = J.w.row_bytes;
  __shared__ __align__(16) _Float16 As[2][2][TM][kARow];
  __shared__ __align__(16) G6Table Tb[2];
  const uint8_t* wr[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    wr[t] = J.w.w + static_cast<int64_t>(min(n0 + 16 * t + jr, rows - 1)) * rb + static_cast<int64_t>(210) * o0;
  const uint8_t* hrow = J.w.w + static_cast<int64_t>(min(nb + tid, rows - 1)) * rb + static_cast<int64_t>(210) * o0;
  const int nout = o1 - o0;
  // token chunks of step s: chunk ch < 4 from K-step 0, ch >= 4 from K-step 1
  auto seg = [](int s, int h) { return 128 * (s >> 1) + 32 * ((s & 1) + 2 * h); };
  auto issue_a = [&](U4* ra, int o, int s) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = tid + i * NT;
      const int part = idx / (8 * TM), r = (idx >> 3) % TM, ch = idx & 7;
      const int tok = min(m0 + r, x.M - 1);
      const _Float16* src = static_cast<const _Float16*>(part ? x.lo : x.hi) + static_cast<int64_t>(tok) * x.K +
                            256 * o + seg(s, ch >> 2) + 8 * (ch & 3);
      ra[i] = GLoad<U4>(src);
    }
  };
  auto store_a = [&](const U4* ra, int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = tid + i * NT;
      const int part = idx / (8 * TM), r = (idx >> 3) % TM, ch = idx & 7;
      *reinterpret_cast<U4*>(&As[buf][part][r][8 * ch]) = m0 + r < x.M ? ra[i] : U4{0u, 0u, 0u, 0u};
    }
  };
  // the lane's ql and qh words of step s: 8 bytes each
  auto issue_raw = [&](U2* rl, U2* rh, int o, int s) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint8_t* blk = wr[t] + 210 * o;
      rl[t] = GLoad<U2A2>(blk + 64 * (s >> 1) + 32 * (s & 1) + 8 * kq);
      rh[t] = GLoad<U2A2>(blk + 128 + 32 * (s >> 1) + 8 * kq);
    }
  };
  // per super-block: scales and d of row tid
  U2 hs0, hs1;
  uint32_t hd;
  auto issue_block = [&](int o) {
    const uint8_t* blk = hrow + 210 * o;
    hs0 = GLoad<U2A2>(blk + 192);
    hs1 = GLoad<U2A2>(blk + 200);
    hd = GLoad<uint16_t>(blk + 208);
  };
  auto store_block = [&](int buf) {
    const uint32_t w[4] = {hs0.x, hs0.y, hs1.x, hs1.y};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int sc = __builtin_amdgcn_sbfe(w[i >> 2], 8 * (i & 3), 8);
      const _Float16 hi = static_cast<_Float16>(static_cast<float>(1024 * (sc >> 4)));
      const _Float16 lo = static_cast<_Float16>(static_cast<float>(64 * (sc & 15)));
      Tb[buf].sc[i][tid] = AsU(H2{hi, lo});
    }
    Tb[buf].d[tid] = dev::HalfToFloatFast(hd & 0xFFFFu);
  };
  uint32_t one;  // the f16 pair (1.0, 1.0) in a VGPR (v_and_or takes no literal pair)
  asm volatile("v_mov_b32 %0, 0x3c003c00" : "=v"(one));
  const H2 m15 = {static_cast<_Float16>(-1.5f), static_cast<_Float16>(-1.5f)};

  F4 C1[MTW][4], T[MTW][4];
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int t = 0; t < 4; ++t) C1[mt][t] = T[mt][t] = F4{0.f, 0.f, 0.f, 0.f};
  constexpr int RD = 2;
  U4 ra[RD][NA];
  U2 rl[RD][4], rh[RD][4];
  auto clamp_o = [&](int o) { return o < nout ? o : nout - 1; };
#pragma unroll
  for (int g = 0; g < RD; ++g) {
    issue_a(ra[g], clamp_o(g / 4), g % 4);
    issue_raw(rl[g], rh[g], clamp_o(g / 4), g % 4);
  }
  issue_block(0);
  store_a(ra[0], 0);
  store_block(0);
  __syncthreads();

  for (int o = 0; o < nout; ++o) {
    const int ob = o & 1, on = o + 1 < nout ? o + 1 : o;
    const G6Table& tb = Tb[ob];
    const int wrow = wn * kWN + jr;
    issue_block(on);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int buf = s & 1, m = s & 1, hh = s >> 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int grp = m + 2 * h;  // group within the half: qh bits 2 grp
        H8 ah[MTW], al[MTW];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
          ah[mt] = *reinterpret_cast<const H8*>(&As[buf][0][16 * mt + jr][32 * h + 8 * kq]);
          al[mt] = *reinterpret_cast<const H8*>(&As[buf][1][16 * mt + jr][32 * h + 8 * kq]);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const U2 l = rl[s % RD][t], q = rh[s % RD][t];
          // nibbles to bits 4..7 (low: << 4 / >> 4; high: in place / >> 8),
          // qh bits 2 grp to bits 8..9
          const uint32_t n02x = h ? l.x : l.x << 4, n13x = h ? l.x >> 8 : l.x >> 4;
          const uint32_t n02y = h ? l.y : l.y << 4, n13y = h ? l.y >> 8 : l.y >> 4;
          const uint32_t q02x = q.x << (8 - 2 * grp), q13x = q.x >> (2 * grp);
          const uint32_t q02y = q.y << (8 - 2 * grp), q13y = q.y >> (2 * grp);
          const H2 v0 = AsH2(Q6Pair(n02x, q02x, one)), v1 = AsH2(Q6Pair(n13x, q13x, one));
          const H2 v2 = AsH2(Q6Pair(n02y, q02y, one)), v3 = AsH2(Q6Pair(n13y, q13y, one));
          const H2 sc = AsH2(tb.sc[8 * hh + 2 * grp + (kq >> 1)][wrow + 16 * t]);
          const H2 nc = sc * m15;  // {-1536 sh, -96 sl}
          const H2 sh2 = {sc.x, sc.x}, nh2 = {nc.x, nc.x}, sl2 = {sc.y, sc.y}, nl2 = {nc.y, nc.y};
          const H8 bh = __builtin_bit_cast(
              H8, U4{AsU(__builtin_elementwise_fma(v0, sh2, nh2)), AsU(__builtin_elementwise_fma(v1, sh2, nh2)),
                     AsU(__builtin_elementwise_fma(v2, sh2, nh2)), AsU(__builtin_elementwise_fma(v3, sh2, nh2))});
          const H8 bl = __builtin_bit_cast(
              H8, U4{AsU(__builtin_elementwise_fma(v0, sl2, nl2)), AsU(__builtin_elementwise_fma(v1, sl2, nl2)),
                     AsU(__builtin_elementwise_fma(v2, sl2, nl2)), AsU(__builtin_elementwise_fma(v3, sl2, nl2))});
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt) {
            const F4 c0 = (s == 0 && h == 0) ? F4{0.f, 0.f, 0.f, 0.f} : C1[mt][t];
            C1[mt][t] = Mfma32(al[mt], bl, Mfma32(al[mt], bh, Mfma32(ah[mt], bl, Mfma32(ah[mt], bh, c0))));
          }
        }
      }
      if (s == 3) {  // block end: T += d * C1
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float d = tb.d[wrow + 16 * t];
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) T[mt][t][e] = __builtin_fmaf(d, C1[mt][t][e], T[mt][t][e]);
        }
      }
      store_a(ra[(s + 1) % RD], buf ^ 1);
      if (s == 3) store_block(ob ^ 1);
      issue_a(ra[s % RD], clamp_o(o + (s + RD) / 4), (s + RD) % 4);
      issue_raw(rl[s % RD], rh[s % RD], clamp_o(o + (s + RD) / 4), (s + RD) % 4);
      __syncthreads();
    }
  }
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tok = m0 + 16 * mt + 4 * kq + e;
      if (tok >= x.M) continue;
      const float is = x.inv_s[tok];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = n0 + 16 * t + jr;
        if (row >= rows) continue;
        PutOut(J, x, x.part, a.part_ld, a.pcol[j], a.ksplit, z, tok, row, T[mt][t][e] * is);
      }
    }
  }
}

// y = silu(g) * u elementwise, glibc-exact expf (reference src/kernels.h:82-92)
__global__ __launch_bounds__(256) void SwiGLUKernel(const float* __restrict__ g, const float* __restrict__ u,
                                                    float* __restrict__ y, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = g[i];
  const float sg = v / __fadd_rn(1.0f, GlibcExpf(-v));
  y[i] = __fmul_rn(sg, u[i]);
}

}  // namespace

void SwiGLURows(const float* g, const float* u, float* y, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(SwiGLUKernel, dim3(static_cast<unsigned>(CeilDiv(n, 256))), dim3(256), 0, s, g, u, y, n);
  HIP_CHECK(hipGetLastError());
}

size_t SplitXBytes(int M, int K, int n_max) {
  const size_t big = static_cast<size_t>(M) * K * 2, small = static_cast<size_t>(M) * (K / 32) * 2;
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  return 2 * up(big) + 2 * up(small) + up(static_cast<size_t>(M) * 4) +
         up(static_cast<size_t>(kGemmSplitMax) * M * n_max * 4);
}

SplitX SplitXView(void* base, int M, int K, int n_max) {
  const size_t big = static_cast<size_t>(M) * K * 2, small = static_cast<size_t>(M) * (K / 32) * 2;
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  uint8_t* p = static_cast<uint8_t*>(base);
  SplitX s;
  s.hi = p;
  s.lo = p + up(big);
  s.sum_hi = p + 2 * up(big);
  s.sum_lo = p + 2 * up(big) + up(small);
  s.inv_s = reinterpret_cast<float*>(p + 2 * up(big) + 2 * up(small));
  s.part = reinterpret_cast<float*>(p + 2 * up(big) + 2 * up(small) + up(static_cast<size_t>(M) * 4));
  s.part_floats = static_cast<int64_t>(kGemmSplitMax) * M * n_max;
  s.M = M;
  s.K = K;
  return s;
}

void SplitRowsAdd(float* X, int64_t ldx, int M, int K, const float* norm_w, float eps, const SplitX& out,
                  const SplitPending& pend, hipStream_t s) {
  RPG_CHECK(M > 0 && M <= out.M && K == out.K, "split rows: %d x %d does not fit the buffer", M, K);
  RPG_CHECK(K % 32 == 0 && K <= 8 * kSplitChunks * kSplitThreadsWide, "split rows: K = %d unsupported", K);
  RPG_CHECK(ldx % 4 == 0, "split rows: row stride must be a multiple of 4");
  RPG_CHECK(pend.part == nullptr || (pend.M == M && (pend.part_ld + pend.pcol) % 4 == 0 && pend.pcol % 4 == 0 &&
                                      pend.ksplit >= 1 && pend.ksplit <= kSplitPendMax),
            "split rows: pending sums do not match the rows");
  SplitX o = out;
  o.M = M;
  const dim3 grid(static_cast<unsigned>(M));
  const bool wide = K > 8 * kSplitChunks * kSplitThreads;
  const int nt = wide ? kSplitThreadsWide : kSplitThreads;
  const int nc = static_cast<int>(CeilDiv(K / 8, nt));
  const int variant = (norm_w != nullptr ? 1 : 0) | (pend.part != nullptr ? 2 : 0);
  auto launch = [&](auto nt_c, auto nc_c) {
    constexpr int NT = decltype(nt_c)::value, NC = decltype(nc_c)::value;
    const dim3 block(NT);
    switch (variant) {
      case 0: hipLaunchKernelGGL((SplitRowsKernel<NT, NC, false, false>), grid, block, 0, s, X, ldx, K, norm_w, eps, o, pend); break;
      case 1: hipLaunchKernelGGL((SplitRowsKernel<NT, NC, true, false>), grid, block, 0, s, X, ldx, K, norm_w, eps, o, pend); break;
      case 2: hipLaunchKernelGGL((SplitRowsKernel<NT, NC, false, true>), grid, block, 0, s, X, ldx, K, norm_w, eps, o, pend); break;
      default: hipLaunchKernelGGL((SplitRowsKernel<NT, NC, true, true>), grid, block, 0, s, X, ldx, K, norm_w, eps, o, pend);
    }
  };
  using N256 = std::integral_constant<int, kSplitThreads>;
  using N1024 = std::integral_constant<int, kSplitThreadsWide>;
  if (wide) {
    // 10240 < K <= 40960: two to five chunks per thread
    switch (nc) {
      case 2: launch(N1024{}, std::integral_constant<int, 2>{}); break;
      case 3: launch(N1024{}, std::integral_constant<int, 3>{}); break;
      case 4: launch(N1024{}, std::integral_constant<int, 4>{}); break;
      default: launch(N1024{}, std::integral_constant<int, kSplitChunks>{});
    }
  } else {
    switch (nc) {
      case 1: launch(N256{}, std::integral_constant<int, 1>{}); break;
      case 2: launch(N256{}, std::integral_constant<int, 2>{}); break;
      case 3: launch(N256{}, std::integral_constant<int, 3>{}); break;
      case 4: launch(N256{}, std::integral_constant<int, 4>{}); break;
      default: launch(N256{}, std::integral_constant<int, kSplitChunks>{});
    }
  }
  HIP_CHECK(hipGetLastError());
}

void SplitRows(const float* X, int64_t ldx, int M, int K, const float* norm_w, float eps, const SplitX& out,
               hipStream_t s) {
  // (no pending sums: the kernel does not write X)
  SplitRowsAdd(const_cast<float*>(X), ldx, M, K, norm_w, eps, out, SplitPending{}, s);
}

bool QGemmSupports(const MatRef& w) {
  return ((w.type == kQ4_K || w.type == kQ6_K) && w.cols % 256 == 0) || (w.type == kQ8_0 && w.cols % 64 == 0);
}

namespace {

// y = (y +) the sum of the split-K partials of one job, in split order.
__global__ __launch_bounds__(256) void SplitKReduceKernel(const float* __restrict__ part, int64_t part_ld, int pcol,
                                                          int ksplit, int M, int N, float* y, int64_t ldy, int epi) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(M) * N) return;
  const int tok = static_cast<int>(i / N), row = static_cast<int>(i % N);
  // every partial (and y) requested before the first is added: one round trip
  float* yp = y + static_cast<int64_t>(tok) * ldy + row;
  const float y0 = epi == kAdd ? *yp : 0.0f;
  float p[kGemmSplitMax];
#pragma unroll
  for (int z = 0; z < kGemmSplitMax; ++z)
    if (z < ksplit) p[z] = part[(static_cast<int64_t>(z) * M + tok) * part_ld + pcol + row];
  float v = 0.0f;
#pragma unroll
  for (int z = 0; z < kGemmSplitMax; ++z)
    if (z < ksplit) v += p[z];
  *yp = epi == kAdd ? y0 + v : v;
}

// K splits of a launch of `wgs` workgroups over `nblk` scale blocks: doubled
// while the launch has fewer than `target` workgroups, every split keeps at
// least `min_blk` blocks and the partials fit (thresholds measured on the
// Qwen3-4B projections at 512 tokens).
int ChooseSplit(int64_t wgs, int nblk, int64_t cols, const SplitX& x, int64_t target, int min_blk) {
  int S = 1;
  while (S < kGemmSplitMax && wgs * S < target && 2 * S * min_blk <= nblk &&
         static_cast<int64_t>(2 * S) * x.M * cols <= x.part_floats)
    S *= 2;
  return S;
}

// Compute units of the current device (queried once per device).
int ComputeUnits() {
  static int cached[64] = {};
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  RPG_CHECK(dev >= 0 && dev < 64, "device %d", dev);
  if (cached[dev] == 0) {
    int n = 0;
    HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    cached[dev] = n > 0 ? n : 1;
  }
  return cached[dev];
}

// K splits of a tiled launch of `wgs` workgroups over `nblk` super-blocks:
// the largest S <= kGemmSplitMax whose S * wgs workgroups fit in one round
// of the compute units (one tiled workgroup per unit), with at least 4
// super-blocks per split and room for the partials. A launch of 80 tiles on
// 256 units takes S = 3 (240 workgroups in one round) rather than 4 (320,
// a second round of 64).
int TiledSplit(int64_t wgs, int nblk, int64_t cols, const SplitX& x) {
  const int64_t cus = ComputeUnits();
  int S = 1;
  for (int c = 2; c <= kGemmSplitMax; ++c)
    if (c * wgs <= cus && 4 * c <= nblk && static_cast<int64_t>(c) * x.M * cols <= x.part_floats) S = c;
  return S;
}

}  // namespace

void QGemm(const SplitX& x, const GemmJob* jobs, int n_jobs, hipStream_t s, SplitPending* defer) {
  if (defer != nullptr) *defer = SplitPending{};
  RPG_CHECK(n_jobs >= 1 && n_jobs <= 3, "qgemm: 1..3 jobs");
  int32_t pcol[3] = {0, 0, 0};
  int64_t cols = 0;
  for (int j = 0; j < n_jobs; ++j) {
    RPG_CHECK(QGemmSupports(jobs[j].w) && jobs[j].w.cols == x.K, "qgemm: unsupported matrix");
    RPG_CHECK(jobs[j].w.type == jobs[0].w.type, "qgemm: one weight type per launch");
    pcol[j] = static_cast<int32_t>(cols);
    cols += jobs[j].w.rows;
  }
  int S = 1;
  const bool q6 = jobs[0].w.type == kQ6_K;
  // Q4_K / Q6_K launches of long segments take the tiled kernel. (Its K
  // split fills at most one round of compute units, so the q,k launch -- 160
  // workgroups at 512 tokens -- leaves room for the v launch beside it on
  // the side stream.)
  if ((jobs[0].w.type == kQ4_K || q6) && x.M >= kTiledMinTokens) {
    TiledArgs t;
    t.x = x;
    t.pair = 0;
    t.n_jobs = n_jobs;
    t.tiles_m = static_cast<int32_t>(CeilDiv(x.M, kTiledTokens));
    int tiles = 0;
    for (int j = 0; j < n_jobs; ++j) {
      t.job[j] = jobs[j];
      t.tiles[j] = static_cast<int32_t>(CeilDiv(jobs[j].w.rows, kTiledRows));
      t.pcol[j] = pcol[j];
      tiles += t.tiles[j];
    }
    S = TiledSplit(static_cast<int64_t>(tiles) * t.tiles_m, x.K / 256, cols, x);
    t.ksplit = S;
    t.part_ld = cols;
    LaunchTiled(t, s);
  } else if (jobs[0].w.type == kQ4_K || q6) {
    using Shape = G4Shape<kG4Mtw, kG4Wm>;
    const int64_t mtiles = CeilDiv(x.M, q6 ? kG6Tokens : Shape::kTokens);
    G4Args g;
    g.x = x;
    g.pair = 0;
    g.n_jobs = n_jobs;
    g.tiles_m = static_cast<int32_t>(mtiles);
    int tiles = 0;
    for (int j = 0; j < n_jobs; ++j) {
      g.job[j] = jobs[j];
      g.tiles[j] = static_cast<int32_t>(CeilDiv(jobs[j].w.rows, kG4Rows));
      g.pcol[j] = pcol[j];
      tiles += g.tiles[j];
    }
    S = ChooseSplit(tiles * mtiles, x.K / 256, cols, x, 640, q6 ? 4 : 8);
    g.ksplit = S;
    g.part_ld = cols;
    const dim3 grid(static_cast<unsigned>(tiles * mtiles), static_cast<unsigned>(S));
    if (q6)
      hipLaunchKernelGGL(QGemm6Kernel, grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((QGemm4Kernel<kG4Rd, kG4Mtw, kG4Wm>), grid, dim3(Shape::kThreads), 0, s, g);
  } else {
    const int64_t mtiles = CeilDiv(x.M, kTM);
    GemmArgs a;
    a.x = x;
    a.n_jobs = n_jobs;
    int tiles = 0;
    for (int j = 0; j < n_jobs; ++j) {
      a.job[j] = jobs[j];
      a.tiles[j] = static_cast<int32_t>(CeilDiv(jobs[j].w.rows, kTN));
      a.pcol[j] = pcol[j];
      tiles += a.tiles[j];
    }
    const int nblk = x.K / 64;
    S = ChooseSplit(tiles * mtiles, nblk, cols, x, 320, 1);
    a.ksplit = S;
    a.part_ld = cols;
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(mtiles), static_cast<unsigned>(S));
    hipLaunchKernelGGL(QGemm8Kernel, grid, dim3(kGT), 0, s, a);
  }
  HIP_CHECK(hipGetLastError());
  if (S > 1 && defer != nullptr && n_jobs == 1 && jobs[0].epi == kAdd) {
    defer->part = x.part;
    defer->part_ld = cols;
    defer->pcol = 0;
    defer->ksplit = S;
    defer->M = x.M;
    return;
  }
  if (S > 1) {
    for (int j = 0; j < n_jobs; ++j) {
      const int64_t n = static_cast<int64_t>(x.M) * jobs[j].w.rows;
      hipLaunchKernelGGL(SplitKReduceKernel, dim3(static_cast<unsigned>(CeilDiv(n, 256))), dim3(256), 0, s, x.part,
                         cols, pcol[j], S, x.M, static_cast<int>(jobs[j].w.rows), jobs[j].y, jobs[j].ldy,
                         static_cast<int>(jobs[j].epi));
    }
    HIP_CHECK(hipGetLastError());
  }
}

void ApplyPending(const SplitPending& pend, float* y, int64_t ldy, int N, hipStream_t s) {
  if (pend.part == nullptr) return;
  RPG_CHECK(pend.ksplit >= 1 && pend.ksplit <= kGemmSplitMax, "pending sums: %d splits", pend.ksplit);
  const int64_t n = static_cast<int64_t>(pend.M) * N;
  hipLaunchKernelGGL(SplitKReduceKernel, dim3(static_cast<unsigned>(CeilDiv(n, 256))), dim3(256), 0, s, pend.part,
                     pend.part_ld, pend.pcol, pend.ksplit, pend.M, N, y, ldy, static_cast<int>(kAdd));
  HIP_CHECK(hipGetLastError());
}

bool QGemmSwiGLU(const SplitX& x, const GemmJob& gate, const GemmJob& up, hipStream_t s) {
  if (gate.w.type != kQ4_K || up.w.type != kQ4_K || gate.w.rows != up.w.rows || gate.w.cols != x.K ||
      up.w.cols != x.K || gate.w.row_bytes != up.w.row_bytes || x.K % 256 != 0)
    return false;
  if (x.M >= kTiledMinTokens) {
    // the tiled launch; fused only where the unfused one would not split
    const int64_t mt = CeilDiv(x.M, kTiledTokens);
    if (TiledSplit(2 * CeilDiv(gate.w.rows, kTiledRows) * mt, x.K / 256, 2 * static_cast<int64_t>(gate.w.rows), x) >
        1)
      return false;
    TiledArgs t;
    t.x = x;
    t.pair = 1;
    t.n_jobs = 1;
    t.tiles_m = static_cast<int32_t>(mt);
    t.job[0] = gate;
    t.job[1] = up;
    t.tiles[0] = static_cast<int32_t>(CeilDiv(gate.w.rows, kTiledRows / 2));
    t.tiles[1] = t.tiles[2] = 0;
    t.pcol[0] = t.pcol[1] = t.pcol[2] = 0;
    t.ksplit = 1;
    t.part_ld = 0;
    // More tiles than compute units, with a last round at most half full:
    // that round's tiles run as two halves each (twice the workgroups at
    // half the length), their sums added by a second launch.
    const int64_t total = t.tiles[0] * mt, cus = ComputeUnits(), tail = total % cus;
    if (total > cus && tail > 0 && 2 * tail <= cus && x.K >= 512 &&
        tail * 2 * kTiledTailFloats <= x.part_floats)
      t.tail_wg = static_cast<int32_t>(total - tail);
    LaunchTiled(t, s);
    return true;
  }
  using Shape = G4Shape<kG4Mtw, kG4Wm>;
  const int64_t mtiles = CeilDiv(x.M, Shape::kTokens);
  const int tiles = static_cast<int>(CeilDiv(gate.w.rows, kG4Rows / 2));
  // the unfused launch's split choice: fuse only where it would not split
  if (ChooseSplit(2 * CeilDiv(gate.w.rows, kG4Rows) * mtiles, x.K / 256, 2 * static_cast<int64_t>(gate.w.rows), x, 640,
                  8) > 1)
    return false;
  G4Args g;
  g.x = x;
  g.pair = 1;
  g.n_jobs = 1;
  g.tiles_m = static_cast<int32_t>(mtiles);
  g.job[0] = gate;
  g.job[1] = up;
  g.tiles[0] = tiles;
  g.tiles[1] = g.tiles[2] = 0;
  g.pcol[0] = g.pcol[1] = g.pcol[2] = 0;
  g.ksplit = 1;
  g.part_ld = 0;
  hipLaunchKernelGGL((QGemm4Kernel<kG4Rd, kG4Mtw, kG4Wm>), dim3(static_cast<unsigned>(tiles * mtiles), 1u),
                     dim3(Shape::kThreads), 0, s, g);
  HIP_CHECK(hipGetLastError());
  return true;
}

}  // namespace k
}  // namespace rpg
