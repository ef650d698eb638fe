// Decode matvec of a few tokens at once -- the decode step of a batch of
// sessions, prefill segments of a few tokens -- on the int8 matrix cores, for
// Q4_K, Q6_K and Q8_0 weights in their tile-major decode copies (decode.h).
//
// v_mfma_i32_16x16x32_i8 computes C[i][j] += sum_k A[i][k] * B[k][j] in exact
// int32; lane L = j + 16g supplies 8 bytes of B column j and 8 bytes of A row
// L % 16 for the same 8 k (k-group g), and holds C[4g..4g+4)[j] afterwards.
// B column j is one output row of a 16-row tile (or 8 rows of each matrix of
// a SwiGLU pair): lane (j, g) feeds 8 unsigned 4- or 6-bit quants of one
// 32-weight group of its row, weights 8g..8g+7 of the group. A holds the
// inputs as exact integers: each aligned 32-element group of a token's input
// is scaled by its own power of two s into |x * s| < 2^22 and rounded,
// x_fix = d0 + 2^8 d1 + 2^16 d2 with signed-byte digits.
// Row 4t + d of A holds digit d of token t of a quad over the 32-group (row
// 4t + 3 repeats digit 2; its sums land in a result nobody reads), so lane
// (j, g) receives token g's three digit sums for row j.
//   Q4_K (32-weight sub-blocks): one MFMA covers one sub-block for 4 tokens.
//   Q6_K (16-weight sub-blocks): a 32-group holds two sub-blocks; one MFMA
//     per half, with the B lanes of the other half zero (k-groups 0, 1 are
//     half 0, k-groups 2, 3 half 1).
// sum(q * x_fix) = C0 + 2^8 C1 + 2^16 C2, and the lane applies its row's
// scales once per MFMA:
//   Q4_K  (d*sc) * sum(q*x) - (dmin*m) * sum(x)   (reference src/quant.cc:159-198)
//   Q6_K  (d*sc) * sum(q*x) - (32*d*sc) * sum(x)  (src/quant.cc:200-237)
//   Q8_0  d * sum(q*x)                            (src/quant.cc:132-142)
// Q8_0 launches (every job Q8_0) stage four digits per input instead, |x *
// s| < 2^30 (rows 4t + d, d = 0..3, all read), the signed quants feed the
// MFMA raw, one 32-weight block per MFMA, and sum(q * x_fix) = C0 + 2^8 C1 +
// 2^16 C2 + 2^24 C3 is formed exactly in double: a block has no min term,
// so nothing cancels the rounding of the inputs and they keep 30 bits.
// with sum(x) = sum(x_fix) / s staged per half group: the reference dot
// (src/matmul.cc:73-102, src/matmul_avx2.cc:95-289) of the inputs rounded to
// 22 bits below their group's maximum, up to the float rounding of the
// scaled terms. Dots are judged by max|d| / sum|a*w| <= 1e-6.
//
// Work: a workgroup of NW waves takes NW / kw tiles and one group of tokens;
// the kw waves of a tile split its super-blocks into contiguous ranges and
// add their sums in LDS in a fixed order. The workgroup stages its tokens'
// inputs in LDS -- RMSNorm per token when the projection consumes one
// (reference src/qwen3.cc:131-134,191-194,284-287) -- as digit rows (3 x 32
// bytes per token and group) and per group (1/s, sums of x_fix / s). When
// all tokens do not fit in LDS (long K),
// they are split into groups taken by separate workgroups; the workgroups of
// one tile are dispatched 8 apart, so they run on the same XCD at about the
// same time and the later ones find the tile's weights in that XCD's L2.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "decode.h"
#include "lanes.h"
#include "mfma_dot.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

using lanes::Dpp;
using lanes::kQuadXor1;
using lanes::kQuadXor2;
using lanes::kRowRor8;
using lanes::Uniform;
using lanes::WaveSumD;
using mfma::LdsBarrier;
using mfma::Rsrc;
using mfma::TileRsrc;

typedef uint32_t U4 __attribute__((ext_vector_type(4)));
typedef uint32_t U2 __attribute__((ext_vector_type(2)));
typedef int I4 __attribute__((ext_vector_type(4)));
typedef float F4 __attribute__((ext_vector_type(4)));
typedef float F2 __attribute__((ext_vector_type(2)));

constexpr int kLdsBudget = 150 * 1024;  // staged tokens + per-group sums of one workgroup
constexpr int kFewTokensDefault = 64;  // measured: the few-token launches beat the GEMMs on every 1.7B / 4B shape up to 64 tokens
constexpr int kRecBytes = 96;       // digit rows of one token and group (three digits)
constexpr int kRecBytes4 = 128;     // the same with four digits (Q8_0 launches)
constexpr int kXgBytes = 16;        // (1/s, sum x, sum x of half 0, of half 1)

struct BatchArgs {
  const float* x;       // [T][ldx]
  const float* norm_w;  // RMSNorm gain, or null
  int64_t ldx;
  int32_t K;
  float eps;
  int32_t T, tpg, n_tg;  // tokens, tokens per group, token groups
  int32_t epi;
  int32_t kw_log2;
  int32_t xg_off, red_off;  // LDS: digit rows at 0, then the group sums, then the cross-wave sums
  int32_t units;            // tile sets (workgroups per token group)
  int32_t n_jobs, tiles0, tiles1;
  DecodeJob job[3];
  int64_t ldy[3];
};

template <typename T>
__device__ __forceinline__ T GLoad(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

// Every lane must call it (quad permutes): lanes 4m..4m+3 hold the four
// 8-element chunks of one 32-element group of one token. LDS: group G's
// records and sums hold the TPG token slots side by side (the tokens a
// matrix-core operand reads together then fall in different banks).
template <bool kFour>
__device__ __forceinline__ void StageChunk(const float (&v)[8], int t, int TPG, int ch, uint8_t* lds, int xg_off) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
  m = fmaxf(m, __uint_as_float(Dpp<kQuadXor1>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(Dpp<kQuadXor2>(__float_as_uint(m))));
  if constexpr (kFour) {
    // s = 2^(30 - E): |x * s| < 2^30, x_fix = rint(x * s) as an integer; u =
    // x_fix + 0x80808080 holds the four signed-byte digits, each offset by
    // 128, as its bytes (no wrap for |x_fix| < 2^30)
    const int eb = static_cast<int>(__float_as_uint(m) >> 23);
    const int se = m > 0.0f ? min(max(156 - eb, -100), 126) : 0;
    const float s = __uint_as_float(static_cast<uint32_t>(se + 127) << 23);
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = static_cast<uint32_t>(__float2int_rn(v[i] * s)) + 0x80808080u;
    uint32_t row[4][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t a1 = __builtin_amdgcn_perm(u[4 * h + 1], u[4 * h], 0x05010400u);  // v0.b0 v1.b0 v0.b1 v1.b1
      const uint32_t a2 = __builtin_amdgcn_perm(u[4 * h + 1], u[4 * h], 0x07030602u);  // v0.b2 v1.b2 v0.b3 v1.b3
      const uint32_t b1 = __builtin_amdgcn_perm(u[4 * h + 3], u[4 * h + 2], 0x05010400u);
      const uint32_t b2 = __builtin_amdgcn_perm(u[4 * h + 3], u[4 * h + 2], 0x07030602u);
      row[0][h] = __builtin_amdgcn_perm(b1, a1, 0x05040100u) ^ 0x80808080u;
      row[1][h] = __builtin_amdgcn_perm(b1, a1, 0x07060302u) ^ 0x80808080u;
      row[2][h] = __builtin_amdgcn_perm(b2, a2, 0x05040100u) ^ 0x80808080u;
      row[3][h] = __builtin_amdgcn_perm(b2, a2, 0x07060302u) ^ 0x80808080u;
    }
    const int G = ch >> 2, q = ch & 3;
    uint8_t* rec = lds + (G * TPG + t) * kRecBytes4 + 8 * q;
#pragma unroll
    for (int d = 0; d < 4; ++d) *reinterpret_cast<uint2*>(rec + 32 * d) = make_uint2(row[d][0], row[d][1]);
    if (q == 0) {
      const float f = __uint_as_float(static_cast<uint32_t>(127 - se) << 23);
      *reinterpret_cast<F4*>(lds + xg_off + (G * TPG + t) * kXgBytes) = F4{f, 0.0f, 0.0f, 0.0f};
    }
    return;
  }
  // s = 2^(22 - E) for max = f * 2^E, f in [0.5, 1): |x * s| < 2^22 (a
  // subnormal max takes the upper clamp)
  const int eb = static_cast<int>(__float_as_uint(m) >> 23);
  const int se = m > 0.0f ? min(max(148 - eb, -100), 126) : 0;
  const float s = __uint_as_float(static_cast<uint32_t>(se + 127) << 23);
  // x_fix = rint(x * s) (ties to even) by the 1.5 * 2^23 shift; u = x_fix +
  // 0x808080 holds the signed-byte digits of x_fix, each offset by 128
  uint32_t u[8];
  int isum = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    u[i] = __float_as_uint(__builtin_fmaf(v[i], s, 12582912.0f)) + (0x808080u - 0x4B400000u);
    isum += static_cast<int>(u[i]);
  }
  isum -= 8 * 0x808080;
  // half sums (chunks 0, 1 and 2, 3 of the group) and the other half's
  const int hs = isum + static_cast<int>(Dpp<kQuadXor1>(static_cast<uint32_t>(isum)));
  const int ho = static_cast<int>(Dpp<kQuadXor2>(static_cast<uint32_t>(hs)));
  uint32_t row[3][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t a1 = __builtin_amdgcn_perm(u[4 * h + 1], u[4 * h], 0x05010400u);
    const uint32_t a2 = __builtin_amdgcn_perm(u[4 * h + 1], u[4 * h], 0x0C0C0602u);
    const uint32_t b1 = __builtin_amdgcn_perm(u[4 * h + 3], u[4 * h + 2], 0x05010400u);
    const uint32_t b2 = __builtin_amdgcn_perm(u[4 * h + 3], u[4 * h + 2], 0x0C0C0602u);
    row[0][h] = __builtin_amdgcn_perm(b1, a1, 0x05040100u) ^ 0x80808080u;
    row[1][h] = __builtin_amdgcn_perm(b1, a1, 0x07060302u) ^ 0x80808080u;
    row[2][h] = __builtin_amdgcn_perm(b2, a2, 0x05040100u) ^ 0x80808080u;
  }
  const int G = ch >> 2, q = ch & 3;
  uint8_t* rec = lds + (G * TPG + t) * kRecBytes + 8 * q;
#pragma unroll
  for (int d = 0; d < 3; ++d) *reinterpret_cast<uint2*>(rec + 32 * d) = make_uint2(row[d][0], row[d][1]);
  if (q == 0) {
    const float f = __uint_as_float(static_cast<uint32_t>(127 - se) << 23);
    *reinterpret_cast<F4*>(lds + xg_off + (G * TPG + t) * kXgBytes) =
        F4{f, static_cast<float>(hs + ho) * f, static_cast<float>(hs) * f, static_cast<float>(ho) * f};
  }
}

// Stages tokens [0, n_tok) of the workgroup's group (rows x + t * ldx):
// chunk c = t * n8 + ch of all tokens goes to thread c % NT, round c / NT,
// so every thread has work whatever the token count (n8 % 4 == 0: a quad's
// four chunks stay one group of one token). prefetch() runs once the input
// loads are issued. With RMSNorm the inputs stay in registers between the
// sum of squares and the scaling (K <= kMaxNormK); each token's sum is then
// formed in a fixed order: per-chunk double sums in LDS (ssq), added by one
// wave per token.
template <int NW, int TPG, bool kFour, typename Prefetch>
__device__ __forceinline__ void StageTokens(const float* x, int64_t ldx, const float* norm_w, float eps, int K,
                                            int n_tok, uint8_t* lds, int xg_off, double* ssq, float* scale_sh,
                                            Prefetch prefetch) {
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n8 = K >> 3, total = n_tok * n8;
  if (norm_w != nullptr) {
    constexpr int R = (TPG * mfma::kMaxNormK / 8 + NT - 1) / NT;
    float v[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = min(tid + r * NT, total - 1);
      const int t = c / n8, ch = c - t * n8;
      const float* xr = x + t * ldx + 8 * ch;
      const F4 p = GLoad<F4>(xr), q = GLoad<F4>(xr + 4);
      v[r][0] = p.x, v[r][1] = p.y, v[r][2] = p.z, v[r][3] = p.w;
      v[r][4] = q.x, v[r][5] = q.y, v[r][6] = q.z, v[r][7] = q.w;
    }
    prefetch();
    // reference RMSNorm: double sum of squares, float scale, (x * scale) * w
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = tid + r * NT;
      if (c < total) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += static_cast<double>(v[r][i]) * v[r][i];
        ssq[c] = ss;
      }
    }
    LdsBarrier();
    for (int t = wave; t < n_tok; t += NW) {
      double ss = 0.0;
      for (int ch = lane; ch < n8; ch += 64) ss += ssq[t * n8 + ch];
      ss = WaveSumD(ss);
      if (lane == 0)
        scale_sh[t] =
            static_cast<float>(1.0 / __builtin_sqrt(ss / static_cast<double>(K) + static_cast<double>(eps)));
    }
    LdsBarrier();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = tid + r * NT;
      if (c < total) {
        const int t = c / n8, ch = c - t * n8;
        const float sc = scale_sh[t];
        const F4 a = GLoad<F4>(norm_w + 8 * ch), b = GLoad<F4>(norm_w + 8 * ch + 4);
        const float w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float u[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = __fmul_rn(__fmul_rn(v[r][i], sc), w[i]);
        StageChunk<kFour>(u, t, TPG, ch, lds, xg_off);
      }
    }
  } else {
    constexpr int R = 4;  // chunks per thread in flight per round
    bool first = true;
    for (int base = 0; base < total; base += R * NT) {
      float v[R][8];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int c = min(base + tid + r * NT, total - 1);
        const int t = c / n8, ch = c - t * n8;
        const float* xr = x + t * ldx + 8 * ch;
        const F4 p = GLoad<F4>(xr), q = GLoad<F4>(xr + 4);
        v[r][0] = p.x, v[r][1] = p.y, v[r][2] = p.z, v[r][3] = p.w;
        v[r][4] = q.x, v[r][5] = q.y, v[r][6] = q.z, v[r][7] = q.w;
      }
      if (first) prefetch();
      first = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int c = base + tid + r * NT;
        if (c < total) {
          const int t = c / n8;
          StageChunk<kFour>(v[r], t, TPG, c - t * n8, lds, xg_off);
        }
      }
    }
  }
  LdsBarrier();
}

// No MFMA here may get a destination that aliases its A or B registers (such
// an MFMA has returned wrong sums on gfx950). HoldSources keeps the sources
// live until the accumulator that uses the product exists, so the register
// allocator cannot give the product their registers. The asm is not volatile
// (loads may still move across it) and rewrites only that float accumulator:
// a VALU result, so no MFMA-to-VALU wait is hidden behind it (an asm that
// rewrote the MFMA result itself would hide the wait its readers need).
__device__ __forceinline__ I4 Mfma32(U2 a, U2 b) {
  const I4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), z, 0, 0, 0);
}
__device__ __forceinline__ void HoldSources(float& acc, U2 a, U2 b) { asm("" : "+v"(acc) : "v"(a), "v"(b)); }
__device__ __forceinline__ void HoldSources(float& acc, U2 a, U2 b0, U2 b1) {
  asm("" : "+v"(acc) : "v"(a), "v"(b0), "v"(b1));
}

// sum(q * x_fix) from the three digit sums
__device__ __forceinline__ float DigitSum(I4 c) {
  const int t = c[1] + c[2] * 256;
  return __builtin_fmaf(static_cast<float>(t), 256.0f, static_cast<float>(c[0]));
}
// The same for 32 weights below 16: |sum| <= 32 * 15 * 2^22 and the top
// digit is within [-64, 64], so the sum is exact in int32.
__device__ __forceinline__ float DigitSum4(I4 c) { return static_cast<float>(c[0] + c[1] * 256 + c[2] * 65536); }

__device__ __forceinline__ U2 LdsU2(const uint8_t* p) { return *reinterpret_cast<const U2*>(p); }

// float(byte I of w) in one instruction
template <int I>
__device__ __forceinline__ float CvtByte(uint32_t w) {
  float r;
  if constexpr (I == 0)
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  else if constexpr (I == 1)
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  else if constexpr (I == 2)
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
  else
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
  return r;
}

// ---------------------------------------------------------------- Q4_K

// One super-block of the lane's row in the tile-major chunk (16 blocks of
// 144 bytes): the header and quant bytes 32p + 8g .. + 8 of each pair p.
struct Q4B {
  U4 hdr;
  U2 q[4];
  __device__ __forceinline__ void Load(Rsrc r, int chunk, int col, int g) {
    hdr = __builtin_amdgcn_raw_buffer_load_b128(r, 144 * col, chunk, 0);
#pragma unroll
    for (int p = 0; p < 4; ++p) q[p] = __builtin_amdgcn_raw_buffer_load_b64(r, 144 * col + 16 + 32 * p + 8 * g, chunk, 0);
  }
};

// acc[Q] += the lane's row . token 4Q + g over super-block sb. rec: the
// lane's digit row of token col / 4 of group 0; xg: token g's sums of group 0.
template <int TPG>
__device__ __forceinline__ void Q4Dot(const Q4B& u, const uint8_t* rec, const uint8_t* xg, int sb,
                                      float (&acc)[TPG / 4]) {
  const float d = dev::HalfToFloatFast(u.hdr.x & 0xFFFFu);
  const float dmin = dev::HalfToFloatFast(u.hdr.x >> 16);
  // scales / mins of sub-blocks 0..3 and 4..7, one per byte (reference
  // src/quant.cc:159-167)
  const uint32_t Y = u.hdr.y, Z = u.hdr.z, W = u.hdr.w;
  const uint32_t scw[2] = {Y & 0x3F3F3F3Fu, (W & 0x0F0F0F0Fu) | ((Y >> 2) & 0x30303030u)};
  const uint32_t mw[2] = {Z & 0x3F3F3F3Fu, ((W >> 4) & 0x0F0F0F0Fu) | ((Z >> 2) & 0x30303030u)};
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const U2 w = u.q[s >> 1];
    const U2 b = (s & 1) ? U2{(w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu}
                         : U2{w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu};
    float sc, mn;
    switch (s & 3) {
      case 0: sc = CvtByte<0>(scw[s >> 2]); mn = CvtByte<0>(mw[s >> 2]); break;
      case 1: sc = CvtByte<1>(scw[s >> 2]); mn = CvtByte<1>(mw[s >> 2]); break;
      case 2: sc = CvtByte<2>(scw[s >> 2]); mn = CvtByte<2>(mw[s >> 2]); break;
      default: sc = CvtByte<3>(scw[s >> 2]); mn = CvtByte<3>(mw[s >> 2]); break;
    }
    const float dsc = d * sc, dm = dmin * mn;
    const int G = 8 * sb + s;
#pragma unroll
    for (int Q = 0; Q < TPG / 4; ++Q) {
      const U2 a = LdsU2(rec + (G * TPG + 4 * Q) * kRecBytes);
      const I4 c = Mfma32(a, b);
      const F2 fx = *reinterpret_cast<const F2*>(xg + (G * TPG + 4 * Q) * kXgBytes);  // (1/s, sum x)
      acc[Q] = __builtin_fmaf(dsc * fx.x, DigitSum4(c), acc[Q]);
      HoldSources(acc[Q], a, b);
      acc[Q] = __builtin_fmaf(-dm, fx.y, acc[Q]);
    }
  }
}

// ---------------------------------------------------------------- Q6_K

// One super-block of the lane's row in the tile-major Q6_K chunk (the 16
// rows' ql, then qh, scales and d, decode.h): ql bytes 64hh + 32r + 8g .. + 8,
// qh bytes 32hh + 8g .. + 8, the 16 scales and d.
struct Q6B {
  U2 ql[4], qh[2];
  U4 sc;
  uint32_t d;
  __device__ __forceinline__ void Load(Rsrc r, int chunk, int col, int g) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ql[i] = __builtin_amdgcn_raw_buffer_load_b64(r, mfma::kQ6Ql + 128 * col + 32 * i + 8 * g, chunk, 0);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      qh[hh] = __builtin_amdgcn_raw_buffer_load_b64(r, mfma::kQ6Qh + 64 * col + 32 * hh + 8 * g, chunk, 0);
    sc = __builtin_amdgcn_raw_buffer_load_b128(r, mfma::kQ6Sc + 16 * col, chunk, 0);
    d = __builtin_amdgcn_raw_buffer_load_b16(r, mfma::kQ6D + 2 * col, chunk, 0);
  }
};

// acc[Q] += the lane's row . token 4Q + g over super-block sb (rec, xg as
// for Q4Dot); lo: the lane's k-group lies in half 0 of each 32-group.
template <int TPG>
__device__ __forceinline__ void Q6Dot(const Q6B& u, const uint8_t* rec, const uint8_t* xg, int sb, bool lo,
                                      float (&acc)[TPG / 4]) {
  const float d = dev::HalfToFloatFast(u.d & 0xFFFFu);
  const uint32_t scw[4] = {u.sc.x, u.sc.y, u.sc.z, u.sc.w};
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      // weights 128hh + 32qq + l: ql[64hh + 32(qq & 1) + l] nibble qq / 2, qh
      // bits 2qq (reference src/quant.cc:200-237)
      const U2 w = u.ql[2 * hh + (qq & 1)], hq = u.qh[hh];
      U2 b;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t we = e ? w.y : w.x, he = e ? hq.y : hq.x;
        const uint32_t nib = (qq >> 1) ? (we >> 4) & 0x0F0F0F0Fu : we & 0x0F0F0F0Fu;
        const uint32_t hb = qq == 0 ? (he << 4) : qq == 1 ? (he << 2) : qq == 2 ? he : (he >> 2);
        b[e] = nib | (hb & 0x30303030u);
      }
      const U2 b0 = lo ? b : U2{0u, 0u}, b1 = lo ? U2{0u, 0u} : b;
      // scales of sub-blocks 8hh + 2qq (half 0) and + 1 (half 1), signed bytes
      const int si = 8 * hh + 2 * qq;
      const float dsc0 = d * static_cast<float>(__builtin_amdgcn_sbfe(scw[si >> 2], 8 * (si & 3), 8));
      const float dsc1 = d * static_cast<float>(__builtin_amdgcn_sbfe(scw[si >> 2], 8 * (si & 3) + 8, 8));
      const int G = 8 * sb + 4 * hh + qq;
#pragma unroll
      for (int Q = 0; Q < TPG / 4; ++Q) {
        const U2 a = LdsU2(rec + (G * TPG + 4 * Q) * kRecBytes);
        const I4 c0 = Mfma32(a, b0);
        const I4 c1 = Mfma32(a, b1);
        const F4 xs = *reinterpret_cast<const F4*>(xg + (G * TPG + 4 * Q) * kXgBytes);  // (1/s, sum, half 0, half 1)
        float r = __builtin_fmaf(dsc0 * xs.x, DigitSum(c0), acc[Q]);
        r = __builtin_fmaf(dsc1 * xs.x, DigitSum(c1), r);
        HoldSources(r, a, b0, b1);
        r = __builtin_fmaf(-32.0f * dsc0, xs.z, r);
        acc[Q] = __builtin_fmaf(-32.0f * dsc1, xs.w, r);
      }
    }
  }
}

// ---------------------------------------------------------------- Q8_0

// One super-block (8 blocks of 32) of the lane's row in the tile-major Q8_0
// chunk (mfma_dot.h: byte 1024 m + 64 j + 16 g' + e is weight 64 m + 16 g'
// + e of row j, then the 16 rows' block scales at 4096 + 16 j): for block b
// the 8 quants 32 b + 8 g .. + 8 (m = b / 2, g' = 2 (b % 2) + g / 2, e from
// 8 (g % 2)), and the row's 8 scales.
struct Q8B {
  U2 q[8];
  U4 s;
  __device__ __forceinline__ void Load(Rsrc r, int chunk, int col, int g) {
#pragma unroll
    for (int b = 0; b < 8; ++b)
      q[b] = __builtin_amdgcn_raw_buffer_load_b64(
          r, 1024 * (b >> 1) + 64 * col + 16 * (2 * (b & 1) + (g >> 1)) + 8 * (g & 1), chunk, 0);
    s = __builtin_amdgcn_raw_buffer_load_b128(r, mfma::kQ8Sc + 16 * col, chunk, 0);
  }
};

// acc[Q] += the lane's row . token 4Q + g over super-block sb (rec: the
// lane's four-digit row of token col / 4 of group 0; xg as for Q4Dot).
template <int TPG>
__device__ __forceinline__ void Q8Dot(const Q8B& u, const uint8_t* rec, const uint8_t* xg, int sb,
                                      float (&acc)[TPG / 4]) {
  const uint32_t sw[4] = {u.s.x, u.s.y, u.s.z, u.s.w};
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const float d = dev::HalfToFloatFast((sw[b >> 1] >> (16 * (b & 1))) & 0xFFFFu);
    const int G = 8 * sb + b;
#pragma unroll
    for (int Q = 0; Q < TPG / 4; ++Q) {
      const U2 a = LdsU2(rec + (G * TPG + 4 * Q) * kRecBytes4);
      const I4 c = Mfma32(a, u.q[b]);
      const float f = *reinterpret_cast<const float*>(xg + (G * TPG + 4 * Q) * kXgBytes);  // 1/s
      // |C| <= 32 * 128 * 128: C1 + 2^8 C2 is exact in int32, the rest in double
      const double t = static_cast<double>(c[1] + 256 * c[2]);
      const float sum = static_cast<float>(__builtin_fma(static_cast<double>(c[3]), 16777216.0,
                                                         __builtin_fma(t, 256.0, static_cast<double>(c[0]))));
      acc[Q] = __builtin_fmaf(d * f, sum, acc[Q]);
      HoldSources(acc[Q], a, u.q[b]);
    }
  }
}

// ---------------------------------------------------------------- tiles

enum : int { kKindQ6 = 0, kKindQ4 = 1, kKindQ8 = 2 };

// One wave's tile (or its part of the tile's super-blocks) for the
// workgroup's token group: Setup picks the tile's range, Prefetch requests
// its first weight batch, Run computes, reduces and writes y (or leaves its
// sums to part 0).
template <int NW, int TPG, int kKind>
struct WaveTile {
  static constexpr bool kQ4 = kKind == kKindQ4, kQ8 = kKind == kKindQ8;
  using U = typename std::conditional<kQ4, Q4B, typename std::conditional<kQ8, Q8B, Q6B>::type>::type;
  static constexpr int kNB = kQ4 ? 2 : 1;  // super-blocks per load batch (Q6_K: 32 MFMAs each at 8 tokens)
  static constexpr int BB = kQ4 ? 144 : kQ8 ? 272 : 210;
  U ua[kNB], ub[kNB];
  Rsrc rsrc;
  int lo, hi, n_part;
  bool active;

  __device__ __forceinline__ void Setup(const DecodeJob& J, int K, int tile, bool act, int part, int kwl) {
    const int n_sb = K >> 8;
    active = act;
    rsrc = TileRsrc(J.w + static_cast<int64_t>(act ? tile : 0) * n_sb * 16 * BB, n_sb * 16 * BB);
    lo = (part * n_sb) >> kwl;
    hi = ((part + 1) * n_sb) >> kwl;
    n_part = hi - lo;
  }
  __device__ __forceinline__ void Load(U* u, int bt) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int b = 0; b < kNB; ++b) u[b].Load(rsrc, 16 * BB * min(lo + bt * kNB + b, hi - 1), lane & 15, lane >> 4);
  }
  __device__ __forceinline__ void Prefetch() {
    if (active) Load(ua, 0);
  }

  __device__ __forceinline__ void Run(const BatchArgs& a, const DecodeJob& J, int64_t ldy, int tile, int part, int kwl,
                                      int tok0, int n_tok, const uint8_t* lds, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4, kw = 1 << kwl;
    // the lane's A row: digit min(col % 4, 2) (four-digit records: col % 4)
    // of token col / 4 of each quad; its results: token g of each quad
    const uint8_t* rec = kQ8 ? lds + (col >> 2) * kRecBytes4 + 32 * (col & 3) + 8 * g
                             : lds + (col >> 2) * kRecBytes + 32 * min(col & 3, 2) + 8 * g;
    const uint8_t* xg = lds + a.xg_off + g * kXgBytes;
    constexpr int NQ = TPG / 4;
    float acc[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) acc[i] = 0.0f;
    auto comp = [&](const U* u, int bt) {
#pragma unroll
      for (int b = 0; b < kNB; ++b) {
        const int i = bt * kNB + b;
        if (i >= n_part) break;
        if constexpr (kQ4)
          Q4Dot<TPG>(u[b], rec, xg, lo + i, acc);
        else if constexpr (kQ8)
          Q8Dot<TPG>(u[b], rec, xg, lo + i, acc);
        else
          Q6Dot<TPG>(u[b], rec, xg, lo + i, g < 2, acc);
      }
    };
    if (active) {
      // ua holds batch 0 (Prefetch). The loads are unconditional (past the
      // range they repeat the last super-block) so that every wait on them
      // has a fixed count.
      const int nb = (n_part + kNB - 1) / kNB;
      for (int bt = 0; bt < nb; bt += 2) {
        Load(ub, bt + 1);
        comp(ua, bt);
        if (bt + 1 >= nb) break;
        Load(ua, bt + 2);
        comp(ub, bt + 1);
      }
    }
    // lane (col, g) holds token 4i + g of row col; cross-wave sums in LDS,
    // red[wave][t][col], added by part 0 in part order
    if (kw > 1) {
#pragma unroll
      for (int i = 0; i < NQ; ++i) red[(wave * TPG + 4 * i + g) * 16 + col] = acc[i];
      LdsBarrier();
      if (part != 0) return;
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int t = 4 * i + g;
        float sum = red[(wave * TPG + t) * 16 + col];
        for (int p = 1; p < kw; ++p) sum += red[((wave + p) * TPG + t) * 16 + col];
        acc[i] = sum;
      }
    }
    if (!active) return;
    const bool pair = J.pair != 0;
    const int row = tile * (pair ? 8 : 16) + (pair ? (col & 7) : col);
    const bool valid = row < J.rows && (!pair || col < 8);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int t = 4 * i + g;
      if (pair) {
        const float up = __uint_as_float(Dpp<kRowRor8>(__float_as_uint(acc[i])));  // cols 0..7 <- 8..15
        if (valid && t < n_tok) {
          // silu(g) * up with glibc-exact expf (reference src/kernels.h:82-92)
          const float gv = acc[i];
          const float sg = gv / __fadd_rn(1.0f, GlibcExpf(-gv));
          J.y[(tok0 + t) * ldy + row] = __fmul_rn(sg, up);
        }
      } else if (valid && t < n_tok) {
        float* y = J.y + (tok0 + t) * ldy + row;
        *y = a.epi == kAdd ? *y + acc[i] : acc[i];
      }
    }
  }
};

// kTypes: bit 0 = Q4_K jobs present, bit 1 = Q6_K jobs present; 4 = every
// job Q8_0 (four-digit staging; never mixed with the others). Each
// workgroup stages its token group once, then takes units first, first +
// stride, ... (a unit: NW / kw tiles); the first unit's weights are
// requested while the inputs are staged.
template <int kTypes, int NW, int TPG>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4, 4))) void MatvecBatchKernel(BatchArgs a) {
  extern __shared__ __align__(256) uint8_t lds[];
  __shared__ float scale_sh[TPG];
  const int wave = threadIdx.x >> 6;
  const int n_tg = Uniform(a.n_tg), units = Uniform(a.units);
  // block -> (token group, first unit): the groups of one unit are 8 blocks
  // apart (the same XCD) and walk the same units
  int first = static_cast<int>(blockIdx.x), tg = 0, stride = static_cast<int>(gridDim.x);
  if (n_tg > 1) {
    const int b = static_cast<int>(blockIdx.x), q = b >> 3;
    tg = q % n_tg;
    first = (q / n_tg) * 8 + (b & 7);
    stride = static_cast<int>(gridDim.x) / n_tg;
  }
  if (first >= units) return;  // the whole workgroup
  const int kwl = Uniform(a.kw_log2);
  const int tpg = Uniform(a.tpg), T = Uniform(a.T);
  const int tok0 = tg * tpg, n_tok = min(tpg, T - tok0);
  const int K = Uniform(a.K);
  const int n_jobs = Uniform(a.n_jobs), tiles0 = Uniform(a.tiles0), tiles1 = Uniform(a.tiles1);
  constexpr int kNWLog2 = NW == 4 ? 2 : NW == 8 ? 3 : 4;
  const int part = __builtin_amdgcn_readfirstlane(wave & ((1 << kwl) - 1));
  struct Map {
    int j, tile;
    bool active;
  };
  auto map = [&](int unit) {
    Map m;
    int tile = __builtin_amdgcn_readfirstlane((unit << (kNWLog2 - kwl)) + (wave >> kwl));
    int j = 0;
    if (n_jobs > 1 && tile >= tiles0) {
      tile -= tiles0;
      j = 1;
      if (n_jobs > 2 && tile >= tiles1) {
        tile -= tiles1;
        j = 2;
      }
    }
    m.j = j;
    m.tile = tile;
    m.active = tile < a.job[j].tiles;
    return m;
  };
  // single-type launches prefetch across the staging; mixed ones load after
  constexpr bool kFour = kTypes == 4;
  constexpr bool kPre = (kTypes & 3) != 3;
  constexpr int kKind = kFour ? kKindQ8 : (kTypes & 3) == 1 ? kKindQ4 : kKindQ6;
  WaveTile<NW, TPG, kKind> pre;
  const Map m0 = map(first);
  if constexpr (kPre) pre.Setup(a.job[m0.j], K, m0.tile, m0.active, part, kwl);
  double* ssq = reinterpret_cast<double*>(lds + a.red_off);  // (the cross-wave sums' space, free until the first unit ends)
  StageTokens<NW, TPG, kFour>(a.x + tok0 * a.ldx, a.ldx, a.norm_w, a.eps, K, n_tok, lds, a.xg_off, ssq, scale_sh, [&]() {
    if constexpr (kPre) pre.Prefetch();
  });
  int parity = 0;
  for (int unit = first; unit < units; unit += stride, parity ^= 1) {
    const Map m = unit == first ? m0 : map(unit);
    const DecodeJob& J = a.job[m.j];
    const int64_t ldy = a.ldy[m.j];
    // cross-wave sums alternate between two buffers: a wave writing unit
    // i + 1's sums has passed unit i + 1's barrier, which every reader of
    // unit i's sums reaches only after reading them
    float* red = reinterpret_cast<float*>(lds + a.red_off) + parity * (NW * TPG * 16);
    if constexpr (kPre) {
      if (unit != first) {
        pre.Setup(J, K, m.tile, m.active, part, kwl);
        pre.Prefetch();
      }
      pre.Run(a, J, ldy, m.tile, part, kwl, tok0, n_tok, lds, red);
    } else {
      if (J.type == kQ4_K) {
        WaveTile<NW, TPG, kKindQ4> w;
        w.Setup(J, K, m.tile, m.active, part, kwl);
        w.Prefetch();
        w.Run(a, J, ldy, m.tile, part, kwl, tok0, n_tok, lds, red);
      } else {
        WaveTile<NW, TPG, kKindQ6> w;
        w.Setup(J, K, m.tile, m.active, part, kwl);
        w.Prefetch();
        w.Run(a, J, ldy, m.tile, part, kwl, tok0, n_tok, lds, red);
      }
    }
  }
}

// dynamic LDS a launch may ask for: the staging budget, the cross-wave sums
constexpr int kMaxDynLds = kLdsBudget + 2 * 8 * 8 * 16 * 4;  // (the budget covers the staging's sums of squares)

template <int kTypes, int NW, int TPG>
void Launch(const BatchArgs& a, unsigned blocks, size_t lds, hipStream_t s) {
  static const bool opted = [] {  // more than 64 KiB of dynamic LDS
    HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(MatvecBatchKernel<kTypes, NW, TPG>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds));
    return true;
  }();
  (void)opted;
  RPG_CHECK(lds <= static_cast<size_t>(kMaxDynLds), "batch matvec: %zu bytes of LDS", lds);
  hipLaunchKernelGGL((MatvecBatchKernel<kTypes, NW, TPG>), dim3(blocks), dim3(64 * NW), lds, s, a);
}

template <int NW, int TPG>
void LaunchTypes(int types, const BatchArgs& a, unsigned blocks, size_t lds, hipStream_t s) {
  switch (types) {
    case 1: Launch<1, NW, TPG>(a, blocks, lds, s); break;
    case 2: Launch<2, NW, TPG>(a, blocks, lds, s); break;
    case 4: Launch<4, NW, TPG>(a, blocks, lds, s); break;
    default: Launch<3, NW, TPG>(a, blocks, lds, s); break;
  }
}

int EnvInt(const char* name) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : 0;
}

}  // namespace

int FewTokenLimit() {
  static const int limit = [] {
    const int e = EnvInt("RPG_FEW_TOKENS");
    return e >= 1 && e <= kMaxBatchTokens ? e : kFewTokensDefault;
  }();
  return limit;
}

namespace {

int ComputeUnits() {
  static int cus[64] = {0};
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) HIP_CHECK(hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
  return cus[dev];
}

}  // namespace

bool DecodeMatvecBatch(const DecodeBatchArgs& in, hipStream_t s) {
  const int K = in.K, T = in.T;
  if (T < 1 || T > kMaxBatchTokens || K <= 0 || K % 256 != 0 || in.n_jobs < 1 || in.n_jobs > 3) return false;
  BatchArgs a{};
  a.x = in.x;
  a.ldx = in.ldx;
  a.norm_w = in.norm_w;
  a.eps = in.eps;
  a.K = K;
  a.T = T;
  a.epi = in.epi;
  a.n_jobs = in.n_jobs;
  int types = 0, tiles = 0;
  for (int j = 0; j < in.n_jobs; ++j) {
    DecodeJob J = in.job[j];
    if (!J.tiled || J.w2 != nullptr || (J.type != kQ4_K && J.type != kQ6_K && J.type != kQ8_0)) return false;
    const int64_t rb = (K / 256) * (J.type == kQ4_K ? 144 : J.type == kQ6_K ? 210 : 272);
    RPG_CHECK(J.row_bytes == rb, "batch matvec: row bytes %lld do not match K = %d", (long long)J.row_bytes, K);
    RPG_CHECK(in.ldy[j] >= J.rows, "batch matvec: output stride %lld below %d rows", (long long)in.ldy[j], J.rows);
    types |= J.type == kQ4_K ? 1 : J.type == kQ6_K ? 2 : 4;
    J.rows_per_tile = J.pair ? 8 : 16;
    J.tiles = static_cast<int32_t>(CeilDiv(J.rows, J.rows_per_tile));
    tiles += J.tiles;
    a.job[j] = J;
    a.ldy[j] = in.ldy[j];
  }
  if ((types & 4) != 0 && types != 4) return false;  // Q8_0 stages four digits: no launch mixes it with the others
  if (in.norm_w != nullptr && K > mfma::kMaxNormK) return false;  // the normed staging holds its inputs in registers
  const int rec = types == 4 ? kRecBytes4 : kRecBytes;
  // Tokens per workgroup: as many as fit the LDS budget, spread evenly over
  // the groups. LDS holds TPG token slots (4 or 8): a token quad's MFMA
  // reads all four slots, staged or not (the unstaged ones feed only the
  // sums of tokens that are not written).
  // (with RMSNorm the staging also keeps a double per 8 inputs)
  const int64_t per_tok = static_cast<int64_t>(K / 32) * (rec + kXgBytes) + (in.norm_w != nullptr ? K : 0);
  const int64_t fit = kLdsBudget / per_tok;
  if (fit < 4) return false;
  const int cap = fit >= 8 ? 8 : 4;
  const int n_tg = (T + cap - 1) / cap;
  const int tpg = (T + n_tg - 1) / n_tg;
  const int TPG = tpg <= 4 ? 4 : 8;
  a.tpg = tpg;
  a.n_tg = n_tg;
  a.tiles0 = a.job[0].tiles;
  a.tiles1 = in.n_jobs > 1 ? a.job[1].tiles : 0;
  constexpr int NW = 8;
  int off = TPG * (K / 32) * rec;
  a.xg_off = off;
  off += TPG * (K / 32) * kXgBytes;
  a.red_off = off;  // the cross-wave sums (two buffers), first the staging's sums of squares
  off += std::max(2 * NW * TPG * 16 * 4, in.norm_w != nullptr ? TPG * K : 0);
  const size_t dyn = static_cast<size_t>(off);
  // Resident workgroups: two per compute unit (16 waves) where the LDS
  // allows, else one; each token group gets its share, in multiples of 8
  // when there are several (a unit's groups sit 8 blocks apart).
  const int per_cu = static_cast<int>(std::min<size_t>(2, 163840 / (dyn + NW * TPG * 8)));
  RPG_CHECK(per_cu >= 1, "batch matvec: %zu bytes of LDS", dyn);
  const int slots = std::max(8, ComputeUnits() * per_cu / n_tg / 8 * 8);
  // Waves per tile (kw): the split of the super-blocks that minimises
  // rounds x (super-blocks per wave + 2), the 2 standing for a round's
  // fixed costs (first loads, cross-wave sums, epilogue).
  const int n_sb = K / 256;
  int kw = 1;
  int64_t best = INT64_MAX;
  for (int c = 1; c <= 8 && c <= n_sb; c *= 2) {
    const int64_t units = CeilDiv(tiles, NW / c);
    const int64_t rounds = CeilDiv(units, slots);
    const int64_t cost = rounds * (CeilDiv(n_sb, c) + 2);
    if (cost < best) {
      best = cost;
      kw = c;
    }
  }
  const int force = EnvInt("RPG_BATCH_KW");  // tuning sweeps
  if (force == 1 || force == 2 || force == 4 || force == 8) kw = std::min(force, n_sb >= 8 ? 8 : n_sb >= 4 ? 4 : n_sb >= 2 ? 2 : 1);
  a.kw_log2 = kw == 1 ? 0 : kw == 2 ? 1 : kw == 4 ? 2 : 3;
  a.units = static_cast<int32_t>(CeilDiv(tiles, NW / kw));
  const int64_t per_group = n_tg == 1 ? std::min<int64_t>(a.units, slots)
                                      : std::min<int64_t>(CeilDiv(a.units, 8) * 8, slots);
  const unsigned blocks = static_cast<unsigned>(per_group * n_tg);
  if (TPG == 4)
    LaunchTypes<NW, 4>(types, a, blocks, dyn, s);
  else
    LaunchTypes<NW, 8>(types, a, blocks, dyn, s);
  HIP_CHECK(hipGetLastError());
  return true;
}

}  // namespace k
}  // namespace rpg
