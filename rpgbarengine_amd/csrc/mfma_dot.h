// Building blocks of the decode matvec on the int8 matrix cores, shared by the
// per-launch kernel (matvec_mfma.hip) and the persistent decode step
// (decode_step.hip).
//
// Decode (one-token) matvec on the matrix cores, for Q4_K, Q6_K and Q8_0
// weights (Q8_0 from its tile-major copy only; see MUnit<kQ8T>).
//
// v_mfma_i32_16x16x64_i8 computes C[i][j] += sum_k A[i][k] * B[k][j] in exact
// int32; lane L = j + 16g supplies 16 bytes of B column j and 16 bytes of A
// row L % 16 for the same 16 k, and holds C[4g..4g+4)[j] afterwards. Here
//   B (weights): column j is one output row (16 rows per tile, or 8 rows of
//     each matrix of a SwiGLU pair). Lane (j, g) feeds the 16 quants of one
//     nibble slot of its own 16 raw quant bytes: w & 0x0F0F0F0F (low nibbles)
//     or (w >> 4) & 0x0F0F0F0F (high nibbles), Q6_K with its two high bits
//     OR-ed in -- unsigned 4- / 6-bit values, so one or two ops per 4 weights.
//   A (input): block diagonal. Row 4g + d (d = 0, 1, 2) is nonzero only at
//     lane group g's 16 k and holds digit d of the fixed-point inputs there;
//     row 4g + 3 is zero. The 16 inputs of one slot are always one aligned
//     16-element group of x; each group is scaled by its own power of two
//     s_g into |x * s_g| < 2^22 and rounded, x_fix = d0 + 2^8 d1 + 2^16 d2
//     with signed-byte digits.
// So C[4g + d][j] is lane (j, g)'s own exact digit sum for one (sub-block,
// slot): sum(q * x_fix) = C0 + 2^8 C1 + 2^16 C2, and the lane applies its
// scales once per MFMA with no data exchange between lanes:
//   Q4_K  (d*sc) * sum(q*x) - (dmin*m) * sum(x)   (reference src/quant.cc:159-198)
//   Q6_K  (d*sc) * sum(q*x) - (32*d*sc) * sum(x)  (src/quant.cc:200-237)
// with sum(x) = f_g * sum(x_fix), f_g = 1 / s_g, staged per group. The dot is
// the reference dot (src/matmul.cc:73-102, src/matmul_avx2.cc:95-289) of the
// inputs rounded to 22 bits below their group's maximum, up to the float
// rounding of the two scaled terms; dots are judged by max|d| / sum|a*w| <=
// 1e-6.
//
// Lane (j, g) covers, per 256-weight super-block, two windows c of 16 quant
// bytes (32 weights each, low and high nibble slots):
//   Q4_K: quant bytes 64c + 16g + [0, 16): weights 64p + 16(g%2) + e (low
//         nibble) and 64p + 32 + 16(g%2) + e (high), p = 2c + g/2, i.e.
//         sub-blocks 2p and 2p + 1;
//   Q6_K: ql bytes 64h + 32c + 16(g%2) + e, qh bytes 32h + 16(g%2) + e
//         (h = g/2): weights 128h + 32c + 16(g%2) + e (low nibble, qh bits
//         2c) and 128h + 64 + 32c + 16(g%2) + e (high nibble, qh bits
//         2c + 4), scales 8h + 2c + g%2 and 8h + 4 + 2c + g%2.
// Q6_K blocks (210 bytes) are only 2-byte aligned: words are loaded from the
// 4-byte-aligned address below and realigned with v_alignbyte.
//
// Work: a workgroup of NW waves takes NW / kw tiles; the kw waves of a tile
// split its super-blocks (part p takes the p-th of kw contiguous ranges) and
// add their sums in LDS in a fixed order. Weights are read row-major or from
// the tile-major decode copy (decode.h), where a wave streams contiguous
// bytes. The input is staged once per workgroup -- RMSNorm
// when the projection consumes one (reference src/qwen3.cc:131-134,191-194,
// 284-287), the digit records (64 bytes per 16-group: digit rows 0..2 and a
// zero row) and per group (f_g, sum(x)) -- with the first batch of weight
// loads in flight meanwhile.

#ifndef RPG_HIP_MFMA_DOT_H_
#define RPG_HIP_MFMA_DOT_H_

#include <hip/hip_runtime.h>

#include "common.h"
#include "decode.h"
#include "expf_glibc.h"
#include "lanes.h"
#include "quant_dev.h"

namespace rpg {
namespace k {
namespace mfma {

constexpr int kMaxK = 10240;
constexpr int kMaxNormK = 4096;
constexpr int kNB = 2;            // super-blocks per load batch
constexpr int kZeroBytes = 1024;  // zeros read by the off-diagonal lanes

typedef uint32_t U4 __attribute__((ext_vector_type(4)));
typedef uint32_t U3 __attribute__((ext_vector_type(3)));
typedef uint32_t U2 __attribute__((ext_vector_type(2)));
typedef U4 U4A4 __attribute__((aligned(4)));
typedef U3 U3A4 __attribute__((aligned(4)));
typedef int I4 __attribute__((ext_vector_type(4)));
typedef float F4 __attribute__((ext_vector_type(4)));

// The header (first 64 bytes) holds what the prologue reads before it knows
// its job; the jobs follow.

// The header in scalar registers, as the staging and the tiles use it.
struct Hdr {
  const float* norm_w;
  int32_t K, epi, kwl, zero_off, xg_off, red_off;
  float eps;
};

using lanes::Uniform;

// A buffer resource over one tile's bytes: loads take the wave-uniform chunk
// offset in a scalar register and the lane's offset in a vector register,
// and an offset past the tile reads zeros.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc TileRsrc(const uint8_t* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, bytes, 0x00020000);
}

template <typename T>
__device__ __forceinline__ T GLoad(const uint8_t* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

using lanes::AddXor16;
using lanes::AddXor32;
using lanes::Dpp;
using lanes::kQuadXor1;
using lanes::kRowRor8;
using lanes::WaveSumD;

// Workgroup barrier that orders LDS only: outstanding global loads (the
// weight prefetch) stay in flight across it.
__device__ __forceinline__ void LdsBarrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int I>
__device__ __forceinline__ float CvtU8(uint32_t w) {
  float r;
  if constexpr (I == 0)
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  else
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  return r;
}

// The thread's 8-value chunks of the input (and of the RMSNorm gain): chunk
// tid + c * 64 * NW in row c. Rows c < nc hold inputs (the test is uniform
// over the workgroup); within a row, indices are clamped into range.
template <int NW>
struct XChunks {
  static constexpr int NT = 64 * NW;
  static constexpr int NC = (kMaxK / 8 + NT - 1) / NT;
  static constexpr int NNC = (kMaxNormK / 8 + NT - 1) / NT;
  float v[NC][8], wv[NNC][8];
  int nc;
  // issued first thing in the kernel: the inputs depend on no job
  __device__ __forceinline__ void Load(const float* x, const float* norm_w, int K) {
    const int tid = threadIdx.x, n8 = K >> 3;
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(x);
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(norm_w != nullptr ? norm_w : x);
    nc = (n8 + NT - 1) / NT;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c >= nc) break;
      const int ch = min(tid + c * NT, n8 - 1);
      const F4 p = GLoad<F4>(xb + 32 * ch), q = GLoad<F4>(xb + 32 * ch + 16);
      v[c][0] = p.x, v[c][1] = p.y, v[c][2] = p.z, v[c][3] = p.w;
      v[c][4] = q.x, v[c][5] = q.y, v[c][6] = q.z, v[c][7] = q.w;
    }
    if (norm_w != nullptr) {
#pragma unroll
      for (int c = 0; c < NNC; ++c) {
        if (c >= nc) break;
        const int ch = min(tid + c * NT, n8 - 1);
        const F4 p = GLoad<F4>(wb + 32 * ch), q = GLoad<F4>(wb + 32 * ch + 16);
        wv[c][0] = p.x, wv[c][1] = p.y, wv[c][2] = p.z, wv[c][3] = p.w;
        wv[c][4] = q.x, wv[c][5] = q.y, wv[c][6] = q.z, wv[c][7] = q.w;
      }
    }
  }
};

// Stages the input (see the file comment) from the chunks in flight.
// prefetch() runs first: it issues the first weight loads, which complete
// after the input loads (loads complete in issue order). kFour (the Q8_0
// launches): four digits per input, |x * s_g| < 2^30, in all four record
// rows (the A operand's row 4g + 3 then holds digit 3); the per-group sum of
// the inputs is not formed (Q8_0 has no min term).
//
// RMSNorm (norm_w set; reference src/kernels.h:56-63: double sum of squares,
// float scale = 1 / sqrt(mean + eps), (x * scale) * w). kDeferNorm: the
// digits are those of x * w and the returned scale multiplies the dot
// products at the end (they are linear in the input), so the staging does
// not wait for the workgroup's sum of squares, whose wave sums ride the
// staging's barrier; otherwise the digits are those of (x * scale) * w, and
// 1 is returned, as it is without RMSNorm.
template <int NW, bool kFour = false, bool kDeferNorm = false, typename Prefetch>
__device__ __forceinline__ float StageDigits(const Hdr& a, XChunks<NW>& xc, uint8_t* lds, double* redd,
                                             Prefetch prefetch) {
  constexpr int NT = XChunks<NW>::NT, NC = XChunks<NW>::NC, NNC = XChunks<NW>::NNC;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K, n8 = K >> 3, nc = xc.nc;
  auto& v = xc.v;
  auto& wv = xc.wv;
  prefetch();
  const bool norm = a.norm_w != nullptr;
  if (norm) {
    double s2 = 0.0;
#pragma unroll
    for (int c = 0; c < NNC; ++c)
      if (tid + c * NT < n8)
#pragma unroll
        for (int i = 0; i < 8; ++i) s2 += static_cast<double>(v[c][i]) * v[c][i];
    s2 = WaveSumD(s2);
    if (lane == 0) redd[wave] = s2;
    if constexpr (kDeferNorm) {
#pragma unroll
      for (int c = 0; c < NNC; ++c)
        if (c < nc)
#pragma unroll
          for (int i = 0; i < 8; ++i) v[c][i] = __fmul_rn(v[c][i], wv[c][i]);
    } else {
      LdsBarrier();
      double total = 0.0;
#pragma unroll
      for (int w = 0; w < NW; ++w) total += redd[w];
      const float scale =
          static_cast<float>(1.0 / __builtin_sqrt(total / static_cast<double>(K) + static_cast<double>(a.eps)));
#pragma unroll
      for (int c = 0; c < NNC; ++c)
        if (c < nc)
#pragma unroll
          for (int i = 0; i < 8; ++i) v[c][i] = __fmul_rn(__fmul_rn(v[c][i], scale), wv[c][i]);
    }
  }
  U4* zero = reinterpret_cast<U4*>(lds + a.zero_off);
  for (int i = tid; i < kZeroBytes / 16; i += NT) zero[i] = U4{0u, 0u, 0u, 0u};
  float2* xg = reinterpret_cast<float2*>(lds + a.xg_off);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c >= nc) break;
    const int ch = tid + c * NT;  // chunks 2G and 2G + 1 of group G sit on adjacent lanes
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[c][i]));
    m = fmaxf(m, __uint_as_float(Dpp<kQuadXor1>(__float_as_uint(m))));
    const int eb = static_cast<int>(__float_as_uint(m) >> 23);
    if constexpr (kFour) {
      // s = 2^(30 - E): |x * s| < 2^30, x_fix = rint(x * s) as an integer;
      // u = x_fix + 0x80808080 holds the four signed-byte digits, each offset
      // by 128, as its bytes (no wrap for |x_fix| < 2^30)
      const int se = m > 0.0f ? min(max(156 - eb, -100), 126) : 0;
      const float s = __uint_as_float(static_cast<uint32_t>(se + 127) << 23);
      uint32_t u[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) u[i] = static_cast<uint32_t>(__float2int_rn(v[c][i] * s)) + 0x80808080u;
      if (ch < n8) {
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
        uint2* rec = reinterpret_cast<uint2*>(lds) + (ch >> 1) * 8 + (ch & 1);
        rec[0] = make_uint2(row[0][0], row[0][1]);
        rec[2] = make_uint2(row[1][0], row[1][1]);
        rec[4] = make_uint2(row[2][0], row[2][1]);
        rec[6] = make_uint2(row[3][0], row[3][1]);
        if ((ch & 1) == 0) xg[ch >> 1] = make_float2(__uint_as_float(static_cast<uint32_t>(127 - se) << 23), 0.0f);
      }
      continue;
    }
    // s = 2^(22 - E) for max = f * 2^E, f in [0.5, 1) (E = biased exponent -
    // 126 for normal max; a subnormal max takes the upper clamp): |x * s| < 2^22
    const int se = m > 0.0f ? min(max(148 - eb, -100), 126) : 0;
    const float s = __uint_as_float(static_cast<uint32_t>(se + 127) << 23);
    // x_fix = rint(x * s): x * s + 1.5 * 2^23 rounds at the units (ties to
    // even) and leaves 0x4B400000 + x_fix in the bits. u = x_fix + 0x808080
    // then holds the signed-byte digits of x_fix, each offset by 128, as its
    // bytes: x_fix = sum_k (byte_k(u) - 128) * 256^k.
    uint32_t u[8];
    int isum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u[i] = __float_as_uint(__builtin_fmaf(v[c][i], s, 12582912.0f)) + (0x808080u - 0x4B400000u);
      isum += static_cast<int>(u[i]);
    }
    isum -= 8 * 0x808080;
    isum += static_cast<int>(Dpp<kQuadXor1>(static_cast<uint32_t>(isum)));
    if (ch < n8) {
      // byte k of four values -> digit row k (v_perm_b32 byte transposes)
      uint32_t row[3][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t a1 = __builtin_amdgcn_perm(u[4 * h + 1], u[4 * h], 0x05010400u);  // v0.b0 v1.b0 v0.b1 v1.b1
        const uint32_t a2 = __builtin_amdgcn_perm(u[4 * h + 1], u[4 * h], 0x0C0C0602u);  // v0.b2 v1.b2
        const uint32_t b1 = __builtin_amdgcn_perm(u[4 * h + 3], u[4 * h + 2], 0x05010400u);
        const uint32_t b2 = __builtin_amdgcn_perm(u[4 * h + 3], u[4 * h + 2], 0x0C0C0602u);
        row[0][h] = __builtin_amdgcn_perm(b1, a1, 0x05040100u) ^ 0x80808080u;
        row[1][h] = __builtin_amdgcn_perm(b1, a1, 0x07060302u) ^ 0x80808080u;
        row[2][h] = __builtin_amdgcn_perm(b2, a2, 0x05040100u) ^ 0x80808080u;
      }
      uint2* rec = reinterpret_cast<uint2*>(lds) + (ch >> 1) * 8 + (ch & 1);  // 64-byte record of group ch / 2
      rec[0] = make_uint2(row[0][0], row[0][1]);
      rec[2] = make_uint2(row[1][0], row[1][1]);
      rec[4] = make_uint2(row[2][0], row[2][1]);
      rec[6] = make_uint2(0u, 0u);
      if ((ch & 1) == 0) {
        const float f = __uint_as_float(static_cast<uint32_t>(127 - se) << 23);
        xg[ch >> 1] = make_float2(f, static_cast<float>(isum) * f);
      }
    }
  }
  LdsBarrier();
  if (!kDeferNorm || !norm) return 1.0f;
  double total = 0.0;
#pragma unroll
  for (int w = 0; w < NW; ++w) total += redd[w];
  return static_cast<float>(1.0 / __builtin_sqrt(total / static_cast<double>(K) + static_cast<double>(a.eps)));
}

template <uint32_t T>
struct MUnit;

template <>
struct MUnit<kQ4_K> {
  static constexpr int kBytes = 144;
  U4 hdr, q0, q1;
  __device__ __forceinline__ void Load(const uint8_t* blk, int g, int) {
    hdr = GLoad<U4>(blk);
    q0 = GLoad<U4>(blk + 16 + 16 * g);
    q1 = GLoad<U4>(blk + 80 + 16 * g);
  }
  // tile-major: the lane's offsets in a 16-block chunk (its block, its quants)
  struct Off {
    uint32_t h, q;
  };
  __device__ static __forceinline__ Off MakeOff(int g, int col) {
    return {static_cast<uint32_t>(144 * col), static_cast<uint32_t>(144 * col + 16 * g)};
  }
  __device__ __forceinline__ void LoadT(Rsrc r, int chunk, const Off& o) {
    hdr = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.h), chunk, 0);
    q0 = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.q) + 16, chunk, 0);
    q1 = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.q) + 80, chunk, 0);
  }
  // first 16-group of the lane's windows within a super-block
  __device__ static __forceinline__ int GroupBase(int g) { return 4 * (g >> 1) + (g & 1); }
};

template <>
struct MUnit<kQ6_K> {
  static constexpr int kBytes = 210;
  U4 a, b, h;
  uint32_t a4, b4, h4, dw, sh;
  U3 s;
  __device__ __forceinline__ void Load(const uint8_t* blk, int g, int) {
    sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* p = blk - sh;
    const int hh = g >> 1, ls = g & 1;
    const int oa = 64 * hh + 16 * ls, oh = 128 + 32 * hh + 16 * ls;
    a = GLoad<U4A4>(p + oa);
    a4 = GLoad<uint32_t>(p + oa + 16);
    b = GLoad<U4A4>(p + oa + 32);
    b4 = GLoad<uint32_t>(p + oa + 48);
    h = GLoad<U4A4>(p + oh);
    h4 = GLoad<uint32_t>(p + oh + 16);
    s = GLoad<U3A4>(p + 192 + 8 * hh);
    dw = GLoad<uint32_t>(p + 208);
  }
  __device__ static __forceinline__ int GroupBase(int g) { return 8 * (g >> 1) + (g & 1); }
};

// Q6_K from a tile-major copy, whose chunk of 16 blocks (one super-block of a
// 16-row tile) holds the fields grouped: ql of the 16 rows (128 bytes each),
// then qh (64), scales (16) and d (2) -- every lane load aligned.
constexpr uint32_t kQ6T = 0x100u | kQ6_K;
constexpr int kQ6Ql = 0, kQ6Qh = 16 * 128, kQ6Sc = kQ6Qh + 16 * 64, kQ6D = kQ6Sc + 16 * 16;

template <>
struct MUnit<kQ6T> {
  static constexpr int kBytes = 210;
  U4 a, b, h;
  U2 s;
  uint32_t d;
  // the lane's offsets in the super-block's 16-block chunk (col: the lane's
  // row in the tile)
  struct Off {
    uint32_t ql, qh, s, d;
  };
  __device__ static __forceinline__ Off MakeOff(int g, int col) {
    const int hh = g >> 1, ls = g & 1;
    return {static_cast<uint32_t>(kQ6Ql + 128 * col + 64 * hh + 16 * ls),
            static_cast<uint32_t>(kQ6Qh + 64 * col + 32 * hh + 16 * ls),
            static_cast<uint32_t>(kQ6Sc + 16 * col + 8 * hh), static_cast<uint32_t>(kQ6D + 2 * col)};
  }
  __device__ __forceinline__ void LoadT(Rsrc r, int chunk, const Off& o) {
    a = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.ql), chunk, 0);
    b = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.ql) + 32, chunk, 0);
    h = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.qh), chunk, 0);
    s = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(o.s), chunk, 0);
    d = __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(o.d), chunk, 0);
  }
  __device__ static __forceinline__ int GroupBase(int g) { return MUnit<kQ6_K>::GroupBase(g); }
};

// Q8_0 from a tile-major copy. The chunk of one super-block of a 16-row tile
// (16 rows x 8 blocks of 34 bytes) holds the quants regrouped by MFMA, then
// the 16 rows' block scales: byte 1024 m + 64 j + 16 g + e is quant 16 (g % 2)
// + e of block 2 m + g / 2 of row j (weights 64 m + 16 g + e of the
// super-block), and bytes 4096 + 16 j + 2 b hold d of block b of row j. Lane
// (j, g) feeds one MFMA per m with the 16 raw quants (signed bytes, no
// unpacking) of its 16-group 4 m + g, and applies that block's d once per
// MFMA (reference src/quant.cc:132-142: w = d * q).
constexpr uint32_t kQ8T = 0x100u | kQ8_0;
constexpr int kQ8Sc = 4096;

template <>
struct MUnit<kQ8T> {
  static constexpr int kBytes = 272;  // 8 blocks of one row per super-block
  U4 q[4];
  U4 s;
  struct Off {
    uint32_t q, s;
  };
  __device__ static __forceinline__ Off MakeOff(int g, int col) {
    return {static_cast<uint32_t>(64 * col + 16 * g), static_cast<uint32_t>(kQ8Sc + 16 * col)};
  }
  __device__ __forceinline__ void LoadT(Rsrc r, int chunk, const Off& o) {
#pragma unroll
    for (int m = 0; m < 4; ++m) q[m] = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.q) + 1024 * m, chunk, 0);
    s = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(o.s), chunk, 0);
  }
  __device__ static __forceinline__ int GroupBase(int g) { return g; }
};

// The empty asm keeps both sources live until the result exists, so the
// result can never be allocated over a source: an MFMA whose destination
// aliases its A or B registers returned wrong sums on gfx950 (measured; the
// compiler allows the aliasing when a source dies at the MFMA).
__device__ __forceinline__ I4 MfmaI8(U4 a, U4 b) {
  const I4 z = {0, 0, 0, 0};
  const I4 r = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(I4, a), __builtin_bit_cast(I4, b), z, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(r));
  return r;
}

// sum(q * x_fix) from the three digit sums (C1 + 2^8 C2 is exact in int32)
__device__ __forceinline__ float DigitSum(I4 c) {
  const int t = c[1] + c[2] * 256;
  return __builtin_fmaf(static_cast<float>(t), 256.0f, static_cast<float>(c[0]));
}

__device__ __forceinline__ U4 LdsU4(const uint8_t* p) { return *reinterpret_cast<const U4*>(p); }

// Lane (j, g)'s contribution from one super-block. ap: this lane's digit row
// of the super-block's first group of its windows (or the zero region), xg:
// the same group's (f, sum x).
__device__ __forceinline__ float UnitDot(const MUnit<kQ4_K>& u, const uint8_t* ap, const float2* xg, int g) {
  const float d = dev::HalfToFloatFast(u.hdr.x & 0xFFFFu);
  const float dmin = dev::HalfToFloatFast(u.hdr.x >> 16);
  // scales / mins of sub-blocks a, a + 1 (window 0) and a + 4, a + 5
  // (window 1), a = 2 * (g / 2) (reference src/quant.cc:159-167)
  const uint32_t sft = 16u * static_cast<uint32_t>(g >> 1);
  const uint32_t Y = u.hdr.y >> sft, Z = u.hdr.z >> sft, W = u.hdr.w >> sft;
  const uint32_t scp[2] = {Y & 0x3F3Fu, (W & 0x0F0Fu) | ((Y >> 2) & 0x3030u)};
  const uint32_t mp[2] = {Z & 0x3F3Fu, ((W >> 4) & 0x0F0Fu) | ((Z >> 2) & 0x3030u)};
  float r = 0.0f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const U4 q = c ? u.q1 : u.q0;
    const U4 lo = {q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu};
    const U4 hi = {(q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                   (q.w >> 4) & 0x0F0F0F0Fu};
    const I4 cl = MfmaI8(LdsU4(ap + (8 * c) * 64), lo);
    const I4 ch = MfmaI8(LdsU4(ap + (8 * c + 2) * 64), hi);
    const float2 gl = xg[8 * c], gh = xg[8 * c + 2];
    r = __builtin_fmaf((d * CvtU8<0>(scp[c])) * gl.x, DigitSum(cl), r);
    r = __builtin_fmaf(-(dmin * CvtU8<0>(mp[c])), gl.y, r);
    r = __builtin_fmaf((d * CvtU8<1>(scp[c])) * gh.x, DigitSum(ch), r);
    r = __builtin_fmaf(-(dmin * CvtU8<1>(mp[c])), gh.y, r);
  }
  return r;
}

// Lane (j, g)'s Q6_K contribution from the lane's aligned words: wa, wb the
// ql words of windows 0 and 1, hq the qh words, s0 / s1 scales 8h .. 8h + 3 /
// 8h + 4 .. 8h + 7, d the block scale.
__device__ __forceinline__ float Q6Dot(const uint32_t (&wa)[4], const uint32_t (&wb)[4], const uint32_t (&hq)[4],
                                       uint32_t s0, uint32_t s1, float d, const uint8_t* ap, const float2* xg, int g) {
  const int ls = g & 1;
  float r = 0.0f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const uint32_t(&w)[4] = c ? wb : wa;
    U4 lo, hi;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t hc = c ? hq[t] >> 2 : hq[t];  // the low slot's 2 bits at 0-1, the high slot's at 4-5
      lo[t] = (w[t] & 0x0F0F0F0Fu) | ((hc << 4) & 0x30303030u);
      hi[t] = ((w[t] >> 4) & 0x0F0F0F0Fu) | (hc & 0x30303030u);
    }
    const I4 cl = MfmaI8(LdsU4(ap + (2 * c) * 64), lo);
    const I4 ch = MfmaI8(LdsU4(ap + (2 * c + 4) * 64), hi);
    const float2 gl = xg[2 * c], gh = xg[2 * c + 4];
    const float sc_lo = static_cast<float>(__builtin_amdgcn_sbfe(s0, 8 * (2 * c + ls), 8));
    const float sc_hi = static_cast<float>(__builtin_amdgcn_sbfe(s1, 8 * (2 * c + ls), 8));
    r = __builtin_fmaf((d * sc_lo) * gl.x, DigitSum(cl), r);
    r = __builtin_fmaf(-(32.0f * d * sc_lo), gl.y, r);
    r = __builtin_fmaf((d * sc_hi) * gh.x, DigitSum(ch), r);
    r = __builtin_fmaf(-(32.0f * d * sc_hi), gh.y, r);
  }
  return r;
}

// row-major blocks: the words realigned from the 4-byte-aligned loads
__device__ __forceinline__ float UnitDot(const MUnit<kQ6_K>& u, const uint8_t* ap, const float2* xg, int g) {
  const uint32_t sh = u.sh;
  const float d = dev::HalfToFloatFast((u.dw >> (8u * sh)) & 0xFFFFu);
  const uint32_t s0 = __builtin_amdgcn_alignbyte(u.s.y, u.s.x, sh);
  const uint32_t s1 = __builtin_amdgcn_alignbyte(u.s.z, u.s.y, sh);
  const uint32_t hq[4] = {__builtin_amdgcn_alignbyte(u.h.y, u.h.x, sh), __builtin_amdgcn_alignbyte(u.h.z, u.h.y, sh),
                          __builtin_amdgcn_alignbyte(u.h.w, u.h.z, sh), __builtin_amdgcn_alignbyte(u.h4, u.h.w, sh)};
  const uint32_t wa[4] = {__builtin_amdgcn_alignbyte(u.a.y, u.a.x, sh), __builtin_amdgcn_alignbyte(u.a.z, u.a.y, sh),
                          __builtin_amdgcn_alignbyte(u.a.w, u.a.z, sh), __builtin_amdgcn_alignbyte(u.a4, u.a.w, sh)};
  const uint32_t wb[4] = {__builtin_amdgcn_alignbyte(u.b.y, u.b.x, sh), __builtin_amdgcn_alignbyte(u.b.z, u.b.y, sh),
                          __builtin_amdgcn_alignbyte(u.b.w, u.b.z, sh), __builtin_amdgcn_alignbyte(u.b4, u.b.w, sh)};
  return Q6Dot(wa, wb, hq, s0, s1, d, ap, xg, g);
}

__device__ __forceinline__ float UnitDot(const MUnit<kQ6T>& u, const uint8_t* ap, const float2* xg, int g) {
  const uint32_t wa[4] = {u.a.x, u.a.y, u.a.z, u.a.w}, wb[4] = {u.b.x, u.b.y, u.b.z, u.b.w};
  const uint32_t hq[4] = {u.h.x, u.h.y, u.h.z, u.h.w};
  return Q6Dot(wa, wb, hq, u.s.x, u.s.y, dev::HalfToFloatFast(u.d & 0xFFFFu), ap, xg, g);
}

// Lane (j, g)'s Q8_0 contribution from one super-block: 16-groups 4 m + g,
// block scale d of block 2 m + g / 2.
__device__ __forceinline__ float UnitDot(const MUnit<kQ8T>& u, const uint8_t* ap, const float2* xg, int g) {
  const uint32_t sh = 16u * static_cast<uint32_t>(g >> 1);
  const uint32_t sw[4] = {u.s.x, u.s.y, u.s.z, u.s.w};
  float r = 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const I4 c = MfmaI8(LdsU4(ap + (4 * m) * 64), u.q[m]);
    // sum(q * x_fix) = C0 + 2^8 C1 + 2^16 C2 + 2^24 C3, exact in double
    // (|C| <= 16 * 128 * 128), one rounding to float
    const double t = static_cast<double>(c[1] + 256 * c[2]);
    const float sum = static_cast<float>(__builtin_fma(static_cast<double>(c[3]), 16777216.0,
                                                       __builtin_fma(t, 256.0, static_cast<double>(c[0]))));
    const float d = dev::HalfToFloatFast((sw[m] >> sh) & 0xFFFFu);
    r = __builtin_fmaf(d * xg[4 * m].x, sum, r);
  }
  return r;
}

}  // namespace mfma
}  // namespace k
}  // namespace rpg

#endif  // RPG_HIP_MFMA_DOT_H_
