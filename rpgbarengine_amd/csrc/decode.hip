// Decode-step (one token) kernels for gfx950.
//
// Matvec: each wave owns a tile of VR "virtual rows" (VR rows of one matrix,
// or VR/2 rows of each matrix of a SwiGLU pair). Lane l works on virtual row
// l % VR and on the 32-weight units u = l / VR, l / VR + 64 / VR, ... of that
// row (quant_dev.h describes the units), so the VR lanes that read one unit of
// the input share it through an LDS broadcast, and a row's partial sums meet
// in a log2(64 / VR)-step shuffle reduction. The workgroup's prologue stages
// the input vector in LDS -- RMS-normalised on the fly for the projections
// that consume a norm (reference src/qwen3.cc:131-134,191-194,284-287) -- with
// sums of each 8 consecutive values; after that the waves never synchronise.
// Per unit the dot product is formed on the raw quants and scaled once:
//   Q4_K  (d*sc)*sum(q*x) - (dmin*m)*sum(x) per 16-weight half-unit
//   Q6_K  (d*sc)*sum((q-32)*x) per 8 weights
//   Q8_0  d*sum(q*x)
// which is the reference's dot (reference src/matmul.cc:73-102,
// src/matmul_avx2.cc:95-289) up to summation order -- dots are judged by the
// max|d|/sum|a*w| <= 1e-6 bound, not bitwise.
//
// Attention: QK-norm + RoPE of the query heads (and of the new key), KV-cache
// write and the split-K partial run in one kernel; a small combine kernel
// rescales the partials.

#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"
#include "decode.h"
#include "expf_glibc.h"
#include "lanes.h"
#include "soft_exp.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kHd = 128;

using lanes::WaveMaxF;
using lanes::WaveSumD;
using lanes::WaveSumF;

// Weight loads through global-address-space pointers: the row pointers come
// out of the job table, where the compiler cannot prove them global, and a
// generic (flat) load would also hold up every LDS wait behind it.
typedef uint32_t U32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t U32x2 __attribute__((ext_vector_type(2)));
typedef float F4 __attribute__((ext_vector_type(4)));
typedef float F2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ T GLoad(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}
__device__ __forceinline__ uint4 GLoad16(const uint8_t* p) {
  const U32x4 v = GLoad<U32x4>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t GLoadU16(const uint8_t* p) { return GLoad<uint16_t>(p); }
// 8 bytes from an address that is only 2-byte aligned (Q6_K and Q8_0 blocks
// are 210 and 34 bytes long): one dwordx2 load, which global memory serves
// at any byte alignment.
typedef U32x2 U32x2A2 __attribute__((aligned(2)));
__device__ __forceinline__ uint2 GLoad8U(const uint8_t* p) {
  const U32x2 v = GLoad<U32x2A2>(p);
  return make_uint2(v.x, v.y);
}

// float(byte I of w) in one instruction (the compiler otherwise extracts the
// byte first).
template <int I>
__device__ __forceinline__ float CvtU8(uint32_t w) {
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

// ---------------------------------------------------------------- units

// Load(row, u) fetches the raw bytes of unit u of a row; Dot(u, xs, xs8)
// returns its dot product with the staged input (xs8[i] = sum of xs[8i..8i+8)).
template <uint32_t T>
struct Unit;

// Per-lane constants of a unit position i within its block (i = u % units
// per block), computed once per tile; a unit is then addressed by its block
// pointer and the block's first staged input.
template <>
struct Unit<12> {  // Q4_K: block header + 16 quant bytes (i = 2g + h)
  static constexpr int kBatch = 4;
  static constexpr int kPerBlock = 8, kBlockBytes = 144;
  struct Lane {
    int qoff, xoff;                // quant byte offset, first low-nibble input
    uint32_t sel_lo, sel_hi;       // sub-block 2g / 2g+1 scale field selectors
  };
  // sc/m of sub-block j from the 12 scale bytes (reference
  // src/quant.cc:159-167), branch-free for a lane-constant j: for j < 4 the
  // 6-bit fields of bytes j (sc) and 4 + j (m); for j >= 4 the nibbles of byte
  // 8 + (j-4) plus the top 2 bits of bytes j-4 and 4 + (j-4).
  __device__ static __forceinline__ uint32_t Selector(int j) {
    return j < 4 ? static_cast<uint32_t>(8 * j) : (0x80u | static_cast<uint32_t>(8 * (j - 4)));
  }
  __device__ static __forceinline__ Lane MakeLane(int i) {
    const int g = i >> 1, h = i & 1;
    return Lane{16 + 32 * g + 16 * h, 64 * g + 16 * h, Selector(2 * g), Selector(2 * g + 1)};
  }
  uint4 hdr, q;
  __device__ __forceinline__ void Load(const uint8_t* blk, const Lane& L) {
    hdr = GLoad16(blk);
    q = GLoad16(blk + L.qoff);
  }
  __device__ static __forceinline__ void ScaleMin(uint32_t sel, uint32_t s0, uint32_t s1, uint32_t s2, float* sc,
                                                  float* mn) {
    const uint32_t sh = sel & 31u;
    const bool hi = sel & 0x80u;
    const uint32_t a = hi ? s2 : s0, b = hi ? s2 : s1;
    const uint32_t wa = hi ? 4u : 6u;
    const uint32_t top_s = hi ? __builtin_amdgcn_ubfe(s0, sh + 6, 2) : 0u;
    const uint32_t top_m = hi ? __builtin_amdgcn_ubfe(s1, sh + 6, 2) : 0u;
    *sc = static_cast<float>(__builtin_amdgcn_ubfe(a, sh, wa) | (top_s << 4));
    *mn = static_cast<float>(__builtin_amdgcn_ubfe(b, hi ? sh + 4 : sh, wa) | (top_m << 4));
  }
  __device__ __forceinline__ float Dot(const Lane& L, const float* xb, const float* x8b) const {
    const float4* xl = reinterpret_cast<const float4*>(xb + L.xoff);
    const float4* xh = xl + 8;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    float l0 = 0.f, l1 = 0.f, h0 = 0.f, h1 = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t lo = qw[c] & 0x0F0F0F0Fu, hi = (qw[c] >> 4) & 0x0F0F0F0Fu;
      const float4 a = xl[c], e = xh[c];
      l0 = __builtin_fmaf(a.x, CvtU8<0>(lo), l0);
      l1 = __builtin_fmaf(a.y, CvtU8<1>(lo), l1);
      l0 = __builtin_fmaf(a.z, CvtU8<2>(lo), l0);
      l1 = __builtin_fmaf(a.w, CvtU8<3>(lo), l1);
      h0 = __builtin_fmaf(e.x, CvtU8<0>(hi), h0);
      h1 = __builtin_fmaf(e.y, CvtU8<1>(hi), h1);
      h0 = __builtin_fmaf(e.z, CvtU8<2>(hi), h0);
      h1 = __builtin_fmaf(e.w, CvtU8<3>(hi), h1);
    }
    const float2 sl = *reinterpret_cast<const float2*>(x8b + (L.xoff >> 3));
    const float2 sh = *reinterpret_cast<const float2*>(x8b + (L.xoff >> 3) + 4);
    const float d = dev::HalfToFloatFast(hdr.x & 0xFFFFu);
    const float dmin = dev::HalfToFloatFast(hdr.x >> 16);
    float scl, mnl, sch, mnh;
    ScaleMin(L.sel_lo, hdr.y, hdr.z, hdr.w, &scl, &mnl);
    ScaleMin(L.sel_hi, hdr.y, hdr.z, hdr.w, &sch, &mnh);
    const float r = __builtin_fmaf(d * scl, l0 + l1, -(dmin * mnl) * (sl.x + sl.y));
    return r + __builtin_fmaf(d * sch, h0 + h1, -(dmin * mnh) * (sh.x + sh.y));
  }
};

template <>
struct Unit<14> {  // Q6_K: (half, j) with i = 4*half + j: ql/qh bytes for l = 8j..8j+7
  static constexpr int kBatch = 4;
  static constexpr int kPerBlock = 8, kBlockBytes = 210;
  struct Lane {
    int lo_off, qh_off, sc_off, xoff, si;
  };
  __device__ static __forceinline__ Lane MakeLane(int i) {
    const int half = i >> 2, j = i & 3;
    return Lane{64 * half + 8 * j, 128 + 32 * half + 8 * j, 192 + 8 * half, 128 * half + 8 * j, j >> 1};
  }
  uint2 l0, l1, hh, s;
  uint32_t dbits;
  __device__ __forceinline__ void Load(const uint8_t* blk, const Lane& L) {
    l0 = GLoad8U(blk + L.lo_off);
    l1 = GLoad8U(blk + L.lo_off + 32);
    hh = GLoad8U(blk + L.qh_off);
    s = GLoad8U(blk + L.sc_off);  // sc[8*half .. +8)
    dbits = GLoadU16(blk + 208);
  }
  // sum over the four 32-apart groups m of (d*sc_m) * sum((q - 32) * x), with
  // sum(q*x) on the unsigned 6-bit quants and 32 * sum(x) from the staged
  // 8-sums
  __device__ __forceinline__ float Dot(const Lane& L, const float* xb, const float* x8b) const {
    const float* base = xb + L.xoff;
    float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t a = w ? l0.y : l0.x, c = w ? l1.y : l1.x, h = w ? hh.y : hh.x;
      const uint32_t qm[4] = {(a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u),
                              (c & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u),
                              ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u),
                              ((c >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u)};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float4 x = *reinterpret_cast<const float4*>(base + 32 * m + 4 * w);
        t[m] = __builtin_fmaf(x.x, CvtU8<0>(qm[m]), t[m]);
        t[m] = __builtin_fmaf(x.y, CvtU8<1>(qm[m]), t[m]);
        t[m] = __builtin_fmaf(x.z, CvtU8<2>(qm[m]), t[m]);
        t[m] = __builtin_fmaf(x.w, CvtU8<3>(qm[m]), t[m]);
      }
    }
    // the four int8 scales sc[si + 2m]: bytes si, si+2 of s.x and of s.y
    const uint32_t sx = s.x >> (8 * L.si), sy = s.y >> (8 * L.si);
    const int8_t scm[4] = {static_cast<int8_t>(sx & 0xFFu), static_cast<int8_t>((sx >> 16) & 0xFFu),
                           static_cast<int8_t>(sy & 0xFFu), static_cast<int8_t>((sy >> 16) & 0xFFu)};
    const float d = dev::HalfToFloatFast(dbits);
    float r = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float xsum = x8b[(L.xoff >> 3) + 4 * m];
      r = __builtin_fmaf(d * static_cast<float>(scm[m]), __builtin_fmaf(-32.0f, xsum, t[m]), r);
    }
    return r;
  }
};

template <>
struct Unit<8> {  // Q8_0: d + 32 int8 (2-byte aligned), one unit per block
  static constexpr int kBatch = 4;
  static constexpr int kPerBlock = 1, kBlockBytes = 34;
  struct Lane {};
  __device__ static __forceinline__ Lane MakeLane(int) { return Lane{}; }
  uint2 q[4];
  uint32_t dbits;
  __device__ __forceinline__ void Load(const uint8_t* blk, const Lane&) {
    dbits = GLoadU16(blk);
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = GLoad8U(blk + 2 + 8 * c);
  }
  // q exactly: float(q ^ 0x80) - 128 (an offset sum -128 * sum(x) would
  // cancel against a large input and lose the row bound)
  __device__ __forceinline__ float Dot(const Lane&, const float* xb, const float*) const {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 x0 = *reinterpret_cast<const float4*>(xb + 8 * c);
      const float4 x1 = *reinterpret_cast<const float4*>(xb + 8 * c + 4);
      const uint32_t u0 = q[c].x ^ 0x80808080u, u1 = q[c].y ^ 0x80808080u;
      a0 = __builtin_fmaf(x0.x, CvtU8<0>(u0) - 128.0f, a0);
      a1 = __builtin_fmaf(x0.y, CvtU8<1>(u0) - 128.0f, a1);
      a0 = __builtin_fmaf(x0.z, CvtU8<2>(u0) - 128.0f, a0);
      a1 = __builtin_fmaf(x0.w, CvtU8<3>(u0) - 128.0f, a1);
      a0 = __builtin_fmaf(x1.x, CvtU8<0>(u1) - 128.0f, a0);
      a1 = __builtin_fmaf(x1.y, CvtU8<1>(u1) - 128.0f, a1);
      a0 = __builtin_fmaf(x1.z, CvtU8<2>(u1) - 128.0f, a0);
      a1 = __builtin_fmaf(x1.w, CvtU8<3>(u1) - 128.0f, a1);
    }
    return dev::HalfToFloatFast(dbits) * (a0 + a1);
  }
};

template <>
struct Unit<0> {  // F32: 32 consecutive floats, one unit per "block"
  static constexpr int kBatch = 1;
  static constexpr int kPerBlock = 1, kBlockBytes = 128;
  struct Lane {};
  __device__ static __forceinline__ Lane MakeLane(int) { return Lane{}; }
  float4 v[8];
  __device__ __forceinline__ void Load(const uint8_t* blk, const Lane&) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint4 w = GLoad16(blk + 16 * c);
      v[c] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
    }
  }
  __device__ __forceinline__ float Dot(const Lane&, const float* xb, const float*) const {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float4 x = *reinterpret_cast<const float4*>(xb + 4 * c);
      a0 = __builtin_fmaf(x.x, v[c].x, a0);
      a1 = __builtin_fmaf(x.y, v[c].y, a1);
      a0 = __builtin_fmaf(x.z, v[c].z, a0);
      a1 = __builtin_fmaf(x.w, v[c].w, a1);
    }
    return a0 + a1;
  }
};

// ---------------------------------------------------------------- prologue

// Workgroup barrier that orders LDS only: outstanding global loads (the
// weight prefetch) stay in flight across it.
__device__ __forceinline__ void LdsBarrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float Sum8(const float4& a, const float4& b) {
  return ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
}

constexpr int kNormChunks = 2;   // 8-value chunks per thread with RMSNorm (K <= 4096)
static_assert(8 * kNormChunks * kThreads >= kDecodeNormMaxK, "the wave kernels' normed staging");
constexpr int kCopyChunks = 5;   // per round without (one round up to K = 10240)

// xs[0..K) = x, or RMSNorm(x) * w when norm_w != nullptr (double sum of
// squares, float scale, (x * scale) * w); xs8[i] = sum of xs[8i..8i+8).
// Thread t owns the 8-value chunks t, t + 256, ...; all loads of a round are
// issued before any is used. prefetch() runs right after the first round's
// loads are issued: loads complete in issue order, so requests made there
// must not delay the input.
template <typename Prefetch>
__device__ __forceinline__ void StageVector(float* xs, float* xs8, const float* __restrict__ x, int K,
                                            const float* __restrict__ norm_w, float eps, double* red,
                                            Prefetch prefetch) {
  const int tid = threadIdx.x;
  const int n8 = K >> 3;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  // Loads are unconditional (indices clamped into range) so that no branch
  // sits between them and their use.
  if (norm_w == nullptr) {
    float4 a[kCopyChunks], b[kCopyChunks];
#pragma unroll
    for (int c = 0; c < kCopyChunks; ++c) {
      const int ch = min(tid + c * kThreads, n8 - 1);
      a[c] = x4[2 * ch];
      b[c] = x4[2 * ch + 1];
    }
    prefetch();
#pragma unroll
    for (int c = 0; c < kCopyChunks; ++c) {
      const int ch = tid + c * kThreads;
      if (ch < n8) {
        xs4[2 * ch] = a[c];
        xs4[2 * ch + 1] = b[c];
        xs8[ch] = Sum8(a[c], b[c]);
      }
    }
    for (int ch = tid + kThreads * kCopyChunks; ch < n8; ch += kThreads) {  // K > 10240 only
      const float4 p = x4[2 * ch], q = x4[2 * ch + 1];
      xs4[2 * ch] = p;
      xs4[2 * ch + 1] = q;
      xs8[ch] = Sum8(p, q);
    }
  } else {
    const float4* w4 = reinterpret_cast<const float4*>(norm_w);
    float4 a[kNormChunks], b[kNormChunks], wa[kNormChunks], wb[kNormChunks];
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
      const int ch = min(tid + c * kThreads, n8 - 1);
      a[c] = x4[2 * ch];
      b[c] = x4[2 * ch + 1];
      wa[c] = w4[2 * ch];
      wb[c] = w4[2 * ch + 1];
    }
    prefetch();
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
      if (tid + c * kThreads < n8) {
        const float v[8] = {a[c].x, a[c].y, a[c].z, a[c].w, b[c].x, b[c].y, b[c].z, b[c].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) s += static_cast<double>(v[i]) * v[i];
      }
    }
    s = WaveSumD(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    LdsBarrier();
    const double total = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale =
        static_cast<float>(1.0 / __builtin_sqrt(total / static_cast<double>(K) + static_cast<double>(eps)));
    auto nrm = [scale](float4 v, float4 w) {
      return make_float4(__fmul_rn(__fmul_rn(v.x, scale), w.x), __fmul_rn(__fmul_rn(v.y, scale), w.y),
                         __fmul_rn(__fmul_rn(v.z, scale), w.z), __fmul_rn(__fmul_rn(v.w, scale), w.w));
    };
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
      const int ch = tid + c * kThreads;
      if (ch < n8) {
        const float4 na = nrm(a[c], wa[c]), nb = nrm(b[c], wb[c]);
        xs4[2 * ch] = na;
        xs4[2 * ch + 1] = nb;
        xs8[ch] = Sum8(na, nb);
      }
    }
  }
  LdsBarrier();
}

// One wave, one tile of J: VR virtual rows starting at real row t * R. The
// first batch of weight units is requested before the input is staged (every
// wave of the workgroup stages, active or not).
template <uint32_t T>
__device__ __forceinline__ void WaveTile(const DecodeJob& J, int t, bool active, const DecodeMatvecArgs& a,
                                         float* xs, float* xs8, double* red) {
  const int K = a.K;
  const int lane = threadIdx.x & 63;
  const int VR = J.rows_per_tile;  // 1, 2, 4 or 8
  const bool pair = J.w2 != nullptr;
  const int R = pair ? VR >> 1 : VR;
  const int vr = lane & (VR - 1);
  const bool second = pair && vr >= R;
  const int row = t * R + (second ? vr - R : vr);
  const bool valid = active && row < J.rows;
  const uint8_t* wrow = (second ? J.w2 : J.w) + static_cast<int64_t>(valid ? row : 0) * J.row_bytes;
  const int U = K >> 5;
  const int stride = 64 / VR;  // a multiple of 8, so every unit of a lane has the same position in its block
  constexpr int kB = Unit<T>::kBatch;
  constexpr int P = Unit<T>::kPerBlock, BB = Unit<T>::kBlockBytes;
  const int u0 = lane / VR;
  const typename Unit<T>::Lane L = Unit<T>::MakeLane(u0 % P);
  const int nblk = U / P, b0 = u0 / P, bstep = stride / P;
  // every lane runs the same number of batches; loads use block indices
  // clamped into the row (no branch between a load and its use) and the
  // dots of units past the row end are discarded
  const int nb = ((U + stride - 1) / stride + kB - 1) / kB;
  auto blk = [&](int k) { return min(b0 + k * bstep, nblk - 1); };
  // two register sets, alternating, so that no set is copied while its
  // loads are in flight
  Unit<T> ua[kB], ub[kB];
  auto load = [&](Unit<T>* u, int i) {
#pragma unroll
    for (int b = 0; b < kB; ++b) u[b].Load(wrow + BB * blk(i * kB + b), L);
  };
  float acc = 0.f;
  auto dot = [&](const Unit<T>* u, int i) {
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int k = i * kB + b;
      const int bi = blk(k);
      const float d = u[b].Dot(L, xs + 32 * P * bi, xs8 + 4 * P * bi);
      acc += (valid && b0 + k * bstep < nblk) ? d : 0.0f;
    }
  };
  StageVector(xs, xs8, a.x, K, a.norm_w, a.eps, red, [&]() { load(ua, 0); });
  if (!active) return;
  for (int i = 0; i < nb; i += 2) {
    load(ub, i + 1);
    dot(ua, i);
    if (i + 1 >= nb) break;
    load(ua, i + 2);
    dot(ub, i + 1);
  }
  for (int off = VR; off < 64; off <<= 1) acc += __shfl_xor(acc, off, 64);
  if (pair) {
    const float up = __shfl(acc, (lane + R) & 63, 64);
    if (lane < R && valid) {
      // silu(g) * up with glibc-exact expf (reference src/kernels.h:82-92)
      const float sg = acc / __fadd_rn(1.0f, GlibcExpf(-acc));
      J.y[row] = __fmul_rn(sg, up);
    }
  } else if (lane < VR && valid) {
    float* y = J.y + row;
    *y = a.epi == kAdd ? *y + acc : acc;
  }
}

// A tile of the other ggml types (quant_dev.h DequantUnit: exact weights,
// any type, read at run time; a SwiGLU pair's matrices may differ): the
// same staging, lane layout, reduction and epilogues as WaveTile.
__device__ __forceinline__ void WaveTileAny(const DecodeJob& J, int t, bool active, const DecodeMatvecArgs& a,
                                            float* xs, float* xs8, double* red) {
  const int K = a.K;
  const int lane = threadIdx.x & 63;
  const int VR = J.rows_per_tile;
  const bool pair = J.w2 != nullptr;
  const int R = pair ? VR >> 1 : VR;
  const int vr = lane & (VR - 1);
  const bool second = pair && vr >= R;
  const int row = t * R + (second ? vr - R : vr);
  const bool valid = active && row < J.rows;
  const uint32_t type = second ? J.type2 : J.type;
  const int64_t rb = second ? J.row_bytes2 : J.row_bytes;
  const uint8_t* wrow = (second ? J.w2 : J.w) + static_cast<int64_t>(valid ? row : 0) * rb;
  StageVector(xs, xs8, a.x, K, a.norm_w, a.eps, red, []() {});
  if (!active) return;
  float acc = 0.f;
  if (valid) {
    for (int u = lane / VR; u < (K >> 5); u += 64 / VR) {
      float w[32];
      dev::DequantUnit(type, wrow, u, w);
      const float4* xb = reinterpret_cast<const float4*>(xs + 32 * u);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float4 x = xb[c];
        acc = __builtin_fmaf(x.x, w[4 * c], acc);
        acc = __builtin_fmaf(x.y, w[4 * c + 1], acc);
        acc = __builtin_fmaf(x.z, w[4 * c + 2], acc);
        acc = __builtin_fmaf(x.w, w[4 * c + 3], acc);
      }
    }
  }
  for (int off = VR; off < 64; off <<= 1) acc += __shfl_xor(acc, off, 64);
  if (pair) {
    const float up = __shfl(acc, (lane + R) & 63, 64);
    if (lane < R && valid) {
      // silu(g) * up with glibc-exact expf (reference src/kernels.h:82-92)
      const float sg = acc / __fadd_rn(1.0f, GlibcExpf(-acc));
      J.y[row] = __fmul_rn(sg, up);
    }
  } else if (lane < VR && valid) {
    float* y = J.y + row;
    *y = a.epi == kAdd ? *y + acc : acc;
  }
}

__global__ __launch_bounds__(kThreads) void MatvecAnyWaveKernel(DecodeMatvecArgs a) {
  extern __shared__ float smem[];
  __shared__ double red[kWaves];
  int t = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kWaves + (threadIdx.x >> 6)), j = 0;
  while (j + 1 < a.n_jobs && t >= a.job[j].tiles) {
    t -= a.job[j].tiles;
    ++j;
  }
  const DecodeJob& J = a.job[j];
  WaveTileAny(J, t, t < J.tiles, a, smem, smem + a.K, red);
}

// All jobs of a launch have weight type TA or TB (a SwiGLU pair's two
// matrices share one type), so no runtime switch inflates register use.
template <uint32_t TA, uint32_t TB>
__global__ __launch_bounds__(kThreads) void MatvecWaveKernel(DecodeMatvecArgs a) {
  extern __shared__ float smem[];
  __shared__ double red[kWaves];
  float* xs = smem;
  float* xs8 = smem + a.K;
  // wave-uniform tile index, kept in scalar registers so the job table is
  // read with scalar loads
  int t = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kWaves + (threadIdx.x >> 6)), j = 0;
  while (j + 1 < a.n_jobs && t >= a.job[j].tiles) {
    t -= a.job[j].tiles;
    ++j;
  }
  const DecodeJob& J = a.job[j];
  const bool active = t < J.tiles;
  if (J.type == TA)
    WaveTile<TA>(J, t, active, a, xs, xs8, red);
  else
    WaveTile<TB>(J, t, active, a, xs, xs8, red);
}

__global__ void IncKernel(int32_t* c) { *c += 1; }

// ---------------------------------------------------------------- attention

// QK-norm + RoPE of one head vector held as lane pairs (i, i + 64), with
// the gains (w0, w1) and the rotation (c, sn) of lane i already loaded.
__device__ __forceinline__ void NormRopePair(float x0, float x1, float w0, float w1, float c, float sn, float eps,
                                             float* o0, float* o1) {
  double s = static_cast<double>(x0) * x0 + static_cast<double>(x1) * x1;
  s = WaveSumD(s);
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(s / static_cast<double>(kHd) + static_cast<double>(eps)));
  const float na = __fmul_rn(__fmul_rn(x0, scale), w0);
  const float nb = __fmul_rn(__fmul_rn(x1, scale), w1);
  *o0 = __fsub_rn(__fmul_rn(na, c), __fmul_rn(nb, sn));
  *o1 = __fadd_rn(__fmul_rn(nb, c), __fmul_rn(na, sn));
}

constexpr int kSplit = 32;           // cache positions per staged tile
constexpr int kSplitsPerHead = 32;   // splits per KV head at most: a split takes whole tiles
constexpr int kKStride = kHd + 4;    // padded K rows in LDS (spreads the banks)
constexpr int kPart = 2 + kHd;       // partial record: max, sum, 128 outputs

// Positions per split for a history of n_keys: whole 32-position tiles, as
// few as keep at most kSplitsPerHead splits (a history of up to 1024
// positions keeps one tile per split).
__device__ __host__ __forceinline__ int SplitSpan(int n_keys) {
  const int tiles = (n_keys + kSplit - 1) / kSplit;
  return kSplit * ((tiles + kSplitsPerHead - 1) / kSplitsPerHead);
}

// grid (n_kv, n_splits), G = n_heads / n_kv: the G query heads of KV head kh against cache
// positions [32 * split, +32) of 0..pos. The split holding `pos` also writes
// the new (normed, rotated) key and the value into the cache. Each workgroup
// leaves a flash-decoding partial (running max, sum of exp, unnormalised
// output) for AttnMergeKernel.
//
// Order of work: the position is read first, with the operands that do not
// depend on it (query and key rows, norm gains, the new value); a split past
// the position then leaves before it loads anything from the cache (the grid
// covers the session's capacity, so at short histories most splits are
// idle), and an active split loads its K/V rows -- only rows up to the
// position -- with the RoPE row. The QK-norm/RoPE jobs (query heads 0..G-1
// and the new key, job G, on waves jb % 4) run while the tile arrives. After
// one barrier each wave takes whole heads h = wave, wave + 4: scores,
// softmax and P.V with no further barrier.
__device__ __forceinline__ void AttnSplitBody(const DecodeAttnArgs& a, int n_splits, int G) {
  const int kh = blockIdx.x, split = blockIdx.y;
  // every argument in the first round trip
  const int64_t max_seq = lanes::Uniform(a.max_seq);
  const auto kcache = lanes::UniformGlobal(a.kcache);
  const auto vcache = lanes::UniformGlobal(a.vcache);
  const auto rope = lanes::UniformGlobal(a.rope);
  const auto work = lanes::UniformGlobal(a.work);
  const float eps = lanes::Uniform(a.eps);
  const auto pos_dev = reinterpret_cast<const int32_t*>(lanes::Uniform(reinterpret_cast<uintptr_t>(a.pos_dev)));
  const int pos = lanes::UniformRead(pos_dev);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  __shared__ __align__(16) float ks[kSplit][kKStride];
  __shared__ __align__(16) float vs[kSplit][kHd];
  __shared__ __align__(16) float qs[8][kHd];
  // 1. job operands, position independent: slot t holds job wave + 4t. The
  // loads are unconditional (a slot past G reads query head 0 and is not
  // used): loads under a branch join as register copies that wait for them.
  float x0[3], x1[3], w0[3], w1[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const int jb = wave + kWaves * t;
    const bool is_k = jb == G;
    const float* src = is_k ? a.k + kh * kHd : a.q + (kh * G + (jb < G ? jb : 0)) * kHd;
    const float* nw = is_k ? a.k_norm : a.q_norm;
    x0[t] = src[lane];
    x1[t] = src[lane + 64];
    w0[t] = nw[lane];
    w1[t] = nw[lane + 64];
  }
  const float nv0 = a.v[kh * kHd + lane], nv1 = a.v[kh * kHd + lane + 64];
  const int n_keys = pos + 1;
  const int s0 = split * kSplit;
  if (s0 >= n_keys) return;
  const int n = min(kSplit, n_keys - s0);
  const bool has_new = s0 + n == n_keys;  // this split holds position pos
  // 2. the K/V tile (row r, 4-float column idx & 31): rows s0 .. s0 + n - 1;
  // the slots past n read row s0 + n - 1 again (no bytes past the history)
  // and are replaced by zeros, and row n - 1 of the split holding pos by the
  // new row, both in LDS below. Native vectors: copies of HIP's float4 class
  // stay memcpys that keep the tile in scratch memory across the jobs.
  const auto kg = kcache + static_cast<int64_t>(kh) * max_seq * kHd;
  const auto vg = vcache + static_cast<int64_t>(kh) * max_seq * kHd;
  constexpr int kPer = kSplit * (kHd / 4) / kThreads;  // 4-float vectors per thread per tensor
  F4 kr[kPer], vr[kPer];
#pragma unroll
  for (int c = 0; c < kPer; ++c) {
    const int idx = tid + c * kThreads;
    const int64_t row = s0 + min(idx >> 5, n - 1);
    kr[c] = *reinterpret_cast<lanes::GlobalPtr<const F4>>(kg + row * kHd + 4 * (idx & 31));
    vr[c] = *reinterpret_cast<lanes::GlobalPtr<const F4>>(vg + row * kHd + 4 * (idx & 31));
  }
  const auto rope_row = rope + static_cast<int64_t>(pos) * kHd;
  const float rc = rope_row[lane], rs = rope_row[64 + lane];
  // 3. the jobs: slots 0 and 1 side by side (independent chains), slot 2
  // (G = 8, wave 0) after them
  float o0[3], o1[3];
  NormRopePair(x0[0], x1[0], w0[0], w1[0], rc, rs, eps, &o0[0], &o1[0]);
  NormRopePair(x0[1], x1[1], w0[1], w1[1], rc, rs, eps, &o0[1], &o1[1]);
  if (wave + 2 * kWaves <= G) NormRopePair(x0[2], x1[2], w0[2], w1[2], rc, rs, eps, &o0[2], &o1[2]);
  float nk0 = 0.f, nk1 = 0.f;
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const int jb = wave + kWaves * t;
    if (jb < G) {
      qs[jb][lane] = o0[t];
      qs[jb][lane + 64] = o1[t];
    } else if (jb == G) {
      nk0 = o0[t];
      nk1 = o1[t];
    }
  }
  const bool new_wave = has_new && wave == G % kWaves;
  if (new_wave) {
    const auto kd = kcache + (static_cast<int64_t>(kh) * max_seq + pos) * kHd;
    const auto vd = vcache + (static_cast<int64_t>(kh) * max_seq + pos) * kHd;
    kd[lane] = nk0;
    kd[lane + 64] = nk1;
    vd[lane] = nv0;
    vd[lane + 64] = nv1;
    ks[n - 1][lane] = nk0;
    ks[n - 1][lane + 64] = nk1;
    vs[n - 1][lane] = nv0;
    vs[n - 1][lane + 64] = nv1;
  }
  // 4. the tile into LDS (row n - 1 of a split holding pos is the new row;
  // rows from n on are zeros, so P.V can run over all 32 rows)
#pragma unroll
  for (int c = 0; c < kPer; ++c) {
    const int idx = tid + c * kThreads, r = idx >> 5, c4 = idx & 31;
    if (has_new && r == n - 1) continue;
    const F4 z = {0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<F4*>(&ks[r][4 * c4]) = r < n ? kr[c] : z;
    *reinterpret_cast<F4*>(&vs[r][4 * c4]) = r < n ? vr[c] : z;
  }
  __syncthreads();
  // 5. per head: lane (j = lane % 32, half = lane / 32) scores key j over
  // dims [64 half, +64); the halves add across lanes j and j + 32
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  const int j = lane & 31, half = lane >> 5;
  for (int h = wave; h < G; h += kWaves) {
    const F4* q4 = reinterpret_cast<const F4*>(&qs[h][64 * half]);
    const F4* k4 = reinterpret_cast<const F4*>(&ks[j][64 * half]);
    float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
    // four vectors per round: fully unrolled, the loads of all sixteen are
    // hoisted (162 VGPRs, three waves per SIMD); this way 116
#pragma unroll 4
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
    const auto w = work + (static_cast<int64_t>(kh * G + h) * n_splits + split) * kPart;
    if (lane == 0) {
      w[0] = m;
      w[1] = l;
    }
    // unnormalised P.V: lane takes dims 2 lane, 2 lane + 1; p_j from lane j
    // (rows from n on add p_j * 0 = +0 with p_j = 0: the sums are those
    // over j < n)
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kSplit; ++jj) {
      const float pj = lanes::ReadLaneF(p, jj);
      const F2 vv = *reinterpret_cast<const F2*>(&vs[jj][2 * lane]);
      acc0 = __builtin_fmaf(pj, vv.x, acc0);
      acc1 = __builtin_fmaf(pj, vv.y, acc1);
    }
    *reinterpret_cast<lanes::GlobalPtr<F2>>(w + 2 + 2 * lane) = F2{acc0, acc1};
  }
}

// AttnSplitBody for capacities past kSplitsPerHead tiles: grid (n_kv,
// kSplitsPerHead), the G query heads of KV head kh against cache positions
// [span * split, + span) of 0..pos (span = SplitSpan(pos + 1)), one
// 32-position tile at a time. The split holding
// `pos` also writes the new (normed, rotated) key and the value into the
// cache. Each workgroup leaves a flash-decoding partial (running max, sum of
// exp, unnormalised output) for AttnMergeKernel.
//
// Order of work: the position is read first, with the operands that do not
// depend on it (query and key rows, norm gains, the new value); a split past
// the position then leaves before it loads anything from the cache, and an
// active split loads its first tile's K/V rows -- only rows up to the
// position -- with the RoPE row. The QK-norm/RoPE jobs (query heads 0..G-1
// and the new key, job G, on waves jb % 4) run while the tile arrives. Per
// tile: the rows into LDS, one barrier, the next tile's loads issued, then
// each wave takes whole heads h = wave, wave + 4: scores, the online softmax
// update and P.V. The running state starts at (max -inf, sum 0, output 0):
// exp(-inf) = 0 leaves the first tile's sums as they are, so a split of one
// tile gives AttnSplitBody's partial.
__device__ __forceinline__ void AttnSplitTiledBody(const DecodeAttnArgs& a, int n_splits, int G) {
  const int kh = blockIdx.x, split = blockIdx.y;
  // every argument in the first round trip
  const int64_t max_seq = lanes::Uniform(a.max_seq);
  const auto kcache = lanes::UniformGlobal(a.kcache);
  const auto vcache = lanes::UniformGlobal(a.vcache);
  const auto rope = lanes::UniformGlobal(a.rope);
  const auto work = lanes::UniformGlobal(a.work);
  const float eps = lanes::Uniform(a.eps);
  const auto pos_dev = reinterpret_cast<const int32_t*>(lanes::Uniform(reinterpret_cast<uintptr_t>(a.pos_dev)));
  const int pos = lanes::UniformRead(pos_dev);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  __shared__ __align__(16) float ks[kSplit][kKStride];
  __shared__ __align__(16) float vs[kSplit][kHd];
  __shared__ __align__(16) float qs[8][kHd];
  // 1. job operands, position independent: slot t holds job wave + 4t. The
  // loads are unconditional (a slot past G reads query head 0 and is not
  // used): loads under a branch join as register copies that wait for them.
  float x0[3], x1[3], w0[3], w1[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const int jb = wave + kWaves * t;
    const bool is_k = jb == G;
    const float* src = is_k ? a.k + kh * kHd : a.q + (kh * G + (jb < G ? jb : 0)) * kHd;
    const float* nw = is_k ? a.k_norm : a.q_norm;
    x0[t] = src[lane];
    x1[t] = src[lane + 64];
    w0[t] = nw[lane];
    w1[t] = nw[lane + 64];
  }
  const float nv0 = a.v[kh * kHd + lane], nv1 = a.v[kh * kHd + lane + 64];
  const int n_keys = pos + 1;
  const int span = SplitSpan(n_keys);
  const int s0 = split * span;
  if (s0 >= n_keys) return;
  const int s1 = min(s0 + span, n_keys);
  const int n_tiles = (s1 - s0 + kSplit - 1) / kSplit;
  const bool has_new = s1 == n_keys;  // this split holds position pos (in its last tile)
  // 2. a tile's K/V rows (row r, 4-float column idx & 31) into registers:
  // rows tb .. tb + n - 1; the slots past n read row tb + n - 1 again (no
  // bytes past the history) and are replaced by zeros, and row n - 1 of the
  // tile holding pos by the new row, both in LDS below. Native vectors:
  // copies of HIP's float4 class stay memcpys that keep the tile in scratch
  // memory across the jobs.
  const auto kg = kcache + static_cast<int64_t>(kh) * max_seq * kHd;
  const auto vg = vcache + static_cast<int64_t>(kh) * max_seq * kHd;
  constexpr int kPer = kSplit * (kHd / 4) / kThreads;  // 4-float vectors per thread per tensor
  F4 kr[kPer], vr[kPer];
  auto load_tile = [&](int tb, int n) {
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int idx = tid + c * kThreads;
      const int64_t row = tb + min(idx >> 5, n - 1);
      kr[c] = *reinterpret_cast<lanes::GlobalPtr<const F4>>(kg + row * kHd + 4 * (idx & 31));
      vr[c] = *reinterpret_cast<lanes::GlobalPtr<const F4>>(vg + row * kHd + 4 * (idx & 31));
    }
  };
  load_tile(s0, min(kSplit, s1 - s0));
  const auto rope_row = rope + static_cast<int64_t>(pos) * kHd;
  const float rc = rope_row[lane], rs = rope_row[64 + lane];
  // 3. the jobs: slots 0 and 1 side by side (independent chains), slot 2
  // (G = 8, wave 0) after them
  float o0[3], o1[3];
  NormRopePair(x0[0], x1[0], w0[0], w1[0], rc, rs, eps, &o0[0], &o1[0]);
  NormRopePair(x0[1], x1[1], w0[1], w1[1], rc, rs, eps, &o0[1], &o1[1]);
  if (wave + 2 * kWaves <= G) NormRopePair(x0[2], x1[2], w0[2], w1[2], rc, rs, eps, &o0[2], &o1[2]);
  float nk0 = 0.f, nk1 = 0.f;
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const int jb = wave + kWaves * t;
    if (jb < G) {
      qs[jb][lane] = o0[t];
      qs[jb][lane + 64] = o1[t];
    } else if (jb == G) {
      nk0 = o0[t];
      nk1 = o1[t];
    }
  }
  const bool new_wave = has_new && wave == G % kWaves;
  if (new_wave) {
    const auto kd = kcache + (static_cast<int64_t>(kh) * max_seq + pos) * kHd;
    const auto vd = vcache + (static_cast<int64_t>(kh) * max_seq + pos) * kHd;
    kd[lane] = nk0;
    kd[lane + 64] = nk1;
    vd[lane] = nv0;
    vd[lane + 64] = nv1;
  }
  // running state of the wave's heads h = wave (slot 0) and wave + 4 (slot
  // 1, G = 8)
  struct Run {
    float m, l, a0, a1;
  };
  Run st0 = {-__builtin_inff(), 0.f, 0.f, 0.f}, st1 = st0;
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  const int j = lane & 31, half = lane >> 5;
  // 5. one head against the tile in LDS: lane (j = lane % 32, half = lane /
  // 32) scores key j over dims [64 half, +64); the halves add across lanes
  // j and j + 32; then the online softmax update and P.V
  auto head = [&](int h, int n, Run& r) {
    const F4* q4 = reinterpret_cast<const F4*>(&qs[h][64 * half]);
    const F4* k4 = reinterpret_cast<const F4*>(&ks[j][64 * half]);
    float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
    // four vectors per round: fully unrolled, the loads of all sixteen are
    // hoisted (162 VGPRs, three waves per SIMD); this way 116
#pragma unroll 4
    for (int ii = 0; ii < 16; ++ii) {
      const F4 qq = q4[ii], kk = k4[ii];
      d0 = __builtin_fmaf(qq.x, kk.x, d0);
      d1 = __builtin_fmaf(qq.y, kk.y, d1);
      d2 = __builtin_fmaf(qq.z, kk.z, d2);
      d3 = __builtin_fmaf(qq.w, kk.w, d3);
    }
    const float sc = lanes::AddXor32((d0 + d1) + (d2 + d3)) * scale;
    const float v = j < n ? sc : -__builtin_inff();
    const float m_new = fmaxf(r.m, WaveMaxF(v));
    const float alpha = ExpSoft(r.m - m_new);
    const float p = j < n ? ExpSoft(v - m_new) : 0.0f;
    r.l = __builtin_fmaf(r.l, alpha, WaveSumF(half == 0 ? p : 0.0f));
    r.m = m_new;
    // unnormalised P.V: lane takes dims 2 lane, 2 lane + 1; p_j from lane j
    // (rows from n on add p_j * 0 = +0 with p_j = 0: the sums are those
    // over j < n)
    float a0 = r.a0 * alpha, a1 = r.a1 * alpha;
#pragma unroll
    for (int jj = 0; jj < kSplit; ++jj) {
      const float pj = lanes::ReadLaneF(p, jj);
      const F2 vv = *reinterpret_cast<const F2*>(&vs[jj][2 * lane]);
      a0 = __builtin_fmaf(pj, vv.x, a0);
      a1 = __builtin_fmaf(pj, vv.y, a1);
    }
    r.a0 = a0;
    r.a1 = a1;
  };
  for (int t = 0; t < n_tiles; ++t) {
    const int tb = s0 + t * kSplit, n = min(kSplit, s1 - tb);
    const bool new_tile = has_new && t == n_tiles - 1;
    if (t > 0) __syncthreads();  // the previous tile's LDS reads are done
    // 4. the tile into LDS (row n - 1 of the tile holding pos is the new row;
    // rows from n on are zeros, so P.V can run over all 32 rows)
    if (new_tile && new_wave) {
      ks[n - 1][lane] = nk0;
      ks[n - 1][lane + 64] = nk1;
      vs[n - 1][lane] = nv0;
      vs[n - 1][lane + 64] = nv1;
    }
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int idx = tid + c * kThreads, r = idx >> 5, c4 = idx & 31;
      if (new_tile && r == n - 1) continue;
      const F4 z = {0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<F4*>(&ks[r][4 * c4]) = r < n ? kr[c] : z;
      *reinterpret_cast<F4*>(&vs[r][4 * c4]) = r < n ? vr[c] : z;
    }
    __syncthreads();
    if (t + 1 < n_tiles) load_tile(tb + kSplit, min(kSplit, s1 - tb - kSplit));
    if (wave < G) head(wave, n, st0);
    if (wave + kWaves < G) head(wave + kWaves, n, st1);
  }
  auto leave = [&](int h, const Run& r) {
    const auto w = work + (static_cast<int64_t>(kh * G + h) * n_splits + split) * kPart;
    if (lane == 0) {
      w[0] = r.m;
      w[1] = r.l;
    }
    *reinterpret_cast<lanes::GlobalPtr<F2>>(w + 2 + 2 * lane) = F2{r.a0, r.a1};
  };
  if (wave < G) leave(wave, st0);
  if (wave + kWaves < G) leave(wave + kWaves, st1);
}

__global__ __launch_bounds__(kThreads) void AttnSplitKernel(DecodeAttnArgs a, int n_splits, int G) {
  AttnSplitBody(a, n_splits, G);
}
__global__ __launch_bounds__(kThreads) void AttnSplitTiledKernel(DecodeAttnArgs a, int n_splits, int G) {
  AttnSplitTiledBody(a, n_splits, G);
}

// The operands of session blockIdx.z of a batch.
__device__ __forceinline__ DecodeAttnArgs BatchSlot(const DecodeAttnBatchArgs& b) {
  const int z = blockIdx.z;
  DecodeAttnArgs a = b.base;
  a.q += z * b.q_stride;
  a.k += z * b.kv_stride;
  a.v += z * b.kv_stride;
  a.out += z * b.q_stride;
  a.work += z * b.work_stride;
  a.pos_dev += z;
  a.kcache = b.kcache[z];
  a.vcache = b.vcache[z];
  a.max_seq = b.max_seq[z];
  return a;
}

// grid (n_kv, n_splits, sessions): AttnSplitKernel for each session of a
// batch, on its own cache and position.
__global__ __launch_bounds__(kThreads) void AttnSplitBatchKernel(DecodeAttnBatchArgs b, int n_splits, int G) {
  AttnSplitBody(BatchSlot(b), n_splits, G);
}
__global__ __launch_bounds__(kThreads) void AttnSplitTiledBatchKernel(DecodeAttnBatchArgs b, int n_splits, int G) {
  AttnSplitTiledBody(BatchSlot(b), n_splits, G);
}

// grid n_heads, one wave: out[h] = sum_s o_s * exp(m_s - M) / sum_s l_s *
// exp(m_s - M) over the splits of AttnSplitKernel.
__device__ __forceinline__ void AttnMergeBody(const DecodeAttnArgs& a, int n_splits) {
  constexpr int kBatch = 32;  // partial outputs per dimension in flight at once
  const int h = blockIdx.x, lane = threadIdx.x;
  const auto out = lanes::UniformGlobal(a.out);
  const auto w = lanes::UniformGlobal(a.work) + static_cast<int64_t>(h) * n_splits * kPart;
  const int n_keys = lanes::UniformRead(a.pos_dev) + 1;
  const int span = SplitSpan(n_keys);
  const int ns = (n_keys + span - 1) / span;
  __shared__ float fs[kSplitsPerHead];
  // one wave: the (max, sum) loads first, then the first batch of outputs
  // of dimensions lane and lane + 64; the weights are formed while the
  // outputs arrive
  constexpr int kPerLane = (kSplitsPerHead + 63) / 64;
  float mv[kPerLane], lv[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int s = min(lane + 64 * i, ns - 1);
    mv[i] = w[static_cast<int64_t>(s) * kPart];
    lv[i] = w[static_cast<int64_t>(s) * kPart + 1];
  }
  float v0[kBatch], v1[kBatch];
  auto load = [&](int sb) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t r = static_cast<int64_t>(min(sb + u, ns - 1)) * kPart + 2;
      v0[u] = w[r + lane];
      v1[u] = w[r + 64 + lane];
    }
  };
  load(0);
  float M = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) M = fmaxf(M, mv[i]);
  M = WaveMaxF(M);
  float L = 0.0f;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int s = lane + 64 * i;
    if (s < ns) {
      const float f = ExpSoft(mv[i] - M);
      fs[s] = f;
      L = __builtin_fmaf(lv[i], f, L);
    }
  }
  L = WaveSumF(L);
  __syncthreads();  // (one wave: orders the weights' LDS stores before the reads)
  float o0 = 0.0f, o1 = 0.0f;
  for (int sb = 0; sb < ns; sb += kBatch) {
    if (sb > 0) load(sb);
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float f = sb + u < ns ? fs[min(sb + u, ns - 1)] : 0.0f;
      o0 = __builtin_fmaf(v0[u], f, o0);
      o1 = __builtin_fmaf(v1[u], f, o1);
    }
  }
  out[static_cast<int64_t>(h) * kHd + lane] = o0 / L;
  out[static_cast<int64_t>(h) * kHd + 64 + lane] = o1 / L;
}

__global__ __launch_bounds__(64) void AttnMergeKernel(DecodeAttnArgs a, int n_splits) { AttnMergeBody(a, n_splits); }

// grid (n_heads, 1, sessions)
__global__ __launch_bounds__(64) void AttnMergeBatchKernel(DecodeAttnBatchArgs b, int n_splits) {
  AttnMergeBody(BatchSlot(b), n_splits);
}

// Virtual rows per wave tile for a matrix of `rows` rows (each side of a
// pair) and K inputs: prefer lanes that all get the same number of units
// (VR * K/32 a multiple of 64) and at least 1024 tiles (256 workgroups).
int ChooseVr(int rows, int K, bool pair) {
  const int U = K / 32;
  int best = pair ? 2 : 1;
  double best_score = -1.0;
  for (int vr = 8; vr >= (pair ? 2 : 1); vr >>= 1) {
    const int R = pair ? vr / 2 : vr;
    const double per_lane = static_cast<double>(vr) * U / 64.0;
    const double eff = per_lane / static_cast<double>(CeilDiv(static_cast<int64_t>(vr) * U, 64));
    const double tiles = static_cast<double>(CeilDiv(rows, R));
    const double score = eff * (tiles >= 1024.0 ? 1.0 : tiles / 1024.0);
    if (score > best_score + 1e-9) {
      best_score = score;
      best = vr;
    }
  }
  return best;
}

// The wave kernels stage the whole input in LDS (K + K/8 floats). Inputs
// wider than 14563 need more than the default 64 KiB of dynamic LDS: the
// kernel's limit is raised once, at its first such launch, to 159 KiB (of
// gfx950's 160 KiB per workgroup; the rest holds the kernel's static LDS):
// inputs up to 36181 wide.
constexpr size_t kWaveMaxLds = 159 * 1024;
template <auto Kern>
void WaveLaunch(const DecodeMatvecArgs& a, unsigned blocks, size_t lds, hipStream_t s) {
  if (lds > 64 * 1024) {
    static const bool opted = [] {
      HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(Kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(kWaveMaxLds)));
      return true;
    }();
    (void)opted;
  }
  hipLaunchKernelGGL(Kern, dim3(blocks), dim3(kThreads), lds, s, a);
}

template <uint32_t TA>
void LaunchWave(const DecodeMatvecArgs& a, unsigned blocks, size_t lds, uint32_t tb, hipStream_t s) {
  switch (tb) {
    case 12: WaveLaunch<MatvecWaveKernel<TA, 12>>(a, blocks, lds, s); break;
    case 14: WaveLaunch<MatvecWaveKernel<TA, 14>>(a, blocks, lds, s); break;
    case 8: WaveLaunch<MatvecWaveKernel<TA, 8>>(a, blocks, lds, s); break;
    case 0: WaveLaunch<MatvecWaveKernel<TA, 0>>(a, blocks, lds, s); break;
    default: Throw("decode matvec: unsupported weight type %u", tb);
  }
}

}  // namespace

void DecodeMatvec(DecodeMatvecArgs a, hipStream_t s) {
  RPG_CHECK(a.n_jobs >= 1 && a.n_jobs <= 3, "decode matvec: 1..3 jobs");
  RPG_CHECK(a.K % 32 == 0 && a.K > 0, "decode matvec: K must be a positive multiple of 32");
  for (int j = 0; j < a.n_jobs; ++j) RPG_CHECK(a.job[j].rows > 0 && a.job[j].w && a.job[j].y, "decode matvec: empty job");
  if (DecodeMatvecMfma(a, s)) return;
  if (a.inc != nullptr) {
    hipLaunchKernelGGL(IncKernel, dim3(1), dim3(1), 0, s, a.inc);
    a.inc = nullptr;
  }
  for (int j = 0; j < a.n_jobs; ++j)
    RPG_CHECK(!a.job[j].tiled && !a.job[j].pair, "decode matvec: tile-major copies run on the matrix-core path only");
  bool any = false;  // a job of another type, or a pair of two types: the generic tiles
  for (int j = 0; j < a.n_jobs; ++j) {
    const DecodeJob& J = a.job[j];
    any = any || !FastType(J.type) || (J.w2 && (!FastType(J.type2) || J.type2 != J.type));
  }
  if (any) {
    int tiles = 0;
    for (int j = 0; j < a.n_jobs; ++j) {
      DecodeJob& J = a.job[j];
      RPG_CHECK(a.K % BlockElems(J.type) == 0 && a.K / BlockElems(J.type) * BlockBytes(J.type) == J.row_bytes,
                "decode matvec: row bytes do not match K");
      RPG_CHECK(!J.w2 || (BlockElems(J.type2) > 0 && a.K % BlockElems(J.type2) == 0 &&
                          a.K / BlockElems(J.type2) * BlockBytes(J.type2) == J.row_bytes2),
                "decode matvec: pair row bytes do not match K");
      RPG_CHECK(!a.norm_w || a.K <= 8 * kNormChunks * kThreads, "decode matvec: RMSNorm input longer than %d",
                8 * kNormChunks * kThreads);
      J.rows_per_tile = ChooseVr(J.rows, a.K, J.w2 != nullptr);
      J.tiles = static_cast<int32_t>(CeilDiv(J.rows, J.w2 ? J.rows_per_tile / 2 : J.rows_per_tile));
      tiles += J.tiles;
    }
    const size_t lds = sizeof(float) * (static_cast<size_t>(a.K) + static_cast<size_t>(a.K / 8));
    RPG_CHECK(lds <= kWaveMaxLds, "decode matvec: input of %d needs %zu bytes of LDS", a.K, lds);
    WaveLaunch<MatvecAnyWaveKernel>(a, static_cast<unsigned>(CeilDiv(tiles, kWaves)), lds, s);
    HIP_CHECK(hipGetLastError());
    return;
  }
  // at most two distinct weight types per launch
  uint32_t types[2] = {a.job[0].type, a.job[0].type};
  int n_types = 1;
  int tiles = 0;
  for (int j = 0; j < a.n_jobs; ++j) {
    DecodeJob& J = a.job[j];
    RPG_CHECK(J.rows > 0 && J.w && J.y, "decode matvec: empty job");
    RPG_CHECK(!J.w2 || (J.type2 == J.type && J.row_bytes2 == J.row_bytes),
              "decode matvec: a SwiGLU pair needs one weight type");
    RPG_CHECK(static_cast<int64_t>(a.K) / BlockElems(J.type) * BlockBytes(J.type) == J.row_bytes,
              "decode matvec: row bytes do not match K");
    if (J.type != types[0] && J.type != types[1]) {
      RPG_CHECK(n_types < 2, "decode matvec: more than two weight types in one launch");
      types[1] = J.type;
      n_types = 2;
    }
    if (J.type == 12 || J.type == 14) RPG_CHECK(a.K % 256 == 0, "decode matvec: K-quant rows need K a multiple of 256");
    RPG_CHECK(!a.norm_w || a.K <= 8 * kNormChunks * kThreads, "decode matvec: RMSNorm input longer than %d",
              8 * kNormChunks * kThreads);
    J.rows_per_tile = ChooseVr(J.rows, a.K, J.w2 != nullptr);
    J.tiles = static_cast<int32_t>(CeilDiv(J.rows, J.w2 ? J.rows_per_tile / 2 : J.rows_per_tile));
    tiles += J.tiles;
  }
  const size_t lds = sizeof(float) * (static_cast<size_t>(a.K) + static_cast<size_t>(a.K / 8));
  RPG_CHECK(lds <= kWaveMaxLds, "decode matvec: input of %d needs %zu bytes of LDS", a.K, lds);
  const unsigned blocks = static_cast<unsigned>(CeilDiv(tiles, kWaves));
  switch (types[0]) {
    case 12: LaunchWave<12>(a, blocks, lds, types[1], s); break;
    case 14: LaunchWave<14>(a, blocks, lds, types[1], s); break;
    case 8: LaunchWave<8>(a, blocks, lds, types[1], s); break;
    case 0: LaunchWave<0>(a, blocks, lds, types[1], s); break;
    default: Throw("decode matvec: unsupported weight type %u", types[0]);
  }
  HIP_CHECK(hipGetLastError());
}

int64_t DecodeAttnWorkFloats(int n_heads, int n_kv, int64_t max_seq) {
  (void)n_kv;
  return static_cast<int64_t>(n_heads) * CeilDiv(max_seq, kSplit) * kPart;
}

int64_t DecodeAttnBatchWorkFloats(int n_heads, int64_t max_seq) {
  return static_cast<int64_t>(n_heads) * CeilDiv(max_seq, kSplit) * kPart;
}

void DecodeAttentionBatch(const DecodeAttnBatchArgs& b, int sessions, int64_t max_seq_all, hipStream_t s) {
  const DecodeAttnArgs& a = b.base;
  RPG_CHECK(sessions >= 1 && sessions <= kMaxDecodeBatch, "decode attention: %d sessions outside [1, %d]", sessions,
            kMaxDecodeBatch);
  RPG_CHECK(a.n_heads % a.n_kv == 0 && a.n_heads / a.n_kv <= 8, "decode attention: unsupported GQA group");
  RPG_CHECK(max_seq_all > 0 && max_seq_all <= INT32_MAX, "decode attention: capacity %lld", (long long)max_seq_all);
  // capacities of up to kSplitsPerHead tiles: one tile per split; longer
  // ones kSplitsPerHead splits of whole tiles (any capacity)
  const bool tiled = CeilDiv(max_seq_all, kSplit) > kSplitsPerHead;
  const int n_splits = static_cast<int>(std::min<int64_t>(CeilDiv(max_seq_all, kSplit), kSplitsPerHead));
  RPG_CHECK(b.work_stride >= DecodeAttnBatchWorkFloats(a.n_heads, max_seq_all), "decode attention: work too small");
  for (int z = 0; z < sessions; ++z)
    RPG_CHECK(b.max_seq[z] <= max_seq_all && b.kcache[z] && b.vcache[z], "decode attention: bad session %d", z);
  hipLaunchKernelGGL(tiled ? AttnSplitTiledBatchKernel : AttnSplitBatchKernel,
                     dim3(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(n_splits), static_cast<unsigned>(sessions)),
                     dim3(kThreads), 0, s, b, n_splits, a.n_heads / a.n_kv);
  hipLaunchKernelGGL(AttnMergeBatchKernel, dim3(static_cast<unsigned>(a.n_heads), 1, static_cast<unsigned>(sessions)),
                     dim3(64), 0, s, b, n_splits);
  HIP_CHECK(hipGetLastError());
}

void DecodeAttention(const DecodeAttnArgs& a, hipStream_t s) {
  RPG_CHECK(a.n_heads % a.n_kv == 0 && a.n_heads / a.n_kv <= 8, "decode attention: unsupported GQA group");
  RPG_CHECK(a.max_seq > 0 && a.max_seq <= INT32_MAX, "decode attention: capacity %lld", (long long)a.max_seq);
  // capacities of up to kSplitsPerHead tiles: one tile per split; longer
  // ones kSplitsPerHead splits of whole tiles (any capacity)
  const bool tiled = CeilDiv(a.max_seq, kSplit) > kSplitsPerHead;
  const int n_splits = static_cast<int>(std::min<int64_t>(CeilDiv(a.max_seq, kSplit), kSplitsPerHead));
  hipLaunchKernelGGL(tiled ? AttnSplitTiledKernel : AttnSplitKernel,
                     dim3(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(n_splits)),
                     dim3(kThreads), 0, s, a, n_splits, a.n_heads / a.n_kv);
  hipLaunchKernelGGL(AttnMergeKernel, dim3(static_cast<unsigned>(a.n_heads)), dim3(64), 0, s, a, n_splits);
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
