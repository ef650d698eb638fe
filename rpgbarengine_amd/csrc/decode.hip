// Decode-step (one token) kernels for gfx950.
//
// Matvec: a workgroup owns a tile of R output rows of one matrix. Its prologue
// stages the input vector in LDS -- RMS-normalised on the fly for the
// projections that consume a norm (reference src/qwen3.cc:131-134,191-194,
// 284-287), so no separate norm kernel runs. The tile's R x K/32 "units"
// (32 weights each, quant_dev.h) are spread over the 256 threads; every thread
// first issues the raw-byte loads of up to 4 units, then decodes and dots
// them against LDS, so a workgroup keeps ~32 KB of weights in flight and the
// raw GGUF rows stream contiguously. Per-(row, thread) partials are reduced
// in LDS in a fixed order (deterministic).
//
// Attention: QK-norm + RoPE of the query heads (and of the new key), KV-cache
// write and the split-K partial run in one kernel; a small combine kernel
// rescales the partials.

#include <hip/hip_runtime.h>

#include "common.h"
#include "decode.h"
#include "expf_glibc.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

constexpr int kThreads = 256;
constexpr int kBatch = 4;  // units in flight per thread
constexpr int kHd = 128;
constexpr int kChunk = 64;  // attention positions per split (matches attention.hip)

__device__ __forceinline__ float WaveSumF(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ double WaveSumD(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------- raw units

template <uint32_t T>
struct Raw;

template <>
struct Raw<12> {  // Q4_K: block header + 16 quant bytes
  uint4 hdr, q;
  __device__ __forceinline__ void Load(const uint8_t* row, int u) {
    const int b = u >> 3, g = (u >> 1) & 3, h = u & 1;
    const uint8_t* blk = row + 144 * b;
    hdr = *reinterpret_cast<const uint4*>(blk);
    q = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g + 16 * h);
  }
  __device__ __forceinline__ float Dot(int u, const float* xs) const {
    const int b = u >> 3, g = (u >> 1) & 3, h = u & 1;
    const float d = dev::HalfToFloatFast(hdr.x & 0xFFFFu);
    const float dmin = dev::HalfToFloatFast(hdr.x >> 16);
    uint32_t sc, mn;
    dev::ScaleMinK4(2 * g, hdr.y, hdr.z, hdr.w, &sc, &mn);
    const float dl = d * static_cast<float>(sc), ml = dmin * static_cast<float>(mn);
    dev::ScaleMinK4(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc, &mn);
    const float dh = d * static_cast<float>(sc), mh = dmin * static_cast<float>(mn);
    const float4* xlo = reinterpret_cast<const float4*>(xs + 256 * b + 64 * g + 16 * h);
    const float4* xhi = xlo + 8;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 a = xlo[c], e = xhi[c];
      const float av[4] = {a.x, a.y, a.z, a.w};
      const float ev[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t byte = dev::Byte(qw[c], i);
        s = __builtin_fmaf(av[i], __builtin_fmaf(dl, static_cast<float>(byte & 0x0Fu), -ml), s);
        s = __builtin_fmaf(ev[i], __builtin_fmaf(dh, static_cast<float>(byte >> 4), -mh), s);
      }
    }
    return s;
  }
};

template <>
struct Raw<14> {  // Q6_K: two 8-byte ql runs, 8 qh bytes, 4 scales, d
  uint2 l0, l1, hh;
  uint32_t sc4;  // the four int8 scales sc[si], sc[si+2], sc[si+4], sc[si+6]
  uint32_t dbits;
  __device__ __forceinline__ void Load(const uint8_t* row, int u) {
    const int b = u >> 3, half = (u >> 2) & 1, j = u & 3;
    const uint8_t* blk = row + 210 * b;
    l0 = dev::Load8Unaligned(blk + 64 * half + 8 * j);
    l1 = dev::Load8Unaligned(blk + 64 * half + 32 + 8 * j);
    hh = dev::Load8Unaligned(blk + 128 + 32 * half + 8 * j);
    const uint2 s = dev::Load8Unaligned(blk + 192 + 8 * half);  // sc[8*half .. +8)
    const int si = j >> 1;
    const uint32_t lo = si ? (s.x >> 8) : s.x;  // bytes si, si+2 live in s.x (si<2)
    const uint32_t hi = si ? (s.y >> 8) : s.y;  // bytes si+4, si+6 in s.y
    sc4 = (lo & 0xFFu) | (((lo >> 16) & 0xFFu) << 8) | ((hi & 0xFFu) << 16) | (((hi >> 16) & 0xFFu) << 24);
    dbits = dev::LoadU16(blk + 208);
  }
  __device__ __forceinline__ float Dot(int u, const float* xs) const {
    const int b = u >> 3, half = (u >> 2) & 1, j = u & 3;
    const float d = dev::HalfToFloatFast(dbits);
    const float s0 = d * static_cast<float>(static_cast<int8_t>(sc4 & 0xFFu));
    const float s1 = d * static_cast<float>(static_cast<int8_t>((sc4 >> 8) & 0xFFu));
    const float s2 = d * static_cast<float>(static_cast<int8_t>((sc4 >> 16) & 0xFFu));
    const float s3 = d * static_cast<float>(static_cast<int8_t>(sc4 >> 24));
    const float* base = xs + 256 * b + 128 * half + 8 * j;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t a = dev::Byte(i < 4 ? l0.x : l0.y, i & 3);
      const uint32_t c = dev::Byte(i < 4 ? l1.x : l1.y, i & 3);
      const uint32_t h = dev::Byte(i < 4 ? hh.x : hh.y, i & 3);
      const float w0 = s0 * static_cast<float>(static_cast<int>((a & 15u) | ((h & 3u) << 4)) - 32);
      const float w1 = s1 * static_cast<float>(static_cast<int>((c & 15u) | (((h >> 2) & 3u) << 4)) - 32);
      const float w2 = s2 * static_cast<float>(static_cast<int>((a >> 4) | (((h >> 4) & 3u) << 4)) - 32);
      const float w3 = s3 * static_cast<float>(static_cast<int>((c >> 4) | (((h >> 6) & 3u) << 4)) - 32);
      acc = __builtin_fmaf(base[i], w0, acc);
      acc = __builtin_fmaf(base[32 + i], w1, acc);
      acc = __builtin_fmaf(base[64 + i], w2, acc);
      acc = __builtin_fmaf(base[96 + i], w3, acc);
    }
    return acc;
  }
};

template <>
struct Raw<8> {  // Q8_0: d + 32 int8 (2-byte aligned)
  uint2 q[4];
  uint32_t dbits;
  __device__ __forceinline__ void Load(const uint8_t* row, int u) {
    const uint8_t* blk = row + 34 * u;
    dbits = dev::LoadU16(blk);
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = dev::Load8Unaligned(blk + 2 + 8 * c);
  }
  __device__ __forceinline__ float Dot(int u, const float* xs) const {
    const float d = dev::HalfToFloatFast(dbits);
    const float* base = xs + 32 * u;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = __builtin_fmaf(base[8 * c + i], static_cast<float>(static_cast<int8_t>(dev::Byte(q[c].x, i))) * d, acc);
        acc = __builtin_fmaf(base[8 * c + 4 + i], static_cast<float>(static_cast<int8_t>(dev::Byte(q[c].y, i))) * d,
                             acc);
      }
    }
    return acc;
  }
};

template <>
struct Raw<0> {  // F32
  float4 v[8];
  __device__ __forceinline__ void Load(const uint8_t* row, int u) {
    const float4* p = reinterpret_cast<const float4*>(row + 128 * u);
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = p[c];
  }
  __device__ __forceinline__ float Dot(int u, const float* xs) const {
    const float* base = xs + 32 * u;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      acc = __builtin_fmaf(base[4 * c + 0], v[c].x, acc);
      acc = __builtin_fmaf(base[4 * c + 1], v[c].y, acc);
      acc = __builtin_fmaf(base[4 * c + 2], v[c].z, acc);
      acc = __builtin_fmaf(base[4 * c + 3], v[c].w, acc);
    }
    return acc;
  }
};

// ---------------------------------------------------------------- prologue

// xs[0..K) = x, or RMSNorm(x) * w when norm_w != nullptr (double sum of
// squares, float scale, (x * scale) * w).
__device__ void StageVector(float* xs, const float* __restrict__ x, int K, const float* __restrict__ norm_w,
                            float eps, double* red) {
  const int tid = threadIdx.x;
  if (norm_w == nullptr) {
    for (int i = tid; i < K; i += kThreads) xs[i] = x[i];
    __syncthreads();
    return;
  }
  double s = 0.0;
  for (int i = tid; i < K; i += kThreads) {
    const float v = x[i];
    xs[i] = v;
    s += static_cast<double>(v) * v;
  }
  s = WaveSumD(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  const double total = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(total / static_cast<double>(K) + static_cast<double>(eps)));
  for (int i = tid; i < K; i += kThreads) xs[i] = __fmul_rn(__fmul_rn(xs[i], scale), norm_w[i]);
  __syncthreads();
}

// part[m][tid] (m < nmat*R) accumulates this thread's contributions to row m.
template <uint32_t T>
__device__ void TileRows(const uint8_t* __restrict__ w, int64_t row_bytes, int r0, int R, int upr, const float* xs,
                         float* part, int slot0) {
  constexpr int kB = T == 0 ? 1 : kBatch;  // F32 units are 128 bytes: no batching
  const int tid = threadIdx.x;
  const int items = R * upr;
  for (int base = tid; base < items; base += kThreads * kB) {
    Raw<T> raw[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int it = base + b * kThreads;
      if (it < items) {
        const int rl = it / upr, u = it - rl * upr;
        raw[b].Load(w + static_cast<int64_t>(r0 + rl) * row_bytes, u);
      }
    }
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int it = base + b * kThreads;
      if (it < items) {
        const int rl = it / upr, u = it - rl * upr;
        part[(slot0 + rl) * kThreads + tid] += raw[b].Dot(u, xs);
      }
    }
  }
}

// Sum part[slot][0..256) for slots [0, n): wave w handles slots w, w+4, ...
__device__ __forceinline__ float SlotSum(const float* part, int slot) {
  const int lane = threadIdx.x & 63;
  const float* p = part + slot * kThreads;
  float v = (p[lane] + p[lane + 64]) + (p[lane + 128] + p[lane + 192]);
  return WaveSumF(v);
}

// One kernel per (weight type, second-matrix type): all jobs of a launch share
// T1 (and T2 for SwiGLU pairs), so no type switch inflates register use.
template <uint32_t T1, uint32_t T2>
__global__ __launch_bounds__(kThreads) void MatvecM1Kernel(DecodeMatvecArgs a) {
  extern __shared__ float smem[];
  __shared__ double red[4];
  int t = blockIdx.x, j = 0;
  while (j + 1 < a.n_jobs && t >= a.job[j].tiles) {
    t -= a.job[j].tiles;
    ++j;
  }
  const DecodeJob& J = a.job[j];
  float* xs = smem;
  float* part = smem + a.K;
  StageVector(xs, a.x, a.K, a.norm_w, a.eps, red);
  const int r0 = t * J.rows_per_tile;
  const int R = min(J.rows_per_tile, J.rows - r0);
  const int nslots = J.w2 ? 2 * R : R;
  for (int i = threadIdx.x; i < nslots * kThreads; i += kThreads) part[i] = 0.0f;
  __syncthreads();
  const int upr = a.K >> 5;
  TileRows<T1>(J.w, J.row_bytes, r0, R, upr, xs, part, 0);
  if (J.w2) TileRows<T2>(J.w2, J.row_bytes2, r0, R, upr, xs, part, R);
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int rl = wave; rl < R; rl += kThreads / 64) {
    const float v = SlotSum(part, rl);
    if (J.w2) {
      const float u = SlotSum(part, R + rl);
      if (lane == 0) {
        // silu(g) * up with glibc-exact expf (reference src/kernels.h:82-92)
        const float sg = v / __fadd_rn(1.0f, GlibcExpf(-v));
        J.y[r0 + rl] = __fmul_rn(sg, u);
      }
    } else if (lane == 0) {
      float* y = J.y + r0 + rl;
      *y = a.epi == kAdd ? *y + v : v;
    }
  }
}

// ---------------------------------------------------------------- attention

// QK-norm + RoPE of one head vector held as lane pairs (i, i + 64).
__device__ __forceinline__ void NormRopePair(float x0, float x1, const float* __restrict__ nw,
                                             const float* __restrict__ rope_row, float eps, int i, float* o0,
                                             float* o1) {
  double s = static_cast<double>(x0) * x0 + static_cast<double>(x1) * x1;
  s = WaveSumD(s);
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(s / static_cast<double>(kHd) + static_cast<double>(eps)));
  const float na = __fmul_rn(__fmul_rn(x0, scale), nw[i]);
  const float nb = __fmul_rn(__fmul_rn(x1, scale), nw[i + 64]);
  const float c = rope_row[i], sn = rope_row[64 + i];
  *o0 = __fsub_rn(__fmul_rn(na, c), __fmul_rn(nb, sn));
  *o1 = __fadd_rn(__fmul_rn(nb, c), __fmul_rn(na, sn));
}

// grid (n_kv, n_splits): queries of the G heads of KV head kh, positions of
// this split; the split holding `pos` also writes the new K/V into the cache.
__global__ __launch_bounds__(kThreads) void AttnDecodeKernel(DecodeAttnArgs a, int n_splits) {
  const int kh = blockIdx.x, split = blockIdx.y;
  const int G = a.n_heads / a.n_kv;
  const int pos = *a.pos_dev;
  const int n_keys = pos + 1;
  const int s0 = split * kChunk;
  if (s0 >= n_keys) return;
  const int n = min(kChunk, n_keys - s0);
  const bool has_new = s0 + n == n_keys;  // this split holds position pos
  __shared__ __align__(16) float qs[8][kHd];
  __shared__ __align__(16) float knew[kHd];
  __shared__ float ps[8][kChunk];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* rope_row = a.rope + static_cast<int64_t>(pos) * kHd;
  // head vectors: jobs 0..G-1 are query heads, job G is the new key
  for (int jb = wave; jb < G + (has_new ? 1 : 0); jb += kThreads / 64) {
    const bool is_k = jb == G;
    const float* src = is_k ? a.k + kh * kHd : a.q + (kh * G + jb) * kHd;
    float o0, o1;
    NormRopePair(src[lane], src[lane + 64], is_k ? a.k_norm : a.q_norm, rope_row, a.eps, lane, &o0, &o1);
    if (is_k) {
      knew[lane] = o0;
      knew[lane + 64] = o1;
      float* kd = a.kcache + (static_cast<int64_t>(kh) * a.max_seq + pos) * kHd;
      float* vd = a.vcache + (static_cast<int64_t>(kh) * a.max_seq + pos) * kHd;
      kd[lane] = o0;
      kd[lane + 64] = o1;
      vd[lane] = a.v[kh * kHd + lane];
      vd[lane + 64] = a.v[kh * kHd + lane + 64];
    } else {
      qs[jb][lane] = o0;
      qs[jb][lane + 64] = o1;
    }
  }
  __syncthreads();
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  const float* kbase = a.kcache + (static_cast<int64_t>(kh) * a.max_seq + s0) * kHd;
  const float* vbase = a.vcache + (static_cast<int64_t>(kh) * a.max_seq + s0) * kHd;
  for (int gi = wave; gi < G; gi += kThreads / 64) {
    if (lane < n) {
      const bool is_new = has_new && lane == n - 1;
      const float4* k4 = reinterpret_cast<const float4*>(is_new ? knew : kbase + static_cast<int64_t>(lane) * kHd);
      const float4* q4 = reinterpret_cast<const float4*>(qs[gi]);
      float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
#pragma unroll 8
      for (int i = 0; i < kHd / 4; ++i) {
        const float4 qq = q4[i], kk = k4[i];
        d0 = __builtin_fmaf(qq.x, kk.x, d0);
        d1 = __builtin_fmaf(qq.y, kk.y, d1);
        d2 = __builtin_fmaf(qq.z, kk.z, d2);
        d3 = __builtin_fmaf(qq.w, kk.w, d3);
      }
      ps[gi][lane] = ((d0 + d1) + (d2 + d3)) * scale;
    }
  }
  __syncthreads();
  for (int gi = wave; gi < G; gi += kThreads / 64) {
    const float v = lane < n ? ps[gi][lane] : -__builtin_inff();
    float m = v;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    const float p = lane < n ? GlibcExpf(v - m) : 0.0f;
    const float l = WaveSumF(p);
    ps[gi][lane] = p;
    if (lane == 0) {
      float* w = a.work + (static_cast<int64_t>(kh * G + gi) * n_splits + split) * (2 + kHd);
      w[0] = m;
      w[1] = l;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * kHd; idx += kThreads) {
    const int gi = idx / kHd, d = idx % kHd;
    float acc = 0.0f;
    for (int t = 0; t < n; ++t) {
      const float vv = (has_new && t == n - 1) ? a.v[kh * kHd + d] : vbase[static_cast<int64_t>(t) * kHd + d];
      acc = __builtin_fmaf(ps[gi][t], vv, acc);
    }
    a.work[(static_cast<int64_t>(kh * G + gi) * n_splits + split) * (2 + kHd) + 2 + d] = acc;
  }
}

__global__ __launch_bounds__(kHd) void AttnCombineKernel(DecodeAttnArgs a, int n_splits) {
  const int h = blockIdx.x, d = threadIdx.x;
  const int ns = (*a.pos_dev + 1 + kChunk - 1) / kChunk;
  const float* w = a.work + static_cast<int64_t>(h) * n_splits * (2 + kHd);
  float M = -__builtin_inff();
  for (int s = 0; s < ns; ++s) M = fmaxf(M, w[s * (2 + kHd)]);
  float L = 0.0f, o = 0.0f;
  for (int s = 0; s < ns; ++s) {
    const float f = GlibcExpf(w[s * (2 + kHd)] - M);
    L = __builtin_fmaf(w[s * (2 + kHd) + 1], f, L);
    o = __builtin_fmaf(w[s * (2 + kHd) + 2 + d], f, o);
  }
  a.out[static_cast<int64_t>(h) * kHd + d] = o / L;
}

}  // namespace

// Rows per workgroup: ~1024 units per tile (4 per thread), at least ~512
// tiles for the whole launch when the matrix allows it.
int DecodeRowsPerTile(int rows, int K, bool paired) {
  const int upr = K / 32;
  int R = (1024 + upr * (paired ? 2 : 1) - 1) / (upr * (paired ? 2 : 1));
  R = R < 1 ? 1 : (R > 16 ? 16 : R);
  const int cap = rows / 512;
  if (cap >= 1 && R > cap) R = cap;
  return R;
}

namespace {

template <uint32_t T1>
void LaunchM1(const DecodeMatvecArgs& a, unsigned tiles, size_t lds, uint32_t t2, hipStream_t s) {
  switch (t2) {
    case 12: hipLaunchKernelGGL((MatvecM1Kernel<T1, 12>), dim3(tiles), dim3(kThreads), lds, s, a); break;
    case 14: hipLaunchKernelGGL((MatvecM1Kernel<T1, 14>), dim3(tiles), dim3(kThreads), lds, s, a); break;
    case 8: hipLaunchKernelGGL((MatvecM1Kernel<T1, 8>), dim3(tiles), dim3(kThreads), lds, s, a); break;
    case 0: hipLaunchKernelGGL((MatvecM1Kernel<T1, 0>), dim3(tiles), dim3(kThreads), lds, s, a); break;
    default: Throw("decode matvec: unsupported second weight type %u", t2);
  }
}

// Launch the jobs of `a` that share one (type, type2) pair.
void LaunchGroup(DecodeMatvecArgs a, hipStream_t s) {
  int tiles = 0, max_slots = 0;
  for (int j = 0; j < a.n_jobs; ++j) {
    DecodeJob& J = a.job[j];
    RPG_CHECK(J.rows_per_tile >= 1 && J.rows_per_tile <= 16, "decode matvec: rows per tile");
    J.tiles = static_cast<int32_t>(CeilDiv(J.rows, J.rows_per_tile));
    tiles += J.tiles;
    const int slots = (J.w2 ? 2 : 1) * J.rows_per_tile;
    max_slots = slots > max_slots ? slots : max_slots;
  }
  const size_t lds = sizeof(float) * (static_cast<size_t>(a.K) + static_cast<size_t>(max_slots) * kThreads);
  RPG_CHECK(lds <= 64 * 1024, "decode matvec: %zu bytes of LDS exceed 64 KiB", lds);
  const uint32_t t1 = a.job[0].type, t2 = a.job[0].w2 ? a.job[0].type2 : a.job[0].type;
  switch (t1) {
    case 12: LaunchM1<12>(a, static_cast<unsigned>(tiles), lds, t2, s); break;
    case 14: LaunchM1<14>(a, static_cast<unsigned>(tiles), lds, t2, s); break;
    case 8: LaunchM1<8>(a, static_cast<unsigned>(tiles), lds, t2, s); break;
    case 0: LaunchM1<0>(a, static_cast<unsigned>(tiles), lds, t2, s); break;
    default: Throw("decode matvec: unsupported weight type %u", t1);
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace

void DecodeMatvec(DecodeMatvecArgs a, hipStream_t s) {
  RPG_CHECK(a.n_jobs >= 1 && a.n_jobs <= 3, "decode matvec: 1..3 jobs");
  RPG_CHECK(a.K % 32 == 0, "decode matvec: K must be a multiple of 32");
  // one launch per distinct (type, type2) among the jobs
  bool done[3] = {false, false, false};
  for (int j = 0; j < a.n_jobs; ++j) {
    if (done[j]) continue;
    DecodeMatvecArgs g = a;
    g.n_jobs = 0;
    for (int i = j; i < a.n_jobs; ++i) {
      const bool same = a.job[i].type == a.job[j].type && (a.job[i].w2 != nullptr) == (a.job[j].w2 != nullptr) &&
                        (!a.job[i].w2 || a.job[i].type2 == a.job[j].type2);
      if (!done[i] && same) {
        g.job[g.n_jobs++] = a.job[i];
        done[i] = true;
      }
    }
    LaunchGroup(g, s);
  }
}

void DecodeAttention(const DecodeAttnArgs& a, hipStream_t s) {
  RPG_CHECK(a.n_heads % a.n_kv == 0 && a.n_heads / a.n_kv <= 8, "decode attention: unsupported GQA group");
  const int n_splits = static_cast<int>(CeilDiv(a.max_seq, kChunk));
  hipLaunchKernelGGL(AttnDecodeKernel, dim3(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(n_splits)),
                     dim3(kThreads), 0, s, a, n_splits);
  hipLaunchKernelGGL(AttnCombineKernel, dim3(static_cast<unsigned>(a.n_heads)), dim3(kHd), 0, s, a, n_splits);
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
