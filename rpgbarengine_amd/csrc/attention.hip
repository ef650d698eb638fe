// GQA causal attention over the device KV cache (reference src/qwen3.cc:79-117).
//
// Cache layout is the reference's: fp32 [layer][kv_head][max_seq][head_dim]
// (reference src/kv_cache.h:19-34), so one KV head's history is one contiguous
// stream. head_dim is 128.
//
// Decode (one query): split-K ("flash-decoding"). Workgroup (kv_head, split)
// takes 64 positions for all G = n_heads / n_kv query heads of that KV head:
// scores in LDS, per-head local max / exp-sum / un-normalised P.V, written as
// a partial; a combine kernel rescales the partials by exp(m_s - M) and
// divides by the global sum. The split grid is sized for max_seq and reads the
// position from device memory, so a captured decode graph replays at any
// position; splits past the position exit at once.
//
// Prefill (several queries): one workgroup per (query head, query), scores for
// every visible position in LDS, softmax, P.V.

#include <hip/hip_runtime.h>

#include "common.h"
#include "expf_glibc.h"
#include "kernels.h"

namespace rpg {
namespace k {

namespace {

constexpr int kChunk = 64;  // positions per decode split
constexpr int kHd = 128;
constexpr int kMaxGroup = 8;

__device__ __forceinline__ float WaveMax(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float WaveSum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float Dot128(const float* __restrict__ q, const float* __restrict__ k) {
  const float4* k4 = reinterpret_cast<const float4*>(k);
  const float4* q4 = reinterpret_cast<const float4*>(q);
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll 8
  for (int i = 0; i < kHd / 4; ++i) {
    const float4 a = q4[i], b = k4[i];
    s0 = __builtin_fmaf(a.x, b.x, s0);
    s1 = __builtin_fmaf(a.y, b.y, s1);
    s2 = __builtin_fmaf(a.z, b.z, s2);
    s3 = __builtin_fmaf(a.w, b.w, s3);
  }
  return (s0 + s1) + (s2 + s3);
}

// work layout: [n_heads][n_splits][2 + kHd] = (m, l, o[128])
__global__ __launch_bounds__(256) void DecodePartialKernel(AttnArgs a, int n_splits) {
  const int kh = blockIdx.x;
  const int split = blockIdx.y;
  const int G = a.n_heads / a.n_kv;
  const int pos = a.pos0_dev ? *a.pos0_dev : a.pos0_host;
  const int n_keys = pos + 1;
  const int s0 = split * kChunk;
  if (s0 >= n_keys) return;
  const int n = min(kChunk, n_keys - s0);
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  __shared__ __align__(16) float qs[kMaxGroup][kHd];
  __shared__ float ps[kMaxGroup][kChunk];
  const int tid = threadIdx.x;
  for (int i = tid; i < G * kHd; i += 256) qs[i / kHd][i % kHd] = a.q[(kh * G) * kHd + i];
  __syncthreads();
  const float* kbase = a.kcache + (static_cast<int64_t>(kh) * a.max_seq + s0) * kHd;
  const float* vbase = a.vcache + (static_cast<int64_t>(kh) * a.max_seq + s0) * kHd;
  for (int gi = tid / 64; gi < G; gi += 4) {
    const int t = tid & 63;
    if (t < n) ps[gi][t] = Dot128(qs[gi], kbase + static_cast<int64_t>(t) * kHd) * scale;
  }
  __syncthreads();
  for (int gi = tid / 64; gi < G; gi += 4) {
    const int t = tid & 63;
    const float v = t < n ? ps[gi][t] : -__builtin_inff();
    const float m = WaveMax(v);
    const float p = t < n ? GlibcExpf(v - m) : 0.0f;
    const float l = WaveSum(p);
    ps[gi][t] = p;
    if (t == 0) {
      float* w = a.work + (static_cast<int64_t>(kh * G + gi) * n_splits + split) * (2 + kHd);
      w[0] = m;
      w[1] = l;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * kHd; idx += 256) {
    const int gi = idx / kHd, d = idx % kHd;
    float acc = 0.0f;
    for (int t = 0; t < n; ++t) acc = __builtin_fmaf(ps[gi][t], vbase[static_cast<int64_t>(t) * kHd + d], acc);
    a.work[(static_cast<int64_t>(kh * G + gi) * n_splits + split) * (2 + kHd) + 2 + d] = acc;
  }
}

__global__ __launch_bounds__(128) void DecodeCombineKernel(AttnArgs a, int n_splits) {
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  const int pos = a.pos0_dev ? *a.pos0_dev : a.pos0_host;
  const int ns = (pos + 1 + kChunk - 1) / kChunk;
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

// grid (n_heads, seq); dynamic LDS: (pos0 + seq) floats of scores.
__global__ __launch_bounds__(256) void PrefillKernel(AttnArgs a) {
  extern __shared__ float sc[];
  __shared__ __align__(16) float qv[kHd];
  __shared__ float red[8];
  __shared__ float part[2][kHd];
  const int h = blockIdx.x;
  const int t = blockIdx.y;
  const int G = a.n_heads / a.n_kv;
  const int kh = h / G;
  const int pos0 = a.pos0_dev ? *a.pos0_dev : a.pos0_host;
  const int n_keys = pos0 + t + 1;
  const int tid = threadIdx.x;
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  const float* q = a.q + (static_cast<int64_t>(t) * a.n_heads + h) * kHd;
  if (tid < kHd) qv[tid] = q[tid];
  __syncthreads();
  const float* kb = a.kcache + static_cast<int64_t>(kh) * a.max_seq * kHd;
  const float* vb = a.vcache + static_cast<int64_t>(kh) * a.max_seq * kHd;
  float m = -__builtin_inff();
  for (int s = tid; s < n_keys; s += 256) {
    const float v = Dot128(qv, kb + static_cast<int64_t>(s) * kHd) * scale;
    sc[s] = v;
    m = fmaxf(m, v);
  }
  m = WaveMax(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.0f;
  for (int s = tid; s < n_keys; s += 256) {
    const float p = GlibcExpf(sc[s] - m);
    sc[s] = p;
    l += p;
  }
  l = WaveSum(l);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = l;
  __syncthreads();
  const float L = (red[4] + red[5]) + (red[6] + red[7]);
  // two halves of the positions, 128 dims each
  const int d = tid & (kHd - 1);
  const int hv = tid >> 7;
  const int mid = n_keys / 2;
  const int sb = hv ? mid : 0, se = hv ? n_keys : mid;
  float acc = 0.0f;
  for (int s = sb; s < se; ++s) acc = __builtin_fmaf(sc[s], vb[static_cast<int64_t>(s) * kHd + d], acc);
  part[hv][d] = acc;
  __syncthreads();
  if (tid < kHd) a.out[(static_cast<int64_t>(t) * a.n_heads + h) * kHd + tid] = (part[0][tid] + part[1][tid]) / L;
}

}  // namespace

int64_t AttnWorkFloats(int n_heads, int64_t max_seq) {
  return static_cast<int64_t>(n_heads) * CeilDiv(max_seq, kChunk) * (2 + kHd);
}

void Attention(const AttnArgs& a, hipStream_t s) {
  RPG_CHECK(a.hd == kHd, "attention kernels are built for head_dim 128 (got %d)", a.hd);
  RPG_CHECK(a.n_heads % a.n_kv == 0 && a.n_heads / a.n_kv <= kMaxGroup, "attention: unsupported GQA group");
  if (a.seq == 1) {
    const int n_splits = static_cast<int>(CeilDiv(a.max_seq, kChunk));
    hipLaunchKernelGGL(DecodePartialKernel, dim3(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(n_splits)),
                       dim3(256), 0, s, a, n_splits);
    hipLaunchKernelGGL(DecodeCombineKernel, dim3(static_cast<unsigned>(a.n_heads)), dim3(kHd), 0, s, a, n_splits);
  } else if (a.seq > 1) {
    RPG_CHECK(a.pos0_dev == nullptr, "prefill attention takes a host position");
    const int64_t n_keys_max = static_cast<int64_t>(a.pos0_host) + a.seq;
    RPG_CHECK(n_keys_max <= a.max_seq, "attention past the cache capacity");
    const size_t lds = static_cast<size_t>(n_keys_max) * sizeof(float);
    RPG_CHECK(lds <= 60 * 1024, "prefill attention: %lld positions exceed the LDS score buffer",
              (long long)n_keys_max);
    hipLaunchKernelGGL(PrefillKernel, dim3(static_cast<unsigned>(a.n_heads), static_cast<unsigned>(a.seq)), dim3(256),
                       lds, s, a);
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
