// GQA causal attention over the device KV cache (reference src/qwen3.cc:79-117).
//
// Cache layout is the reference's: fp32 [layer][kv_head][max_seq][head_dim]
// (reference src/kv_cache.h:19-34), so one KV head's history is one contiguous
// stream. head_dim is 128.
//
// One-query segments of the prefill path (a single new token after a reused
// prefix): split-K ("flash-decoding"). Workgroup (kv_head, split) takes 64
// positions for all G = n_heads / n_kv query heads of that KV head: scores
// in LDS, per-head local max / exp-sum / un-normalised P.V, written as a
// partial; a combine kernel rescales the partials by exp(m_s - M) and
// divides by the global sum. (The decode step's attention, with QK-norm,
// RoPE and the cache write folded in, is in decode.hip.)
//
// Prefill (several queries): PrefillKernel, workgroup (kv head, 16 or 32
// queries), two waves per query head of the group splitting the key blocks,
// scores and P.V as f16 hi/lo products on the matrix cores (16x16x32), K/V
// blocks of 32 positions staged once for the group, online softmax.

#include <hip/hip_runtime.h>

#include "common.h"
#include "expf_glibc.h"
#include "kernels.h"
#include "lanes.h"
#include "soft_exp.h"

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
// Prefill: workgroup (kv head, block of 16 queries), one wave per query head
// of the group. Scores Q.K^T and P.V run on v_mfma_f32_16x16x32_f16 with
// every fp32 operand split x = hi + lo into two f16 (hi = f16(x), lo =
// f16(x - hi): 22 significant bits) and three products per pair (hi.hi +
// hi.lo + lo.hi; the dropped lo.lo is below 2^-22 of the product), summed in
// fp32. Keys come in blocks of 32 positions, staged in LDS once for the G
// waves (K row-major, V transposed, hi and lo planes); softmax is online per
// query row: running max m and sum l, the earlier blocks' P.V and l
// rescaled by exp(m_old - m_new), the output divided by l at the end -- the
// reference's max / exp / sum / weighted sum up to summation order, the
// 22-bit operands and ExpSoft's exp (these probabilities only feed logits
// judged within 1e-3 of max|logit|). The operands are scaled by powers of
// two per query row, key row and (value dimension, key block) before the
// split (ScaleExp): any fp32 magnitude is safe, and each value block's P.V
// product is scaled back as it is added to the running output.
//
// MFMA 16x16x32 f16 lane layout: A[i][k] in lane i + 16 (k / 8), element
// k % 8; B[k][j] in lane j + 16 (k / 8); C[4 (l / 16) + e][l % 16] in element
// e of lane l. Scores are formed transposed, S^T = K.Q^T (A = 16 keys, B =
// 16 queries; a 32-dimension chunk c gives lane group g the dimensions 32 c
// + 8 g .. + 7 of its key and of its query), so lane l holds query l % 16
// and keys 16 jt + 4 (l / 16) + e of the block's two key tiles jt: its 8
// probabilities are a B operand of O^T = V^T.P^T as they stand, keys taken
// in slot order 8 g + 4 jt + e. V^T rows are staged in that slot order.
constexpr int kQB = 16;        // queries per query tile (one tile per workgroup, or two: PrefillKernel)
constexpr int kWideQueries = 1024;  // segments at least this long take two query tiles per workgroup (G <= 2)
constexpr int kKB = 32;        // keys per block
constexpr int kKH = kHd + 8;   // K row in LDS (halfs)
constexpr int kVH = kKB + 8;   // V^T row in LDS (halfs)

typedef float F4v __attribute__((ext_vector_type(4)));
typedef _Float16 H4v __attribute__((ext_vector_type(4)));
typedef _Float16 H8v __attribute__((ext_vector_type(8)));

// Range guard of the f16 operands: every fp32 operand row (a query, a key)
// or column block (a value dimension over 32 keys) is multiplied by a power
// of two that brings its largest magnitude into [2^14, 2^15) before the
// hi / lo split, and the products are multiplied back by the inverse power
// (both exact while they stay normal floats): no value overflows the f16
// range (65504) or falls into its subnormals relative to its row's maximum.
// The exponent is clamped so that both powers stay normal; a zero row takes 1.
__device__ __forceinline__ int ScaleExp(float max_abs) {
  const int eb = static_cast<int>(__float_as_uint(max_abs) >> 23);
  return max_abs > 0.0f ? min(max(141 - eb, -126), 126) : 0;
}
__device__ __forceinline__ float Pow2(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }
// maxima over aligned groups of 8 and 32 lanes (DPP quad and half-row /
// row mirrors, then the permlane16 swap)
__device__ __forceinline__ float Max8Lanes(float v) {
  v = fmaxf(v, lanes::DppF<lanes::kQuadXor1>(v));
  v = fmaxf(v, lanes::DppF<lanes::kQuadXor2>(v));
  return fmaxf(v, lanes::DppF<lanes::kRowHalfMirror>(v));
}
__device__ __forceinline__ float Max32Lanes(float v) {
  v = Max8Lanes(v);
  v = fmaxf(v, lanes::DppF<lanes::kRowMirror>(v));
  return lanes::MaxXor16(v);
}

// x = hi[i] + lo[i] to 22 bits
template <typename V>
__device__ __forceinline__ void SplitHalf(float x, V& hi, V& lo, int i) {
  const _Float16 h = static_cast<_Float16>(x);
  hi[i] = h;
  lo[i] = static_cast<_Float16>(x - static_cast<float>(h));
}

// The empty asm keeps a and b live past the product, so the result is never
// allocated over them (an MFMA whose destination aliases its A/B registers
// gives wrong sums on gfx950, and the compiler allows it when a source dies
// at the MFMA). The kernel keeps its accumulators in VGPRs, where the
// constraint costs nothing.
__device__ __forceinline__ F4v Mfma16(H8v a, H8v b, F4v c) {
  const F4v r = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(r));
  return r;
}
// the three products of (ah + al) (bh + bl)
__device__ __forceinline__ F4v Mfma16x3(H8v ah, H8v al, H8v bh, H8v bl, F4v c) {
  return Mfma16(al, bh, Mfma16(ah, bl, Mfma16(ah, bh, c)));
}

// G: query heads per KV head. Two waves per head split the key blocks (even
// and odd) and merge their online-softmax states at the end; QT query tiles
// of 16 share the workgroup's staged K/V blocks (long segments at G <= 2:
// half the staging per query), so a workgroup has 2 G QT waves.
template <int G, int QT>
__global__ __launch_bounds__(128 * G * QT) void PrefillKernel(AttnArgs a) {
  constexpr int nt = 128 * G * QT;
  // halfs of one K block ([hi, lo][key][dimension]) and of one V^T block
  // ([hi, lo][dimension][key])
  constexpr int kKbH = 2 * kKB * kKH, kVbH = 2 * kHd * kVH;
  // blocks per half and step (two, with 148 KB of LDS at G = 4, measured
  // no faster: the per-block chain of scores, softmax and P.V sets the
  // time, not the step's barriers)
  constexpr int kSB = 1, kBS = 2 * kSB;
  // the step's K and V^T blocks; reused at the end for the merge exchange
  __shared__ __align__(16) _Float16 kv[kBS * (kKbH + kVbH)];
  // inverse operand scales of the step's blocks: per key, per value dimension
  __shared__ __align__(16) float kinv[kBS][kKB];
  __shared__ __align__(16) float vinv[kBS][kHd];
  // the longest query blocks (most keys) are dispatched first
  const int kh = blockIdx.x, qb = static_cast<int>(gridDim.y - 1 - blockIdx.y);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int hg = w % G, half = (w / G) & 1, qt = w / (2 * G);  // head within the group, key half, query tile
  const int h = kh * G + hg;
  const int c16 = lane & 15, kg = lane >> 4;
  const int pos0 = a.pos0_host;
  const int t0b = qb * kQB * QT, t0 = t0b + kQB * qt;  // the workgroup's and the wave's first query
  const int t_last = min(t0b + kQB * QT, a.seq) - 1;
  const int n_keys = pos0 + t_last + 1;  // keys the block's last query sees
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  // this lane's query t0 + c16 (clamped) sees keys up to tmax; its output
  // dimensions 16 ct + 4 kg + e sit in element e of o[ct]
  const int tmax = pos0 + min(t0 + c16, a.seq - 1);
  F4v o[8];
#pragma unroll
  for (int ct = 0; ct < 8; ++ct) o[ct] = F4v{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.0f;
  const float* kb = a.kcache + static_cast<int64_t>(kh) * a.max_seq * kHd;
  const float* vb = a.vcache + static_cast<int64_t>(kh) * a.max_seq * kHd;
  const int n_blocks = (n_keys + kKB - 1) / kKB;
  const int n_steps = (n_blocks + kBS - 1) / kBS;
  // step i stages blocks kBS i .. kBS i + kBS - 1: K as float4 units u = block
  // (u / 1024), key ((u / 32) % 32), column (u % 32) (32 lanes read one key
  // row and write it contiguously); V as units of 4 keys x
  // 4 dimensions u = block (u / 256), key quad (u % 8), column ((u / 8) %
  // 32), so that a thread writes 4 consecutive keys of a V^T row and 8
  // consecutive lanes one 64-byte run of it (no bank conflicts); thread tid
  // takes u = tid + i * nt. Keys past the last visible one repeat it (masked
  // below). The next step's loads are in flight while the current one is
  // multiplied.
  constexpr int kKUnits = kBS * kKB * (kHd / 4), kVUnits = kBS * (kKB / 4) * (kHd / 4);
  constexpr int kKPer = (kKUnits + nt - 1) / nt, kVPer = (kVUnits + nt - 1) / nt;
  // (native vectors: copies of HIP's float4 class stay memcpys that can keep
  // the registers in scratch memory)
  F4v kreg[kKPer], vreg[kVPer][4];
  auto load_step = [&](int st) {
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      const int u = min(tid + i * nt, kKUnits - 1), c4 = u & 31, j = (u >> 5) & (kKB - 1), bb = u >> 10;
      const int64_t row = static_cast<int64_t>(min((kBS * st + bb) * kKB + j, n_keys - 1)) * kHd;
      kreg[i] = *(const __attribute__((address_space(1))) F4v*)(kb + row + 4 * c4);
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int u = min(tid + i * nt, kVUnits - 1), jq = u & 7, c4 = (u >> 3) & 31, bb = u >> 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = static_cast<int64_t>(min((kBS * st + bb) * kKB + 4 * jq + r, n_keys - 1)) * kHd;
        vreg[i][r] = *(const __attribute__((address_space(1))) F4v*)(vb + row + 4 * c4);
      }
    }
  };
  load_step(0);
  // (after the first K/V loads, so that both round trips overlap)
  // this lane's query row c16 (clamped past the segment: computed, not
  // stored), dimensions 32 c + 8 kg .. + 7 of chunk c, split hi + lo
  H8v qh[4], ql[4];
  float qinv;  // the inverse of the query row's scale, times 1 / sqrt(128)
  {
    const int tq = min(t0 + c16, a.seq - 1);
    const float* qrow = a.q + (static_cast<int64_t>(tq) * a.n_heads + h) * kHd + 8 * kg;
    float x[4][8];
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v0 = *reinterpret_cast<const float4*>(qrow + 32 * c);
      const float4 v1 = *reinterpret_cast<const float4*>(qrow + 32 * c + 4);
      x[c][0] = v0.x, x[c][1] = v0.y, x[c][2] = v0.z, x[c][3] = v0.w;
      x[c][4] = v1.x, x[c][5] = v1.y, x[c][6] = v1.z, x[c][7] = v1.w;
#pragma unroll
      for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(x[c][i]));
    }
    // the row's 128 dimensions sit in the four lanes 16 apart
    mx = lanes::MaxXor16(mx);
    mx = lanes::MaxXor32(mx);
    const int se = ScaleExp(mx);
    const float sq = Pow2(se);
    qinv = scale * Pow2(-se);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) SplitHalf(x[c][i] * sq, qh[c], ql[c], i);
  }
  for (int st = 0; st < n_steps; ++st) {
    __syncthreads();  // the previous step's LDS reads are done
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      const int u = tid + i * nt, c4 = u & 31, j = (u >> 5) & (kKB - 1), bb = u >> 10;
      if (kKUnits % nt != 0 && u >= kKUnits) break;
      // the key row's scale (its 32 column chunks sit in 32 adjacent lanes)
      float mx = fmaxf(fmaxf(fabsf(kreg[i][0]), fabsf(kreg[i][1])), fmaxf(fabsf(kreg[i][2]), fabsf(kreg[i][3])));
      const int se = ScaleExp(Max32Lanes(mx));
      const float sk = Pow2(se);
      if (c4 == 0) kinv[bb][j] = Pow2(-se);
      _Float16* ks = kv + bb * kKbH + j * kKH + 4 * c4;
      H4v hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) SplitHalf(kreg[i][e] * sk, hi, lo, e);
      *reinterpret_cast<H4v*>(ks) = hi;
      *reinterpret_cast<H4v*>(ks + kKB * kKH) = lo;
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int u = tid + i * nt, jq = u & 7, c4 = (u >> 3) & 31, bb = u >> 8;
      if (kVUnits % nt != 0 && u >= kVUnits) break;
      const int slot = jq < 4 ? 8 * jq : 8 * (jq - 4) + 4;  // keys 4 jq .. + 3 in slot order
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        // dimension 4 c4 + d of the block: its 32 keys sit in 8 adjacent lanes
        float mx = fmaxf(fmaxf(fabsf(vreg[i][0][d]), fabsf(vreg[i][1][d])),
                         fmaxf(fabsf(vreg[i][2][d]), fabsf(vreg[i][3][d])));
        const int se = ScaleExp(Max8Lanes(mx));
        const float sv = Pow2(se);
        if (jq == 0) vinv[bb][4 * c4 + d] = Pow2(-se);
        _Float16* vt = kv + kBS * kKbH + bb * kVbH + (4 * c4 + d) * kVH + slot;
        H4v hi, lo;
#pragma unroll
        for (int r = 0; r < 4; ++r) SplitHalf(vreg[i][r][d] * sv, hi, lo, r);
        *reinterpret_cast<H4v*>(vt) = hi;
        *reinterpret_cast<H4v*>(vt + kHd * kVH) = lo;
      }
    }
    __syncthreads();
    if (st + 1 < n_steps) load_step(st + 1);
    // this half's blocks b0 .. b0 + nsb - 1 (uniform per wave)
    const int b0 = kBS * st + kSB * half, nsb = min(kSB, n_blocks - b0);
    if (nsb <= 0) continue;
    // transposed scores of two 16-key tiles per block, one chain each over
    // the four 32-dimension chunks (three products per chunk)
    float sv[kSB][2][4];
    float bm = -__builtin_inff();
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) {
      if (sb >= nsb) {
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
#pragma unroll
          for (int e = 0; e < 4; ++e) sv[sb][jt][e] = -__builtin_inff();
        continue;
      }
      const _Float16* ks = kv + (kSB * half + sb) * kKbH;
      F4v c[2];
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) c[jt] = F4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          const _Float16* kr = ks + (16 * jt + c16) * kKH + 32 * ch + 8 * kg;
          const H8v kh = *reinterpret_cast<const H8v*>(kr), kl = *reinterpret_cast<const H8v*>(kr + kKB * kKH);
          c[jt] = Mfma16x3(kh, kl, qh[ch], ql[ch], c[jt]);
        }
      }
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const F4v ki = *reinterpret_cast<const F4v*>(&kinv[kSB * half + sb][16 * jt + 4 * kg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = (b0 + sb) * kKB + 16 * jt + 4 * kg + e;
          sv[sb][jt][e] = key <= tmax ? c[jt][e] * (qinv * ki[e]) : -__builtin_inff();
          bm = fmaxf(bm, sv[sb][jt][e]);
        }
      }
    }
    // online softmax of this lane's query: its 32 keys of a block sit in
    // the four lanes 16 apart
    bm = lanes::MaxXor16(bm);
    bm = lanes::MaxXor32(bm);
    // the odd half can have seen no visible key yet (all masked): it keeps
    // m = -inf, l = 0 and a zero output
    const float mn = fmaxf(m, bm);
    const bool none = mn == -__builtin_inff();
    const float alpha = none ? 1.0f : ExpSoft(m - mn);
    m = mn;
    H8v ph[kSB], pl[kSB];
    float rs = 0.0f;
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = none ? 0.0f : ExpSoft(sv[sb][jt][e] - mn);
          rs += p;
          SplitHalf(p, ph[sb], pl[sb], 4 * jt + e);
        }
    // (each pair of lanes adds the same two values, so the four lanes hold
    // the same bits)
    rs = lanes::AddXor16(rs);
    rs = lanes::AddXor32(rs);
    l = __builtin_fmaf(l, alpha, rs);
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) o[ct] *= alpha;
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) {
      if (sb >= nsb) continue;
      const _Float16* vt = kv + kBS * kKbH + (kSB * half + sb) * kVbH;
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        const _Float16* vr = vt + (16 * ct + c16) * kVH + 8 * kg;
        const H8v vh = *reinterpret_cast<const H8v*>(vr), vl = *reinterpret_cast<const H8v*>(vr + kHd * kVH);
        // this block's product, scaled back per dimension 16 ct + 4 kg + e
        const F4v ob = Mfma16x3(vh, vl, ph[sb], pl[sb], F4v{0.f, 0.f, 0.f, 0.f});
        const F4v vi = *reinterpret_cast<const F4v*>(&vinv[kSB * half + sb][16 * ct + 4 * kg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[ct][e] = __builtin_fmaf(ob[e], vi[e], o[ct][e]);
      }
    }
  }
  // merge the odd half into the even one through the K/V region: first the
  // query states (m, l), then the outputs in two rounds of four column tiles
  float* const kvf = reinterpret_cast<float*>(kv);
  float* xm = kvf + (qt * G + hg) * 64 * 2;  // [lane][m, l] of head hg, query tile qt
  float f0 = 0.0f, f1 = 0.0f;
  __syncthreads();
  if (half == 1) xm[lane * 2] = m, xm[lane * 2 + 1] = l;
  __syncthreads();
  if (half == 0) {
    const float m1 = xm[lane * 2], l1 = xm[lane * 2 + 1];
    const float mn = fmaxf(m, m1);
    f0 = ExpSoft(m - mn);
    f1 = ExpSoft(m1 - mn);
    l = __builtin_fmaf(l, f0, l1 * f1);
  }
  float* xo = kvf + QT * G * 64 * 2 + (qt * G + hg) * 64 * 16;  // [lane][4 tiles x 4 dimensions]
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    __syncthreads();
    if (half == 1) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) xo[lane * 16 + 4 * q + e] = o[4 * r + q][e];
    }
    __syncthreads();
    if (half == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[4 * r + q][e] = __builtin_fmaf(o[4 * r + q][e], f0, xo[lane * 16 + 4 * q + e] * f1);
    }
  }
  if (half != 0) return;
  const int t = t0 + c16;
  if (t >= a.seq) return;
  float* out = a.out + (static_cast<int64_t>(t) * a.n_heads + h) * kHd + 4 * kg;
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
    *reinterpret_cast<float4*>(out + 16 * ct) = make_float4(o[ct][0] / l, o[ct][1] / l, o[ct][2] / l, o[ct][3] / l);
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
    RPG_CHECK(a.pos0_host >= 0 && n_keys_max <= a.max_seq, "attention past the cache capacity");
    const dim3 grid(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(CeilDiv(a.seq, kQB)));
    // long segments at G <= 2: two query tiles per workgroup (half the
    // workgroups, each staged K/V block read by twice the queries)
    const bool wide = a.seq >= kWideQueries && CeilDiv(a.seq, 2 * kQB) * a.n_kv >= 256;
    const dim3 grid2(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(CeilDiv(a.seq, 2 * kQB)));
    switch (a.n_heads / a.n_kv) {
      case 1:
        if (wide)
          hipLaunchKernelGGL((PrefillKernel<1, 2>), grid2, dim3(256), 0, s, a);
        else
          hipLaunchKernelGGL((PrefillKernel<1, 1>), grid, dim3(128), 0, s, a);
        break;
      case 2:
        if (wide)
          hipLaunchKernelGGL((PrefillKernel<2, 2>), grid2, dim3(512), 0, s, a);
        else
          hipLaunchKernelGGL((PrefillKernel<2, 1>), grid, dim3(256), 0, s, a);
        break;
      case 3: hipLaunchKernelGGL((PrefillKernel<3, 1>), grid, dim3(384), 0, s, a); break;
      case 4: hipLaunchKernelGGL((PrefillKernel<4, 1>), grid, dim3(512), 0, s, a); break;
      case 5: hipLaunchKernelGGL((PrefillKernel<5, 1>), grid, dim3(640), 0, s, a); break;
      case 6: hipLaunchKernelGGL((PrefillKernel<6, 1>), grid, dim3(768), 0, s, a); break;
      case 7: hipLaunchKernelGGL((PrefillKernel<7, 1>), grid, dim3(896), 0, s, a); break;
      default: hipLaunchKernelGGL((PrefillKernel<8, 1>), grid, dim3(1024), 0, s, a); break;
    }
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
