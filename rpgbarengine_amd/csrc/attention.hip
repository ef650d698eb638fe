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
// Prefill (several queries): workgroup (kv head, 16 queries) with one wave
// per query head of the group, scores and P.V on the fp32 matrix cores, K/V
// blocks of 32 positions staged once for the group, online softmax.

#include <hip/hip_runtime.h>

#include "common.h"
#include "expf_glibc.h"
#include "kernels.h"
#include "lanes.h"

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
// judged within 1e-3 of max|logit|). Operands must lie below the f16 range
// limit (65504).
//
// MFMA 16x16x32 f16 lane layout: A[i][k] in lane i + 16 (k / 8), element
// k % 8; B[k][j] in lane j + 16 (k / 8); C[4 (l / 16) + e][l % 16] in element
// e of lane l. A score tile's 32-dimension chunk c gives lane group g the
// dimensions 32 c + 8 g .. + 7 of its query and of its key; P.V gives lane
// group g the keys 8 g .. + 7.
constexpr int kQB = 16;        // queries per workgroup
constexpr int kKB = 32;        // keys per block
constexpr int kKH = kHd + 8;   // K row in LDS (halfs)
constexpr int kVH = kKB + 8;   // V^T row in LDS (halfs)
constexpr int kPS = kKB + 4;   // P row in LDS (floats)

typedef float F4v __attribute__((ext_vector_type(4)));
typedef _Float16 H4v __attribute__((ext_vector_type(4)));
typedef _Float16 H8v __attribute__((ext_vector_type(8)));

// exp(x) for x <= 0 as the hardware 2^y at y = x log2(e): the product's
// rounding moves the result by at most |x| 2^-24 relative (under 1.2e-6 for
// x >= -20; below that exp(x) < 2.1e-9 of the row's largest term), where
// glibc's expf would cost a table load and double arithmetic per call.
__device__ __forceinline__ float ExpSoft(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

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
// and odd) and merge their online-softmax states at the end, so a workgroup
// has 2 G waves.
template <int G>
__global__ __launch_bounds__(128 * G) void PrefillKernel(AttnArgs a) {
  constexpr int nt = 128 * G;
  // halfs of one K block ([hi, lo][key][dimension]) and of one V^T block
  // ([hi, lo][dimension][key])
  constexpr int kKbH = 2 * kKB * kKH, kVbH = 2 * kHd * kVH;
  // two K and two V^T blocks; reused at the end for the merge exchange
  __shared__ __align__(16) _Float16 kv[2 * (kKbH + kVbH)];
  __shared__ __align__(16) float ps[2 * G][kQB][kPS];
  // the longest query blocks (most keys) are dispatched first
  const int kh = blockIdx.x, qb = static_cast<int>(gridDim.y - 1 - blockIdx.y);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int hg = w % G, half = w / G;  // head within the group, key half
  const int h = kh * G + hg;
  const int c16 = lane & 15, kg = lane >> 4;
  const int pos0 = a.pos0_host;
  const int t0 = qb * kQB;
  const int t_last = min(t0 + kQB, a.seq) - 1;
  const int n_keys = pos0 + t_last + 1;  // keys the block's last query sees
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHd));
  // rows r = 4 kg + e of this lane's accumulators: query t0 + r (clamped)
  int tmax[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) tmax[e] = pos0 + min(t0 + 4 * kg + e, a.seq - 1);
  F4v o[8];
#pragma unroll
  for (int ct = 0; ct < 8; ++ct) o[ct] = F4v{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) m[e] = -__builtin_inff(), l[e] = 0.0f;
  const float* kb = a.kcache + static_cast<int64_t>(kh) * a.max_seq * kHd;
  const float* vb = a.vcache + static_cast<int64_t>(kh) * a.max_seq * kHd;
  const int n_blocks = (n_keys + kKB - 1) / kKB;
  const int n_steps = (n_blocks + 1) / 2;
  // step i stages blocks 2i and 2i + 1: K as float4 units u = block
  // (u / 1024), key ((u / 32) % 32), column (u % 32) (32 lanes read one key
  // row and write it contiguously); V as units of 4 keys x
  // 4 dimensions u = block (u / 256), key quad (u % 8), column ((u / 8) %
  // 32), so that a thread writes 4 consecutive keys of a V^T row and 8
  // consecutive lanes one 64-byte run of it (no bank conflicts); thread tid
  // takes u = tid + i * nt. Keys past the last visible one repeat it (masked
  // below). The next step's loads are in flight while the current one is
  // multiplied.
  constexpr int kKUnits = 2 * kKB * (kHd / 4), kVUnits = 2 * (kKB / 4) * (kHd / 4);
  constexpr int kKPer = (kKUnits + nt - 1) / nt, kVPer = (kVUnits + nt - 1) / nt;
  // (native vectors: copies of HIP's float4 class stay memcpys that can keep
  // the registers in scratch memory)
  F4v kreg[kKPer], vreg[kVPer][4];
  auto load_step = [&](int st) {
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      const int u = min(tid + i * nt, kKUnits - 1), c4 = u & 31, j = (u >> 5) & (kKB - 1), bb = u >> 10;
      const int64_t row = static_cast<int64_t>(min((2 * st + bb) * kKB + j, n_keys - 1)) * kHd;
      kreg[i] = *(const __attribute__((address_space(1))) F4v*)(kb + row + 4 * c4);
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int u = min(tid + i * nt, kVUnits - 1), jq = u & 7, c4 = (u >> 3) & 31, bb = u >> 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = static_cast<int64_t>(min((2 * st + bb) * kKB + 4 * jq + r, n_keys - 1)) * kHd;
        vreg[i][r] = *(const __attribute__((address_space(1))) F4v*)(vb + row + 4 * c4);
      }
    }
  };
  load_step(0);
  // (after the first K/V loads, so that both round trips overlap)
  // this lane's query row c16 (clamped past the segment: computed, not
  // stored), dimensions 32 c + 8 kg .. + 7 of chunk c, split hi + lo
  H8v qh[4], ql[4];
  {
    const int tq = min(t0 + c16, a.seq - 1);
    const float* qrow = a.q + (static_cast<int64_t>(tq) * a.n_heads + h) * kHd + 8 * kg;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v0 = *reinterpret_cast<const float4*>(qrow + 32 * c);
      const float4 v1 = *reinterpret_cast<const float4*>(qrow + 32 * c + 4);
      const float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) SplitHalf(x[i], qh[c], ql[c], i);
    }
  }
  for (int st = 0; st < n_steps; ++st) {
    __syncthreads();  // the previous step's LDS reads are done
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      const int u = tid + i * nt, c4 = u & 31, j = (u >> 5) & (kKB - 1), bb = u >> 10;
      if (kKUnits % nt != 0 && u >= kKUnits) break;
      _Float16* ks = kv + bb * kKbH + j * kKH + 4 * c4;
      H4v hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) SplitHalf(kreg[i][e], hi, lo, e);
      *reinterpret_cast<H4v*>(ks) = hi;
      *reinterpret_cast<H4v*>(ks + kKB * kKH) = lo;
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int u = tid + i * nt, jq = u & 7, c4 = (u >> 3) & 31, bb = u >> 8;
      if (kVUnits % nt != 0 && u >= kVUnits) break;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        _Float16* vt = kv + 2 * kKbH + bb * kVbH + (4 * c4 + d) * kVH + 4 * jq;
        H4v hi, lo;
#pragma unroll
        for (int r = 0; r < 4; ++r) SplitHalf(vreg[i][r][d], hi, lo, r);
        *reinterpret_cast<H4v*>(vt) = hi;
        *reinterpret_cast<H4v*>(vt + kHd * kVH) = lo;
      }
    }
    __syncthreads();
    if (st + 1 < n_steps) load_step(st + 1);
    const int blk = 2 * st + half;
    if (blk >= n_blocks) continue;  // this half has no block this step (uniform per wave)
    const int j0 = blk * kKB;
    const _Float16* ks = kv + half * kKbH;
    const _Float16* vt = kv + 2 * kKbH + half * kVbH;
    // scores of two 16-key tiles, one chain each over the four 32-dimension
    // chunks (three products per chunk)
    F4v c[2];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) c[jt] = F4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const _Float16* kr = ks + (16 * jt + c16) * kKH + 32 * ch + 8 * kg;
        const H8v kh = *reinterpret_cast<const H8v*>(kr), kl = *reinterpret_cast<const H8v*>(kr + kKB * kKH);
        c[jt] = Mfma16x3(qh[ch], ql[ch], kh, kl, c[jt]);
      }
    }
    float sv[2][4];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      const F4v cs = c[jt];
      const int key = j0 + 16 * jt + c16;
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[jt][e] = key <= tmax[e] ? cs[e] * scale : -__builtin_inff();
    }
    // online softmax per row: the 16 lanes of a lane group hold the row
    float p[2][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float bm = fmaxf(sv[0][e], sv[1][e]);
      bm = fmaxf(bm, lanes::DppF<lanes::kQuadXor1>(bm));
      bm = fmaxf(bm, lanes::DppF<lanes::kQuadXor2>(bm));
      bm = fmaxf(bm, lanes::DppF<lanes::kRowHalfMirror>(bm));
      bm = fmaxf(bm, lanes::DppF<lanes::kRowMirror>(bm));
      // a row of the odd half can have seen no visible key yet (all masked):
      // it keeps m = -inf, l = 0 and a zero output
      const float mn = fmaxf(m[e], bm);
      const bool none = mn == -__builtin_inff();
      const float alpha = none ? 1.0f : ExpSoft(m[e] - mn);
      m[e] = mn;
      p[0][e] = none ? 0.0f : ExpSoft(sv[0][e] - mn);
      p[1][e] = none ? 0.0f : ExpSoft(sv[1][e] - mn);
      // (the butterfly pairs equal partial sums, so all 16 lanes hold the
      // same bits)
      float rs = p[0][e] + p[1][e];
      rs += lanes::DppF<lanes::kQuadXor1>(rs);
      rs += lanes::DppF<lanes::kQuadXor2>(rs);
      rs += lanes::DppF<lanes::kRowHalfMirror>(rs);
      rs += lanes::DppF<lanes::kRowMirror>(rs);
      l[e] = __builtin_fmaf(l[e], alpha, rs);
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) o[ct][e] *= alpha;
    }
    // P to the A layout through this wave's own LDS rows (one wave's LDS
    // accesses complete in order; the fence keeps the compiler from
    // reordering them)
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int e = 0; e < 4; ++e) ps[w][4 * kg + e][16 * jt + c16] = p[jt][e];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    H8v ph, pl;
    {
      const float4* pr = reinterpret_cast<const float4*>(&ps[w][c16][8 * kg]);
      const float4 p0 = pr[0], p1 = pr[1];
      const float x[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) SplitHalf(x[i], ph, pl, i);
    }
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      const _Float16* vr = vt + (16 * ct + c16) * kVH + 8 * kg;
      const H8v vh = *reinterpret_cast<const H8v*>(vr), vl = *reinterpret_cast<const H8v*>(vr + kHd * kVH);
      o[ct] = Mfma16x3(ph, pl, vh, vl, o[ct]);
    }
  }
  // merge the odd half into the even one through the K/V region: first the
  // row states (m, l), then the outputs in two rounds of four column tiles
  float* const kvf = reinterpret_cast<float*>(kv);
  float* xm = kvf + hg * 64 * 8;  // [lane][m 0..3, l 0..3] of head hg
  float f0[4], f1[4];
  __syncthreads();
  if (half == 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) xm[lane * 8 + e] = m[e], xm[lane * 8 + 4 + e] = l[e];
  }
  __syncthreads();
  if (half == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float m1 = xm[lane * 8 + e], l1 = xm[lane * 8 + 4 + e];
      const float mn = fmaxf(m[e], m1);
      f0[e] = ExpSoft(m[e] - mn);
      f1[e] = ExpSoft(m1 - mn);
      l[e] = __builtin_fmaf(l[e], f0[e], l1 * f1[e]);
    }
  }
  float* xo = kvf + G * 64 * 8 + hg * 64 * 16;  // [lane][4 tiles x 4 rows] of head hg
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
        for (int e = 0; e < 4; ++e)
          o[4 * r + q][e] = __builtin_fmaf(o[4 * r + q][e], f0[e], xo[lane * 16 + 4 * q + e] * f1[e]);
    }
  }
  if (half != 0) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = t0 + 4 * kg + e;
    if (t >= a.seq) continue;
    float* out = a.out + (static_cast<int64_t>(t) * a.n_heads + h) * kHd + c16;
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) out[16 * ct] = o[ct][e] / l[e];
  }
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
    switch (a.n_heads / a.n_kv) {
      case 1: hipLaunchKernelGGL(PrefillKernel<1>, grid, dim3(128), 0, s, a); break;
      case 2: hipLaunchKernelGGL(PrefillKernel<2>, grid, dim3(256), 0, s, a); break;
      case 3: hipLaunchKernelGGL(PrefillKernel<3>, grid, dim3(384), 0, s, a); break;
      case 4: hipLaunchKernelGGL(PrefillKernel<4>, grid, dim3(512), 0, s, a); break;
      case 5: hipLaunchKernelGGL(PrefillKernel<5>, grid, dim3(640), 0, s, a); break;
      case 6: hipLaunchKernelGGL(PrefillKernel<6>, grid, dim3(768), 0, s, a); break;
      case 7: hipLaunchKernelGGL(PrefillKernel<7>, grid, dim3(896), 0, s, a); break;
      default: hipLaunchKernelGGL(PrefillKernel<8>, grid, dim3(1024), 0, s, a); break;
    }
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
