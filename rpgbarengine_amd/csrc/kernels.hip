// gfx950 kernels of the Qwen3 token loop: fused dequant matvec, exact
// dequant/gather, RMSNorm, QK-norm + RoPE + KV-cache write, argmax.
//
// Wave64 throughout. The matvec gives one wavefront per output row: the 64
// lanes stride over the row's 32-weight units (quant_dev.h), so a wave streams
// its row's raw GGUF bytes contiguously, decodes in registers, and reduces the
// dot with a butterfly over the wave. Up to 8 tokens share one weight decode.

#include <hip/hip_runtime.h>

#include "common.h"
#include "decode.h"
#include "expf_glibc.h"
#include "kernels.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float WaveSum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ double WaveSumD(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// 32 activations of unit u (the element pattern of quant_dev.h Unit<T>).
template <uint32_t T>
__device__ __forceinline__ void LoadX(const float* x, int u, float* xv) {
  if constexpr (T == 12) {  // Q4_K: two runs of 16
    const int b = u >> 3, g = (u >> 1) & 3, h = u & 1;
    const float4* p = reinterpret_cast<const float4*>(x + 256 * b + 64 * g + 16 * h);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 lo = p[c], hi = p[8 + c];
      xv[4 * c] = lo.x; xv[4 * c + 1] = lo.y; xv[4 * c + 2] = lo.z; xv[4 * c + 3] = lo.w;
      xv[16 + 4 * c] = hi.x; xv[16 + 4 * c + 1] = hi.y; xv[16 + 4 * c + 2] = hi.z; xv[16 + 4 * c + 3] = hi.w;
    }
  } else if constexpr (T == 14) {  // Q6_K: four runs of 8, 32 apart
    const int b = u >> 3, half = (u >> 2) & 1, j = u & 3;
    const float* base = x + 256 * b + 128 * half + 8 * j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float4 a = *reinterpret_cast<const float4*>(base + 32 * r);
      const float4 c = *reinterpret_cast<const float4*>(base + 32 * r + 4);
      xv[8 * r] = a.x; xv[8 * r + 1] = a.y; xv[8 * r + 2] = a.z; xv[8 * r + 3] = a.w;
      xv[8 * r + 4] = c.x; xv[8 * r + 5] = c.y; xv[8 * r + 6] = c.z; xv[8 * r + 7] = c.w;
    }
  } else {  // Q8_0, F32: 32 consecutive
    const float4* p = reinterpret_cast<const float4*>(x + 32 * u);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float4 v = p[c];
      xv[4 * c] = v.x; xv[4 * c + 1] = v.y; xv[4 * c + 2] = v.z; xv[4 * c + 3] = v.w;
    }
  }
}

// acc[m] += row . X[m] over this lane's units.
template <uint32_t T, int M>
__device__ __forceinline__ void RowDotLanes(const uint8_t* row, int cols, const float* X, int64_t ldx, int mcount,
                                            int lane, float* acc) {
  const int units = cols >> 5;
  for (int u = lane; u < units; u += kWave) {
    float w[32];
    dev::Unit<T>::Decode(row, u, w);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (m < mcount) {
        float xv[32];
        LoadX<T>(X + m * ldx, u, xv);
        float s = acc[m];
#pragma unroll
        for (int i = 0; i < 32; ++i) s = __builtin_fmaf(xv[i], w[i], s);
        acc[m] = s;
      }
    }
  }
}

template <uint32_t T, int M>
__global__ __launch_bounds__(256) void MatvecKernel(const uint8_t* __restrict__ W, int rows, int cols,
                                                    int64_t row_bytes, const float* __restrict__ X, int64_t ldx,
                                                    int mcount, float* __restrict__ Y, int64_t ldy, int epi) {
  const int lane = threadIdx.x & (kWave - 1);
  const int r = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  RowDotLanes<T, M>(W + static_cast<int64_t>(r) * row_bytes, cols, X, ldx, mcount, lane, acc);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (m < mcount) {
      const float v = WaveSum(acc[m]);
      if (lane == 0) {
        float* y = Y + m * ldy + r;
        *y = epi == kAdd ? *y + v : v;
      }
    }
  }
}

template <uint32_t TG, uint32_t TU, int M>
__global__ __launch_bounds__(256) void SwiGLUKernel(const uint8_t* __restrict__ G, int64_t g_row_bytes,
                                                    const uint8_t* __restrict__ U, int64_t u_row_bytes, int rows,
                                                    int cols, const float* __restrict__ X, int64_t ldx, int mcount,
                                                    float* __restrict__ Y, int64_t ldy) {
  const int lane = threadIdx.x & (kWave - 1);
  const int r = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float ag[M], au[M];
#pragma unroll
  for (int m = 0; m < M; ++m) ag[m] = au[m] = 0.0f;
  RowDotLanes<TG, M>(G + static_cast<int64_t>(r) * g_row_bytes, cols, X, ldx, mcount, lane, ag);
  RowDotLanes<TU, M>(U + static_cast<int64_t>(r) * u_row_bytes, cols, X, ldx, mcount, lane, au);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (m < mcount) {
      const float g = WaveSum(ag[m]);
      const float u = WaveSum(au[m]);
      if (lane == 0) {
        // silu(g) = g / (1 + expf(-g)), then * up (reference src/kernels.h:82-92)
        const float sg = g / __fadd_rn(1.0f, GlibcExpf(-g));
        Y[m * ldy + r] = __fmul_rn(sg, u);
      }
    }
  }
}

// The other ggml types (Q4_0 .. Q8_K but Q8_0 / Q4_K / Q6_K, F16, BF16): the
// lane's 32-weight units dequantised exactly (quant_dev.h DequantUnit, the
// reference's DequantizeRow values) and dotted with the activations in
// fp32 -- the reference's DotRowQuantRef (src/matmul.cc:73-102) up to
// summation order. Weight type read at run time: one kernel for all.
template <int M>
__device__ __forceinline__ void RowDotAny(uint32_t type, const uint8_t* row, int cols, const float* X, int64_t ldx,
                                          int mcount, int lane, float* acc) {
  const int units = cols >> 5;
  for (int u = lane; u < units; u += kWave) {
    float w[32];
    dev::DequantUnit(type, row, u, w);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (m < mcount) {
        const float4* p = reinterpret_cast<const float4*>(X + m * ldx + 32 * u);
        float s = acc[m];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float4 v = p[c];
          s = __builtin_fmaf(v.x, w[4 * c], s);
          s = __builtin_fmaf(v.y, w[4 * c + 1], s);
          s = __builtin_fmaf(v.z, w[4 * c + 2], s);
          s = __builtin_fmaf(v.w, w[4 * c + 3], s);
        }
        acc[m] = s;
      }
    }
  }
}

template <int M>
__global__ __launch_bounds__(256) void MatvecAnyKernel(uint32_t type, const uint8_t* __restrict__ W, int rows,
                                                       int cols, int64_t row_bytes, const float* __restrict__ X,
                                                       int64_t ldx, int mcount, float* __restrict__ Y, int64_t ldy,
                                                       int epi) {
  const int lane = threadIdx.x & (kWave - 1);
  const int r = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  RowDotAny<M>(type, W + static_cast<int64_t>(r) * row_bytes, cols, X, ldx, mcount, lane, acc);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (m < mcount) {
      const float v = WaveSum(acc[m]);
      if (lane == 0) {
        float* y = Y + m * ldy + r;
        *y = epi == kAdd ? *y + v : v;
      }
    }
  }
}

template <int M>
__global__ __launch_bounds__(256) void SwiGLUAnyKernel(uint32_t tg, const uint8_t* __restrict__ G, int64_t g_row_bytes,
                                                       uint32_t tu, const uint8_t* __restrict__ U, int64_t u_row_bytes,
                                                       int rows, int cols, const float* __restrict__ X, int64_t ldx,
                                                       int mcount, float* __restrict__ Y, int64_t ldy) {
  const int lane = threadIdx.x & (kWave - 1);
  const int r = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  float ag[M], au[M];
#pragma unroll
  for (int m = 0; m < M; ++m) ag[m] = au[m] = 0.0f;
  RowDotAny<M>(tg, G + static_cast<int64_t>(r) * g_row_bytes, cols, X, ldx, mcount, lane, ag);
  RowDotAny<M>(tu, U + static_cast<int64_t>(r) * u_row_bytes, cols, X, ldx, mcount, lane, au);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (m < mcount) {
      const float g = WaveSum(ag[m]);
      const float u = WaveSum(au[m]);
      if (lane == 0) {
        // silu(g) = g / (1 + expf(-g)), then * up (reference src/kernels.h:82-92)
        const float sg = g / __fadd_rn(1.0f, GlibcExpf(-g));
        Y[m * ldy + r] = __fmul_rn(sg, u);
      }
    }
  }
}

void LaunchMatvecAny(const MatRef& W, const float* X, int64_t ldx, int M, float* Y, int64_t ldy, Epilogue epi,
                     hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(CeilDiv(W.rows, 4))), block(256);
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    const float* Xm = X + m0 * ldx;
    float* Ym = Y + m0 * ldy;
    if (mc == 1)
      hipLaunchKernelGGL((MatvecAnyKernel<1>), grid, block, 0, s, W.type, W.w, W.rows, W.cols, W.row_bytes, Xm, ldx,
                         mc, Ym, ldy, static_cast<int>(epi));
    else
      hipLaunchKernelGGL((MatvecAnyKernel<8>), grid, block, 0, s, W.type, W.w, W.rows, W.cols, W.row_bytes, Xm, ldx,
                         mc, Ym, ldy, static_cast<int>(epi));
  }
}

void LaunchSwiGLUAny(const MatRef& G, const MatRef& U, const float* X, int64_t ldx, int M, float* Y, int64_t ldy,
                     hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(CeilDiv(G.rows, 4))), block(256);
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    const float* Xm = X + m0 * ldx;
    float* Ym = Y + m0 * ldy;
    if (mc == 1)
      hipLaunchKernelGGL((SwiGLUAnyKernel<1>), grid, block, 0, s, G.type, G.w, G.row_bytes, U.type, U.w, U.row_bytes,
                         G.rows, G.cols, Xm, ldx, mc, Ym, ldy);
    else
      hipLaunchKernelGGL((SwiGLUAnyKernel<8>), grid, block, 0, s, G.type, G.w, G.row_bytes, U.type, U.w, U.row_bytes,
                         G.rows, G.cols, Xm, ldx, mc, Ym, ldy);
  }
}

template <uint32_t T>
void LaunchMatvecT(const MatRef& W, const float* X, int64_t ldx, int M, float* Y, int64_t ldy, Epilogue epi,
                   hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(CeilDiv(W.rows, 4))), block(256);
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    const float* Xm = X + m0 * ldx;
    float* Ym = Y + m0 * ldy;
    if (mc == 1)
      hipLaunchKernelGGL((MatvecKernel<T, 1>), grid, block, 0, s, W.w, W.rows, W.cols, W.row_bytes, Xm, ldx, mc, Ym,
                         ldy, static_cast<int>(epi));
    else if (mc <= 4)
      hipLaunchKernelGGL((MatvecKernel<T, 4>), grid, block, 0, s, W.w, W.rows, W.cols, W.row_bytes, Xm, ldx, mc, Ym,
                         ldy, static_cast<int>(epi));
    else
      hipLaunchKernelGGL((MatvecKernel<T, 8>), grid, block, 0, s, W.w, W.rows, W.cols, W.row_bytes, Xm, ldx, mc, Ym,
                         ldy, static_cast<int>(epi));
  }
}

template <uint32_t TG, uint32_t TU>
void LaunchSwiGLUT(const MatRef& G, const MatRef& U, const float* X, int64_t ldx, int M, float* Y, int64_t ldy,
                   hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(CeilDiv(G.rows, 4))), block(256);
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    const float* Xm = X + m0 * ldx;
    float* Ym = Y + m0 * ldy;
    if (mc == 1)
      hipLaunchKernelGGL((SwiGLUKernel<TG, TU, 1>), grid, block, 0, s, G.w, G.row_bytes, U.w, U.row_bytes, G.rows,
                         G.cols, Xm, ldx, mc, Ym, ldy);
    else if (mc <= 4)
      hipLaunchKernelGGL((SwiGLUKernel<TG, TU, 4>), grid, block, 0, s, G.w, G.row_bytes, U.w, U.row_bytes, G.rows,
                         G.cols, Xm, ldx, mc, Ym, ldy);
    else
      hipLaunchKernelGGL((SwiGLUKernel<TG, TU, 8>), grid, block, 0, s, G.w, G.row_bytes, U.w, U.row_bytes, G.rows,
                         G.cols, Xm, ldx, mc, Ym, ldy);
  }
}

template <uint32_t TG>
void LaunchSwiGLUU(const MatRef& G, const MatRef& U, const float* X, int64_t ldx, int M, float* Y, int64_t ldy,
                   hipStream_t s) {
  switch (U.type) {
    case kQ4_K: LaunchSwiGLUT<TG, 12>(G, U, X, ldx, M, Y, ldy, s); return;
    case kQ6_K: LaunchSwiGLUT<TG, 14>(G, U, X, ldx, M, Y, ldy, s); return;
    case kQ8_0: LaunchSwiGLUT<TG, 8>(G, U, X, ldx, M, Y, ldy, s); return;
    case kF32: LaunchSwiGLUT<TG, 0>(G, U, X, ldx, M, Y, ldy, s); return;
    default: Throw("SwiGLU: unsupported up type %s", TypeName(U.type));
  }
}

// ---------------------------------------------------------------- exact dequant / gather

__global__ void DequantKernel(uint32_t type, const uint8_t* __restrict__ src, int64_t n, float* __restrict__ dst) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) dst[i] = dev::DequantExact(type, src, i);
}

__global__ void GatherKernel(uint32_t type, const uint8_t* __restrict__ W, int rows, int cols, int64_t row_bytes,
                             const int32_t* __restrict__ ids, float* __restrict__ out, int64_t ldo,
                             int32_t* __restrict__ err, int32_t* rec_ids, int32_t* rec_step, int64_t rec_ld) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  int32_t id = ids[t];
  if (rec_ids != nullptr && c == 0) {
    if (rec_ld > 0) {
      rec_ids[t * rec_ld + *rec_step] = id;  // the step advances in a later launch
    } else if (t == 0) {
      const int st = *rec_step;
      rec_ids[st] = id;
      *rec_step = st + 1;
    }
  }
  if (id < 0 || id >= rows) {
    if (c == 0 && err) *err = 1;
    id = 0;
  }
  if (c < cols) out[t * ldo + c] = dev::DequantExact(type, W + static_cast<int64_t>(id) * row_bytes, c);
}

// ---------------------------------------------------------------- RMSNorm

// One 256-thread block per row. Sum of squares in double (exact squares),
// scale = float(1 / sqrt(mean + eps)), out = (x * scale) * w.
__global__ __launch_bounds__(256) void RmsNormKernel(const float* __restrict__ x, int64_t ldx,
                                                     const float* __restrict__ w, int n, float eps,
                                                     float* __restrict__ out, int64_t ldo) {
  const float* xr = x + blockIdx.x * ldx;
  float* orow = out + blockIdx.x * ldo;
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const double v = xr[i];
    s += v * v;
  }
  s = WaveSumD(s);
  __shared__ double part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const double total = (part[0] + part[1]) + (part[2] + part[3]);
  const double mean = total / static_cast<double>(n);
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(mean + static_cast<double>(eps)));
  for (int i = threadIdx.x; i < n; i += blockDim.x) orow[i] = __fmul_rn(__fmul_rn(xr[i], scale), w[i]);
}

// ---------------------------------------------------------------- QK-norm + RoPE + cache

// grid (n_heads + n_kv, seq), 64 threads: lane i holds the RoPE pair (i, i + hd/2)
// for hd = 128.
__global__ __launch_bounds__(64) void QkNormRopeKernel(QkvArgs a) {
  const int t = blockIdx.y;
  const int hidx = blockIdx.x;
  const int i = threadIdx.x;
  const int half = a.hd >> 1;
  const int pos = (a.pos0_dev ? *a.pos0_dev : a.pos0_host) + t;
  const bool is_q = hidx < a.n_heads;
  const int head = is_q ? hidx : hidx - a.n_heads;
  const float* src = is_q ? a.q + (static_cast<int64_t>(t) * a.n_heads + head) * a.hd
                          : a.k + (static_cast<int64_t>(t) * a.n_kv + head) * a.hd;
  const float* nw = is_q ? a.q_norm : a.k_norm;
  const float x0 = src[i], x1 = src[i + half];
  double s = static_cast<double>(x0) * x0 + static_cast<double>(x1) * x1;
  s = WaveSumD(s);
  const double mean = s / static_cast<double>(a.hd);
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(mean + static_cast<double>(a.eps)));
  const float na = __fmul_rn(__fmul_rn(x0, scale), nw[i]);
  const float nb = __fmul_rn(__fmul_rn(x1, scale), nw[i + half]);
  const float c = a.rope[static_cast<int64_t>(pos) * a.hd + i];
  const float sn = a.rope[static_cast<int64_t>(pos) * a.hd + half + i];
  // a*c - b*s and b*c + a*s, each product rounded (reference src/kernels.h:108-120)
  const float ra = __fsub_rn(__fmul_rn(na, c), __fmul_rn(nb, sn));
  const float rb = __fadd_rn(__fmul_rn(nb, c), __fmul_rn(na, sn));
  if (is_q) {
    float* dst = a.q + (static_cast<int64_t>(t) * a.n_heads + head) * a.hd;
    dst[i] = ra;
    dst[i + half] = rb;
  } else {
    float* kd = a.kcache + (static_cast<int64_t>(head) * a.max_seq + pos) * a.hd;
    float* vd = a.vcache + (static_cast<int64_t>(head) * a.max_seq + pos) * a.hd;
    const float* vs = a.v + (static_cast<int64_t>(t) * a.n_kv + head) * a.hd;
    kd[i] = ra;
    kd[i + half] = rb;
    vd[i] = vs[i];
    vd[i + half] = vs[i + half];
  }
}

// ---------------------------------------------------------------- argmax

// One 1024-thread block per row; ties resolve to the lowest index, NaN never
// wins (reference strict `>` scan; a NaN first element returns 0). Rows of
// 16-byte aligned floats (vec4) are read as float4, eight loads in flight
// per thread before any comparison (a 151936-logit row is ~37 vectors per
// thread: one dependent load after another took ~57 us).
__device__ __forceinline__ void ArgMaxTake(float v, int i, float& bv, int& bi) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__global__ __launch_bounds__(1024) void ArgMaxKernel(const float* __restrict__ x, int64_t ldx, int n, int vec4,
                                                     int32_t* __restrict__ out) {
  const float* xr = x + blockIdx.x * ldx;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  const int tid = static_cast<int>(threadIdx.x), nt = static_cast<int>(blockDim.x);
  int tail = 0;
  if (vec4) {
    constexpr int kU = 8;
    const int n4 = n >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    for (int base = tid; base < n4; base += nt * kU) {
      float4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = x4[min(base + u * nt, n4 - 1)];  // clamped: loads stay unconditional
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int j = base + u * nt;
        if (j < n4) {
          ArgMaxTake(v[u].x, 4 * j, bv, bi);
          ArgMaxTake(v[u].y, 4 * j + 1, bv, bi);
          ArgMaxTake(v[u].z, 4 * j + 2, bv, bi);
          ArgMaxTake(v[u].w, 4 * j + 3, bv, bi);
        }
      }
    }
    tail = 4 * n4;
  }
  for (int i = tail + tid; i < n; i += nt) ArgMaxTake(xr[i], i, bv, bi);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int idx = si[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) {
      if (sv[w] > v || (sv[w] == v && si[w] < idx)) {
        v = sv[w];
        idx = si[w];
      }
    }
    if (idx == 0x7fffffff || xr[0] != xr[0]) idx = 0;  // all -inf/NaN, or NaN first
    out[blockIdx.x] = idx;
  }
}

// The same pick over many workgroups of one launch (one 4096-logit slice
// each), for one row with a scratch pair (key, count) that starts at zero:
// each workgroup folds its slice into key = order(v) << 32 | ~i (larger
// value, then smaller index, compares larger; NaN never enters) with one
// device-scope atomic max, then counts itself in; the last workgroup to
// count reads the key -- every other workgroup's max was performed before
// its count, the count waiting on the max's returned value -- writes the
// index and clears the pair for the next launch. A key of 0 (every logit
// NaN) and a NaN first logit give index 0, as the reference's strict scan
// does; -0 keys as +0 (the scan's > holds them equal: the first wins).
constexpr int kPickSlice = 4096;

__device__ __forceinline__ unsigned long long PickKey(float v, int i) {
  const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
  const uint32_t ok = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<unsigned long long>(ok) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
}

__global__ __launch_bounds__(256) void ArgMaxSliceKernel(const float* __restrict__ x, int n, int vec4,
                                                         int32_t* __restrict__ out, unsigned long long* pair) {
  const int tid = static_cast<int>(threadIdx.x), i0 = static_cast<int>(blockIdx.x) * kPickSlice;
  const float first = x[0];
  unsigned long long best = 0ull;
  const int m4 = vec4 ? min(kPickSlice, n - i0) >> 2 : 0;
  if (m4 > 0) {
    // four float4 per thread, each load coalesced across the workgroup
    // (clamped into the slice's whole vectors)
    const float4* x4 = reinterpret_cast<const float4*>(x + i0);
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = x4[min(tid + 256 * u, m4 - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = tid + 256 * u, i = i0 + 4 * j;
      if (j < m4) {
        const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (e[q] == e[q]) best = max(best, PickKey(e[q], i + q));
      }
    }
    for (int i = i0 + 4 * m4 + tid; i < min(i0 + kPickSlice, n); i += 256)
      if (x[i] == x[i]) best = max(best, PickKey(x[i], i));
  } else {
    for (int i = i0 + tid; i < min(i0 + kPickSlice, n); i += 256)
      if (x[i] == x[i]) best = max(best, PickKey(x[i], i));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) best = max(best, static_cast<unsigned long long>(__shfl_xor(best, off, kWave)));
  __shared__ unsigned long long wbest[4];
  if ((tid & 63) == 0) wbest[tid >> 6] = best;
  __syncthreads();
  if (tid != 0) return;
  best = max(max(wbest[0], wbest[1]), max(wbest[2], wbest[3]));
  const unsigned long long seen = __hip_atomic_fetch_max(&pair[0], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the count waits on the max's returned value (the max has been performed)
  unsigned long long one = 1ull;
  asm volatile("" : "+v"(one) : "v"(seen));
  const unsigned long long done =
      __hip_atomic_fetch_add(&pair[1], one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (done != gridDim.x - 1) return;
  const unsigned long long key = __hip_atomic_fetch_max(&pair[0], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int idx = key == 0ull ? 0 : static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key));
  out[0] = first != first ? 0 : idx;
  __hip_atomic_store(&pair[0], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&pair[1], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

void Matvec(const MatRef& W, const float* X, int64_t ldx, int M, float* Y, int64_t ldy, Epilogue epi, hipStream_t s) {
  RPG_CHECK(W.cols % 32 == 0, "matvec: %d columns is not a multiple of 32", W.cols);
  RPG_CHECK(ldx % 4 == 0, "matvec: activation stride must be a multiple of 4");
  if (M == 1 && (W.type == kF32 || W.type == kQ8_0 || W.cols % 256 == 0 || !FastType(W.type))) {
    // one token: the decode-step kernel
    DecodeMatvecArgs a;
    a.job[0].w = W.w;
    a.job[0].row_bytes = W.row_bytes;
    a.job[0].type = W.type;
    a.job[0].rows = W.rows;
    a.job[0].y = Y;
    a.x = X;
    a.K = W.cols;
    a.epi = epi;
    DecodeMatvec(a, s);
    return;
  }
  switch (W.type) {
    case kQ4_K: LaunchMatvecT<12>(W, X, ldx, M, Y, ldy, epi, s); break;
    case kQ6_K: LaunchMatvecT<14>(W, X, ldx, M, Y, ldy, epi, s); break;
    case kQ8_0: LaunchMatvecT<8>(W, X, ldx, M, Y, ldy, epi, s); break;
    case kF32: LaunchMatvecT<0>(W, X, ldx, M, Y, ldy, epi, s); break;
    default:
      RPG_CHECK(BlockElems(W.type) > 0, "matvec: unsupported weight type %u", W.type);
      LaunchMatvecAny(W, X, ldx, M, Y, ldy, epi, s);
  }
  HIP_CHECK(hipGetLastError());
}

void MatvecSwiGLU(const MatRef& G, const MatRef& U, const float* X, int64_t ldx, int M, float* Y, int64_t ldy,
                  hipStream_t s) {
  RPG_CHECK(G.rows == U.rows && G.cols == U.cols, "SwiGLU: gate and up shapes differ");
  RPG_CHECK(G.cols % 32 == 0 && ldx % 4 == 0, "SwiGLU: bad column count or stride");
  if (!FastType(G.type) || !FastType(U.type)) {
    RPG_CHECK(BlockElems(G.type) > 0 && BlockElems(U.type) > 0, "SwiGLU: unsupported weight types %u / %u", G.type,
              U.type);
    LaunchSwiGLUAny(G, U, X, ldx, M, Y, ldy, s);
    HIP_CHECK(hipGetLastError());
    return;
  }
  switch (G.type) {
    case kQ4_K: LaunchSwiGLUU<12>(G, U, X, ldx, M, Y, ldy, s); break;
    case kQ6_K: LaunchSwiGLUU<14>(G, U, X, ldx, M, Y, ldy, s); break;
    case kQ8_0: LaunchSwiGLUU<8>(G, U, X, ldx, M, Y, ldy, s); break;
    case kF32: LaunchSwiGLUU<0>(G, U, X, ldx, M, Y, ldy, s); break;
    default: Throw("SwiGLU: unsupported gate type %s", TypeName(G.type));
  }
  HIP_CHECK(hipGetLastError());
}

void GatherRows(const MatRef& W, const int32_t* ids, int n, float* out, int64_t ldo, int32_t* err, hipStream_t s,
                int32_t* rec_ids, int32_t* rec_step, int64_t rec_ld) {
  if (n <= 0) return;
  RPG_CHECK(rec_ids == nullptr || (rec_step != nullptr && (n == 1 || rec_ld > 0)),
            "gather: a token record needs a step, and a row stride for several ids");
  const dim3 grid(static_cast<unsigned>(CeilDiv(W.cols, 256)), static_cast<unsigned>(n));
  hipLaunchKernelGGL(GatherKernel, grid, dim3(256), 0, s, W.type, W.w, W.rows, W.cols, W.row_bytes, ids, out, ldo,
                     err, rec_ids, rec_step, rec_ld);
  HIP_CHECK(hipGetLastError());
}

namespace {
__global__ void AdvanceKernel(int32_t* pos, int n, int32_t* step) {
  const int i = threadIdx.x;
  if (i < n) pos[i] += 1;
  if (i == 0 && step != nullptr) *step += 1;
}
}  // namespace

void AdvancePositions(int32_t* pos, int n, int32_t* step, hipStream_t s) {
  RPG_CHECK(n >= 1 && n <= 1024, "advance: %d positions", n);
  hipLaunchKernelGGL(AdvanceKernel, dim3(1), dim3(static_cast<unsigned>(n)), 0, s, pos, n, step);
  HIP_CHECK(hipGetLastError());
}

namespace {
__global__ void ForceTokensKernel(int32_t* tokens, int n, const int32_t* force, int32_t* drawn, const int32_t* step,
                                  int64_t ld) {
  const int i = threadIdx.x;
  if (i >= n) return;
  const int64_t at = i * ld + *step;
  drawn[at] = tokens[i];
  tokens[i] = force[at];
}
}  // namespace

void ForceTokens(int32_t* tokens, int n, const int32_t* force, int32_t* drawn, const int32_t* step, int64_t ld,
                 hipStream_t s) {
  RPG_CHECK(n >= 1 && n <= 1024 && force && drawn && step, "force: bad arguments");
  hipLaunchKernelGGL(ForceTokensKernel, dim3(1), dim3(static_cast<unsigned>(n)), 0, s, tokens, n, force, drawn, step,
                     ld);
  HIP_CHECK(hipGetLastError());
}

void Dequant(uint32_t type, const uint8_t* src, int64_t n, float* dst, hipStream_t s) {
  RPG_CHECK(BlockElems(type) > 0 && n % BlockElems(type) == 0, "dequant: bad type or length");
  if (n == 0) return;
  hipLaunchKernelGGL(DequantKernel, dim3(static_cast<unsigned>(CeilDiv(n, 256))), dim3(256), 0, s, type, src, n, dst);
  HIP_CHECK(hipGetLastError());
}

void RmsNormRows(const float* x, int64_t ldx, const float* w, int n, int rows, float eps, float* out, int64_t ldo,
                 hipStream_t s) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(RmsNormKernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, x, ldx, w, n, eps, out, ldo);
  HIP_CHECK(hipGetLastError());
}

void QkNormRopeCache(const QkvArgs& a, hipStream_t s) {
  RPG_CHECK(a.hd == 128, "QK-norm/RoPE kernel is built for head_dim 128 (got %d)", a.hd);
  if (a.seq <= 0) return;
  hipLaunchKernelGGL(QkNormRopeKernel, dim3(static_cast<unsigned>(a.n_heads + a.n_kv), static_cast<unsigned>(a.seq)),
                     dim3(64), 0, s, a);
  HIP_CHECK(hipGetLastError());
}

void ArgMaxRows(const float* x, int64_t ldx, int n, int rows, int32_t* out, hipStream_t s, uint64_t* pair) {
  if (rows <= 0) return;
  const int vec4 = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % 4 == 0 ? 1 : 0;
  if (rows == 1 && pair != nullptr) {
    RPG_CHECK(n >= 1, "argmax: empty row");
    hipLaunchKernelGGL(ArgMaxSliceKernel, dim3(static_cast<unsigned>(CeilDiv(n, kPickSlice))), dim3(256), 0, s, x, n,
                       vec4, out, reinterpret_cast<unsigned long long*>(pair));
    HIP_CHECK(hipGetLastError());
    return;
  }
  hipLaunchKernelGGL(ArgMaxKernel, dim3(static_cast<unsigned>(rows)), dim3(1024), 0, s, x, ldx, n, vec4, out);
  HIP_CHECK(hipGetLastError());
}


}  // namespace k
}  // namespace rpg
