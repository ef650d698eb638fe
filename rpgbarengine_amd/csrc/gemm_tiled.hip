// Tiled prefill GEMM for long segments: Q4_K and Q6_K weights dequantised
// once per workgroup into LDS, v_mfma_f32_32x32x16_f16 over 128 tokens x 128
// rows.
//
// The operands are those of prefill.h (exact integer weight operands, token
// rows split into f16 hi + lo, the fp16 block scales applied in fp32), so
// every output meets the same bound. What differs from the 32-token kernels
// is where the work sits:
//  * a step (64 inputs) of the workgroup's 128 weight rows is unpacked once,
//    by all 512 threads (a quarter row each: Q4_K 8 quant bytes -> 16 f16
//    operands q * sc; Q6_K 16 positions of one strip -> 16 operands q - 32
//    with the slice's d * sc in a table), into LDS, and read by the four
//    waves that share those rows; the tokens' hi/lo rows of the step arrive
//    beside them by LDS DMA;
//  * each of the 8 waves owns 32 tokens x 64 rows (two 32 x 32 tiles), so
//    every token operand read from LDS feeds two products and every weight
//    operand two (hi, lo);
//  * Q4_K: the min term sum_j m_j * sum(x in sub-block j) of a super-block
//    is one v_mfma_f32_32x32x8_f16 pair over the 8 sub-blocks (the sums
//    hi/lo as A, the integer mins as B), added with d * P at its end; Q6_K:
//    each 16-input slice's sums are scaled by its d * sc as they are formed.
// One workgroup per compute unit (two waves per SIMD); weight loads run
// three steps ahead in registers, the token rows one step ahead.
//
// MFMA layouts (gfx950): 32x32x16 f16: lane l holds A[l % 32][8 (l / 32) ..
// +8) and B[8 (l / 32) .. +8][l % 32]; 32x32x8 f16 the same with 4 k per
// lane; the 16 results of lane l are C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32],
// v < 16.

#include <hip/hip_runtime.h>

#include "common.h"
#include "expf_glibc.h"
#include "prefill.h"
#include "quant_dev.h"

namespace rpg {
namespace k {

namespace {

typedef _Float16 H2 __attribute__((ext_vector_type(2)));
typedef _Float16 H4 __attribute__((ext_vector_type(4)));
typedef _Float16 H8 __attribute__((ext_vector_type(8)));
typedef float F16v __attribute__((ext_vector_type(16)));
typedef uint32_t U2 __attribute__((ext_vector_type(2)));
typedef uint32_t U4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;      // 8 waves: 4 token tiles of 32 x 2 row halves of 64
constexpr int kTM = kTiledTokens;  // tokens per workgroup
constexpr int kTN = kTiledRows;    // weight rows per workgroup
constexpr int kRow = 64 + 8;       // LDS row of a step: 64 f16 + 8 padding (144 bytes: conflict-free b128 reads)

// 8 bytes at an address that is only 2-byte aligned (Q6_K blocks are 210
// bytes long): one dwordx2 load, which global memory serves at any byte
// alignment.
typedef U2 U2A2 __attribute__((aligned(2)));

template <typename T>
__device__ __forceinline__ T GLoad(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc MakeRsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Chunk swizzle of the token rows in LDS (128-byte rows, 16-byte chunks):
// logical chunk c of row r sits at chunk c ^ ASwz(r). Any 8 consecutive rows
// (from a multiple of 8) use 8 different chunks, and so do the 8 even and the
// 8 odd rows of any 16, so the b128 reads of 32 consecutive rows at one
// logical chunk meet no bank conflict with either 32 or 64 banks.
__device__ __forceinline__ int ASwz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Chunk swizzle of the Q4_K weight rows in LDS (128-byte rows, 16-byte
// chunks): logical chunk c of row r sits at chunk c ^ BSwz(r), BSwz linear
// in the bits of r (bit 0 -> 4, bit 1 -> 5, bit 2 -> 2, bit 3 -> 1). The
// reads (32 consecutive rows at one logical chunk) meet no bank conflict with
// either 32 or 64 banks, as for the token rows; so do the unpacking threads'
// writes (four threads per row write chunks 0..3, then 4..7, of two or four
// consecutive rows at once): bit 2 of BSwz differs between rows 2i and
// 2i + 1, and between rows 4i + j and 4i + j + 2.
__device__ __forceinline__ int BSwz(int r) {
  return ((r & 1) << 2) ^ (((r >> 1) & 1) * 5) ^ (((r >> 2) & 1) << 1) ^ ((r >> 3) & 1);
}

__device__ __forceinline__ uint32_t AsU(H2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ H2 AsH2(uint32_t v) { return __builtin_bit_cast(H2, v); }

__device__ __forceinline__ uint32_t HalfPair(float v) {
  const _Float16 h = static_cast<_Float16>(v);
  return AsU(H2{h, h});
}

__device__ __forceinline__ F16v Mma(H8 a, H8 b, F16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// A product from zero. The empty asm after it marks both sources as still in
// use, so the result is never allocated over them: an MFMA whose destination
// aliases its A or B registers returned wrong sums on gfx950 (measured), and
// the compiler allows that allocation when a source dies at the product.
__device__ __forceinline__ F16v MmaFresh(H8 a, H8 b) {
  const F16v r = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, F16v{}, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(r));
  return r;
}
__device__ __forceinline__ F16v Mma8Fresh(H4 a, H4 b) {
  const F16v r = __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, F16v{}, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(r));
  return r;
}
__device__ __forceinline__ F16v Mma8(H4 a, H4 b, F16v c) {
  const F16v r = __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, c, 0, 0, 0);
  asm volatile("" ::"v"(a), "v"(b), "v"(c), "v"(r));
  return r;
}

// (a & mask) | c with the mask in an SGPR (gfx9 VOP3 takes no literal).
__device__ __forceinline__ uint32_t AndOr(uint32_t a, uint32_t mask, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(c));
  return r;
}

// 8 quant bytes of one row and step quarter -> the 8 low-nibble operands
// (sub-block 2s) and the 8 high-nibble operands (sub-block 2s + 1), each
// q * sc exactly, in the operand order of SplitX (within every 8 inputs:
// 0, 2, 1, 3, 4, 6, 5, 7). A low nibble read as the f16 1024 + q gives
// (1024 + q) sc - 1024 sc; a high nibble in place, 1024 + 16 q, gives
// (1024 + 16 q) sc/16 - 64 sc; the fused multiply-add never rounds (q sc <=
// 945).
__device__ __forceinline__ void DequantQuarter(U2 w, uint32_t mlo, uint32_t mhi, uint32_t magic, uint32_t slo,
                                               uint32_t nlo, uint32_t shi, uint32_t nhi, U4* lo, U4* hi) {
  const H2 sl = AsH2(slo), nl = AsH2(nlo), sh = AsH2(shi), nh = AsH2(nhi);
  uint32_t l[4], h[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t v = w[i], v8 = v >> 8;
    l[2 * i] = AsU(__builtin_elementwise_fma(AsH2(AndOr(v, mlo, magic)), sl, nl));     // inputs 4i, 4i + 2
    l[2 * i + 1] = AsU(__builtin_elementwise_fma(AsH2(AndOr(v8, mlo, magic)), sl, nl));  // 4i + 1, 4i + 3
    h[2 * i] = AsU(__builtin_elementwise_fma(AsH2(AndOr(v, mhi, magic)), sh, nh));
    h[2 * i + 1] = AsU(__builtin_elementwise_fma(AsH2(AndOr(v8, mhi, magic)), sh, nh));
  }
  *lo = U4{l[0], l[1], l[2], l[3]};
  *hi = U4{h[0], h[1], h[2], h[3]};
}

// Q6_K weight operands of 16 weights (one row, one sub-block of a step):
// from 16 ql bytes (low or high nibbles) and the 16 matching qh bytes (2
// bits at `shift`), q = nibble | bits << 4 read as the f16 1024 + q, less
// 1056: the exact operand q - 32 (|q - 32| <= 32); the sub-block's scale
// d * sc multiplies its products. Operand order as in DequantQuarter.
__device__ __forceinline__ void DequantQ6(U4 ql, U4 qh, bool high, int shift, uint32_t m00ff, uint32_t magic,
                                           U4* ba, U4* bb) {
  const H2 off = H2{static_cast<_Float16>(1056.0f), static_cast<_Float16>(1056.0f)};
  uint32_t r[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t nib = (high ? (ql[i] >> 4) : ql[i]) & 0x0F0F0F0Fu;
    const uint32_t q = nib | (((qh[i] >> shift) & 0x03030303u) << 4);
    r[2 * i] = AsU(AsH2(AndOr(q, m00ff, magic)) - off);
    r[2 * i + 1] = AsU(AsH2(AndOr(q >> 8, m00ff, magic)) - off);
  }
  *ba = U4{r[0], r[1], r[2], r[3]};
  *bb = U4{r[4], r[5], r[6], r[7]};
}

// QT: the weight type (kQ4_K or kQ6_K).
//
// A step is 64 inputs of a super-block. For Q4_K, step s holds sub-blocks 2s
// and 2s + 1 (inputs 64 s .. + 64: low and high nibbles of 32 quant bytes).
// For Q6_K, step s = 2 h + m holds strips m and m + 2 of half h (inputs
// 128 h + 32 m + [0, 32) and 128 h + 64 + 32 m + [0, 32): low and high
// nibbles of the same 32 ql bytes, with their qh bits); the token rows are
// staged in that order.
template <int QT>
__global__ __launch_bounds__(kThreads) void TGemmKernel(TiledArgs a) {
  constexpr bool kQ6 = QT == kQ6_K;
  constexpr int kNB = 1;  // weight operand arrays
  // a pair's last round in halves: workgroup tail_wg + 2 i + h takes half h
  // of tile tail_wg + i
  int wgi = static_cast<int>(blockIdx.x), zh = -1;
  if (a.tail_wg > 0 && wgi >= a.tail_wg) {
    zh = (wgi - a.tail_wg) & 1;
    wgi = a.tail_wg + ((wgi - a.tail_wg) >> 1);
  }
  const int tm = wgi % a.tiles_m;
  int nt = wgi / a.tiles_m, j = 0;
  while (j + 1 < a.n_jobs && nt >= a.tiles[j]) {
    nt -= a.tiles[j];
    ++j;
  }
  const GemmJob& J = a.job[j];
  const SplitX& x = a.x;
  const int M = x.M, K = x.K;
  // this split's super-blocks [o0, o1)
  const int z = blockIdx.y, nall = K >> 8;
  const int o0 = zh >= 0 ? zh * nall / 2 : z * nall / a.ksplit;
  const int o1 = zh >= 0 ? (zh + 1) * nall / 2 : (z + 1) * nall / a.ksplit;
  const int m0 = tm * kTM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // 32-token tile, 64-row half
  const int l32 = lane & 31, lh = lane >> 5;
  const int rows = J.w.rows;
  const int64_t rb = J.w.row_bytes;
  const bool pair = a.pair != 0;

  // Two stages (a step's operands) alternate: while the waves multiply stage
  // g % 2, the next step is unpacked into the other one; the per-super-block
  // tables alternate with the super-block.
  // token rows [hi, lo][token], swizzled (ASwz), one array per stage: the
  // compiler tells LDS arrays apart when it places the waits for its DMA
  // loads, so reads of one stage do not wait for the DMA into the other
  __shared__ __align__(16) _Float16 As0[2][kTM][64];
  __shared__ __align__(16) _Float16 As1[2][kTM][64];
  auto as = [&](int st) -> _Float16(*)[kTM][64] { return st ? As1 : As0; };
  // [stage][operand][row]: Q4_K 128-byte rows with chunks swizzled (BSwz),
  // Q6_K 144-byte rows (its writes, two chunks 16 bytes apart per thread,
  // meet no conflict there)
  constexpr int kBRow = kQ6 ? kRow : 64;
  __shared__ __align__(16) _Float16 Bs[2][kNB][kTN][kBRow];
  __shared__ __align__(16) _Float16 Ss[kQ6 ? 1 : 2][2][kTM][8];  // Q4_K [table][hi, lo][token]: sub-block sums
  __shared__ __align__(16) _Float16 Mn[kQ6 ? 1 : 2][kTN][8];     // Q4_K [table][row]: integer mins
  __shared__ float2 Dd[2][kTN];                                  // [table][row]: d, -32 dmin (Q4_K)
  // Q6_K [stage][row][16-input slice]: d * sc of the slice's sub-block
  __shared__ float Sc6[kQ6 ? 2 : 1][kQ6 ? kTN : 1][4];

  // The weight row this thread unpacks: local row br, quarter bq of a step
  // (Q4_K: 8 of its 32 quant bytes; Q6_K: strip bq / 2, half bq % 2 of it).
  // A pair's workgroup holds 64 output rows: local rows 64 h + [0, 32) are
  // gate rows 64 nt + 32 h + [0, 32), 64 h + [32, 64) the same rows of up
  // (so the matrix is wave-uniform: wave bit 1).
  const int br = tid >> 2, bq = tid & 3;
  const uint8_t* bmat = (pair && ((wave >> 1) & 1)) ? a.job[1].w.w : J.w.w;
  const int brow_i = pair ? min(64 * nt + 32 * (br >> 6) + (br & 31), rows - 1) : min(kTN * nt + br, rows - 1);
  const Rsrc rwt = MakeRsrc(bmat, static_cast<uint32_t>(rows) * static_cast<uint32_t>(rb));
  const uint32_t b_off = static_cast<uint32_t>(brow_i) * static_cast<uint32_t>(rb);
  const uint8_t* brow = bmat + b_off;  // (Q6_K blocks are 2-byte aligned: global loads)
  // The token rows of a step reach LDS by DMA (buffer loads with an LDS
  // destination: a wave's 64 lanes x 16 bytes land as 1 KB in a row). A
  // step's rows are 2 parts x 128 tokens x 128 bytes = 32 such loads, 4 per
  // wave: load i of wave w fills part w / 4, rows 8 b .. 8 b + 7, b =
  // (4 w + i) % 16; lane L reads token row 8 b + L / 8 and lands at chunk
  // L % 8 of it, which holds logical chunk (L % 8) ^ ASwz(row). Logical chunk
  // c holds step inputs 8 c .. + 8 (Q6_K: 8 c and 32 + 8 c of the step's two
  // strips). The buffer resources end at the last token, so the rows past it
  // read as zeros.
  const uint32_t a_bytes = static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u;
  const Rsrc ra_src = MakeRsrc(wave < 4 ? x.hi : x.lo, a_bytes);
  uint32_t a_voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * ((4 * wave + i) & 15) + (lane >> 3);
    const int lc = (lane & 7) ^ ASwz(r);
    a_voff[i] = (static_cast<uint32_t>(m0 + r) * static_cast<uint32_t>(K) + 8u * lc + (kQ6 && lc >= 4 ? 32u : 0u)) * 2u;
  }
  // Q4_K sub-block sums: part x token, one chunk of 8 (threads 256.. repeat
  // 0..255 and store nothing)
  const int sp = (wave >> 1) & 1, sr = tid & (kTM - 1);
  const Rsrc rsum = MakeRsrc(sp ? x.sum_lo : x.sum_hi, static_cast<uint32_t>(M) * static_cast<uint32_t>(K >> 5) * 2u);
  const uint32_t s_off = static_cast<uint32_t>(m0 + sr) * static_cast<uint32_t>(K >> 5) * 2u;

  uint32_t mlo, mhi, magic;
  asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(mlo));
  asm volatile("s_mov_b32 %0, 0xf000f0" : "=s"(mhi));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
  uint32_t m00ff;
  asm volatile("s_mov_b32 %0, 0xff00ff" : "=s"(m00ff));

  // The weights' loads run three steps ahead in a register ring: step g's
  // quant bytes sit in slot g % 2 from their issue until they are unpacked;
  // a super-block's first step also loads its header (Q4_K: d, dmin,
  // scales; Q6_K: scales, d) and the tokens' sub-block sums. Every step
  // issues the same loads, unconditionally (steps past the end re-read the
  // last one), so the compiler counts them and waits for one step's loads
  // while the next steps' stay in flight; the end of a step waits, by count,
  // for its token rows' DMA, issued before that step's weight loads.
  U4 hn, sn, hcur;
  U2 rw[2];      // Q4_K quant bytes
  U4 rl[2], rh[2];  // Q6_K ql, qh bytes
  uint32_t dn = 0, dcur = 0;  // Q6_K d
  const int nsteps = 4 * (o1 - o0);
  // step g = 4 o + s of the split (super-block o0 + o); ss = g % 4 (known
  // at compile time at every call)
  // the token rows of step g into stage st (4 DMA loads per wave)
  // VMEM instructions of one issue() of a super-block's first step
  // (ss == 0) and of the others (the counts of the compiled code)
  // (fewer would only wait longer; more would let a step read rows still
  // in flight)
  constexpr int kLoads0 = kQ6 ? 4 : 3, kLoads1 = kQ6 ? 2 : 1;
  auto issue_a = [&](int g, int st) {
    g = min(g, nsteps - 1);
    const int ob = o0 + (g >> 2), s = g & 3;
    const int so = kQ6 ? 2 * (256 * ob + 128 * (s >> 1) + 32 * (s & 1)) : 2 * (256 * ob + 64 * s);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra_src, (__attribute__((address_space(3))) void*)(&as(st)[wave >> 2][8 * ((4 * wave + i) & 15)][0]),
          16, a_voff[i], so, 0, 0);
  };
  auto issue = [&](int g, int slot, int ss) {
    g = min(g, nsteps - 1);
    const int ob = o0 + (g >> 2), s = g & 3;
    if constexpr (kQ6) {
      const uint8_t* blk = brow + 210 * static_cast<int64_t>(ob);
      const int lq = 16 * (bq & 1);
      const uint8_t* pl = blk + 64 * (s >> 1) + 32 * (s & 1) + lq;
      const uint8_t* ph = blk + 128 + 32 * (s >> 1) + lq;
      const U2 l0 = GLoad<U2A2>(pl), l1 = GLoad<U2A2>(pl + 8), h0 = GLoad<U2A2>(ph), h1 = GLoad<U2A2>(ph + 8);
      rl[slot] = U4{l0.x, l0.y, l1.x, l1.y};
      rh[slot] = U4{h0.x, h0.y, h1.x, h1.y};
      if (ss == 0) {
        const U2 s0 = GLoad<U2A2>(blk + 192), s1 = GLoad<U2A2>(blk + 200);
        hn = U4{s0.x, s0.y, s1.x, s1.y};
        dn = GLoad<uint16_t>(blk + 208);
      }
    } else {
      rw[slot] =
          __builtin_bit_cast(U2, __builtin_amdgcn_raw_buffer_load_b64(rwt, b_off + 16 + 8 * bq, 144 * ob + 32 * s, 0));
      if (ss == 0) {
        hn = __builtin_bit_cast(U4, __builtin_amdgcn_raw_buffer_load_b128(rwt, b_off, 144 * ob, 0));
        sn = __builtin_bit_cast(U4, __builtin_amdgcn_raw_buffer_load_b128(rsum, s_off, 16 * ob, 0));
      }
    }
  };
  // the tables of a super-block (table tb), from its header and sums
  auto store_tables = [&](int tb) {
    hcur = hn;
    if constexpr (kQ6) {
      dcur = dn;
    } else {
      if (tid < 2 * kTM) *reinterpret_cast<U4*>(&Ss[tb][sp][sr][0]) = sn;
      if (bq == 0) {
        uint32_t sc, mn[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) dev::ScaleMinK4(e, hcur.y, hcur.z, hcur.w, &sc, &mn[e]);
        U4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = AsU(H2{static_cast<_Float16>(static_cast<float>(mn[2 * e])),
                        static_cast<_Float16>(static_cast<float>(mn[2 * e + 1]))});
        *reinterpret_cast<U4*>(&Mn[tb][br][0]) = v;
        Dd[tb][br] = float2{dev::HalfToFloatFast(hcur.x & 0xFFFFu), -32.0f * dev::HalfToFloatFast(hcur.x >> 16)};
      }
    }
  };
  // the weight operands of a step (sub-step s of its super-block) into stage st
  auto store_b = [&](int slot, int s, int st) {
    if constexpr (kQ6) {
      const int strip = bq >> 1;
      // scale sc[8 h + 2 k + l / 16] of strip k = m + 2 strip, l = 16 (bq % 2) ..;
      // the thread's 16 inputs are slice bq (inputs 16 bq ..) of the step
      const int si = 8 * (s >> 1) + 2 * ((s & 1) + 2 * strip) + (bq & 1);
      const int sc = static_cast<int8_t>((hcur[si >> 2] >> (8 * (si & 3))) & 0xFFu);
      U4 ba, bb;
      DequantQ6(rl[slot], rh[slot], strip != 0, 2 * ((s & 1) + 2 * strip), m00ff, magic, &ba, &bb);
      const int c0 = 32 * strip + 16 * (bq & 1);
      *reinterpret_cast<U4*>(&Bs[st][0][br][c0]) = ba;
      *reinterpret_cast<U4*>(&Bs[st][0][br][c0 + 8]) = bb;
      Sc6[st][br][bq] = dev::HalfToFloatFast(dcur) * static_cast<float>(sc);
    } else {
      uint32_t sc0, sc1, unused;
      dev::ScaleMinK4(2 * s, hcur.y, hcur.z, hcur.w, &sc0, &unused);
      dev::ScaleMinK4(2 * s + 1, hcur.y, hcur.z, hcur.w, &sc1, &unused);
      const float f0 = static_cast<float>(sc0), f1 = static_cast<float>(sc1);
      U4 lo, hi;
      DequantQuarter(rw[slot], mlo, mhi, magic, HalfPair(f0), HalfPair(-1024.0f * f0), HalfPair(0.0625f * f1),
                     HalfPair(-64.0f * f1), &lo, &hi);
      *reinterpret_cast<U4*>(&Bs[st][0][br][8 * (bq ^ BSwz(br))]) = lo;
      *reinterpret_cast<U4*>(&Bs[st][0][br][8 * ((4 + bq) ^ BSwz(br))]) = hi;
    }
  };

  // Q4_K: the products of a super-block accumulate apart for the tokens' hi
  // and lo parts (four independent chains per wave), summed at its end.
  // Q6_K: each 16-input slice is one sub-block: its products (hi and lo
  // chained, C) are scaled by d * sc (Cs) into T while the next slice's
  // products run (the first such step adds zeros).
  F16v T[2], P0[2], P1[2], C[2];
  float Cs[2] = {0.0f, 0.0f};
  T[0] = T[1] = F16v{};
  if constexpr (kQ6) C[0] = C[1] = F16v{};

  // prologue: step 0's token rows and weights, step 1's weights; step 0
  // stored, step 2's weights issued
  issue_a(0, 0);
  issue(0, 0, 0);
  issue(1, 1, 1);
  store_tables(0);
  store_b(0, 0, 0);
  issue(2, 0, 2);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int o = 0; o < o1 - o0; ++o) {
    const int tb = o & 1;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // step g = 4 o + s: multiply stage s % 2; DMA step g + 1's token rows
      // into the other stage and unpack its weights there between the
      // slices; issue step g + 3's weight loads into the ring slot just
      // unpacked. After the last step the stores fill the idle stage.
      const int g = 4 * o + s, st = s & 1, nx = st ^ 1, ns = (s + 1) & 3;
      // the operands of 16-input slice kk + 1 are read from LDS while slice
      // kk is multiplied; the scheduling barriers keep the compiler from
      // hoisting every slice's reads
      constexpr int NO = 2 + 2 * kNB;
      H8 op[2][NO];
      auto read_ops = [&](H8* q, int kk) {
        const int ar = 32 * wm + l32, ac = 8 * ((2 * kk + lh) ^ ASwz(ar));
        q[0] = *reinterpret_cast<const H8*>(&as(st)[0][ar][ac]);
        q[1] = *reinterpret_cast<const H8*>(&as(st)[1][ar][ac]);
#pragma unroll
        for (int b = 0; b < kNB; ++b)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int r = 64 * wn + 32 * t + l32;
            const int bc = kQ6 ? 2 * kk + lh : (2 * kk + lh) ^ BSwz(r);
            q[2 + 2 * b + t] = *reinterpret_cast<const H8*>(&Bs[st][b][r][8 * bc]);
          }
      };
      read_ops(op[0], 0);
      float4 sc6[2];
      if constexpr (kQ6) {
#pragma unroll
        for (int t = 0; t < 2; ++t) sc6[t] = *reinterpret_cast<const float4*>(&Sc6[st][64 * wn + 32 * t + l32][0]);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk < 3) read_ops(op[(kk + 1) & 1], kk + 1);
        const H8* q = op[kk & 1];
        const bool fresh = s == 0 && kk == 0;
        if constexpr (kQ6) {
          F16v c[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) c[t] = Mma(q[1], q[2 + t], MmaFresh(q[0], q[2 + t]));
#pragma unroll
          for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) T[t][v] = __builtin_fmaf(Cs[t], C[t][v], T[t][v]);
            C[t] = c[t];
            Cs[t] = sc6[t][kk];
          }
        } else {
#pragma unroll
          for (int t = 0; t < 2; ++t) P0[t] = fresh ? MmaFresh(q[0], q[2 + t]) : Mma(q[0], q[2 + t], P0[t]);
#pragma unroll
          for (int t = 0; t < 2; ++t) P1[t] = fresh ? MmaFresh(q[1], q[2 + t]) : Mma(q[1], q[2 + t], P1[t]);
        }
        // the next step's staging, spread over the slices while the
        // products run
        if (kk == 0) issue_a(g + 1, nx);
        if (kk == 1 && s == 3) store_tables(tb ^ 1);  // step g + 1 starts super-block o + 1
        if (kk == 2) store_b(ns & 1, ns, nx);
        if (kk == 3) issue(g + 3, ns & 1, (s + 3) & 3);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (s == 3) {
        const int tr = 32 * wm + l32;
        if constexpr (kQ6) {
          // (each slice's products went into T with their scale)
        } else {
          // super-block end: T += d * P - 32 dmin * sum_j m_j * S_j
          const H4 xh = *reinterpret_cast<const H4*>(&Ss[tb][0][tr][4 * lh]);
          const H4 xl = *reinterpret_cast<const H4*>(&Ss[tb][1][tr][4 * lh]);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int lr = 64 * wn + 32 * t + l32;
            const float2 dd = Dd[tb][lr];
            const H4 bm = *reinterpret_cast<const H4*>(&Mn[tb][lr][4 * lh]);
            const F16v qm = Mma8(xl, bm, Mma8Fresh(xh, bm));
#pragma unroll
            for (int v = 0; v < 16; ++v)
              T[t][v] = __builtin_fmaf(dd.y, qm[v], __builtin_fmaf(dd.x, P0[t][v] + P1[t][v], T[t][v]));
          }
        }
      }
      // step g + 1's token rows have landed (only step g + 3's weight loads,
      // issued after them, may still be in flight)
      if (s == 1)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads0) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads1) : "memory");
      __syncthreads();
    }
  }

  if constexpr (kQ6) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) T[t][v] = __builtin_fmaf(Cs[t], C[t][v], T[t][v]);
  }

  // epilogue: result v of tile t is token 32 wm + 8 (v / 4) + 4 lh + v % 4,
  // local row 64 wn + 32 t + l32
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int tok = m0 + 32 * wm + 8 * (v >> 2) + 4 * lh + (v & 3);
    if (tok >= M) continue;
    const float is = x.inv_s[tok];
    if (pair) {
      // gate (tile 0) and up (tile 1) of the same row: silu(g) * u
      // (reference src/kernels.h:82-92), the bits of the unfused stores
      // followed by SwiGLURows
      const int row = 64 * nt + 32 * wn + l32;
      if (row >= rows) continue;
      if (zh >= 0) {
        // half of a tail tile: raw sums, [token][gate 64 | up 64]
        float* pt = x.part + (static_cast<int64_t>(wgi - a.tail_wg) * 2 + zh) * kTiledTailFloats +
                    (tok - m0) * kTiledRows + 32 * wn + l32;
        pt[0] = T[0][v];
        pt[64] = T[1][v];
        continue;
      }
      const float g = T[0][v] * is, u = T[1][v] * is;
      const float sg = g / __fadd_rn(1.0f, GlibcExpf(-g));
      J.y[static_cast<int64_t>(tok) * J.ldy + row] = __fmul_rn(sg, u);
      continue;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = kTN * nt + 64 * wn + 32 * t + l32;
      if (row >= rows) continue;
      const float val = T[t][v] * is;
      if (a.ksplit > 1) {
        x.part[(static_cast<int64_t>(z) * M + tok) * a.part_ld + a.pcol[j] + row] = val;
      } else {
        float* y = J.y + static_cast<int64_t>(tok) * J.ldy + row;
        *y = J.epi == kAdd ? *y + val : val;
      }
    }
  }
}

// The tail tiles of a halved pair launch: y = silu(g) * u with g, u the sums
// of the two halves (added in half order, then scaled as the full tiles'
// sums are), the full tiles' SwiGLU arithmetic. Workgroup (tile, y) takes
// tokens 16 y .. 16 y + 15 of the tile, four outputs per thread.
constexpr int kTailPer = 4, kTailSlices = kTM * 64 / (256 * kTailPer);
__global__ __launch_bounds__(256) void TailSwiGLUKernel(TiledArgs a) {
  const int tt = static_cast<int>(blockIdx.x), tile = a.tail_wg + tt;
  const int tm = tile % a.tiles_m, nt = tile / a.tiles_m;
  const GemmJob& J = a.job[0];
  const int rows = J.w.rows, M = a.x.M;
  const float* p0 = a.x.part + static_cast<int64_t>(tt) * 2 * kTiledTailFloats;
  const float* p1 = p0 + kTiledTailFloats;
  float g0[kTailPer], g1[kTailPer], u0[kTailPer], u1[kTailPer], is[kTailPer];
#pragma unroll
  for (int i = 0; i < kTailPer; ++i) {
    const int e = (static_cast<int>(blockIdx.y) * kTailPer + i) * 256 + static_cast<int>(threadIdx.x);
    const int tl = e >> 6, c = e & 63;
    g0[i] = p0[tl * kTiledRows + c];
    g1[i] = p1[tl * kTiledRows + c];
    u0[i] = p0[tl * kTiledRows + 64 + c];
    u1[i] = p1[tl * kTiledRows + 64 + c];
    is[i] = a.x.inv_s[min(tm * kTM + tl, M - 1)];
  }
#pragma unroll
  for (int i = 0; i < kTailPer; ++i) {
    const int e = (static_cast<int>(blockIdx.y) * kTailPer + i) * 256 + static_cast<int>(threadIdx.x);
    const int tl = e >> 6, c = e & 63;
    const int tok = tm * kTM + tl, row = 64 * nt + c;
    if (tok >= M || row >= rows) continue;
    const float g = (g0[i] + g1[i]) * is[i];
    const float u = (u0[i] + u1[i]) * is[i];
    const float sg = g / __fadd_rn(1.0f, GlibcExpf(-g));
    J.y[static_cast<int64_t>(tok) * J.ldy + row] = __fmul_rn(sg, u);
  }
}

}  // namespace

void LaunchTiled(const TiledArgs& a, hipStream_t s) {
  int tiles = 0;
  for (int j = 0; j < a.n_jobs; ++j) tiles += a.tiles[j];
  const uint32_t type = a.job[0].w.type;
  RPG_CHECK(type == kQ4_K || type == kQ6_K, "tiled gemm: weight type %u", type);
  for (int j = 1; j < a.n_jobs; ++j) RPG_CHECK(a.job[j].w.type == type, "tiled gemm: one weight type per launch");
  RPG_CHECK(type == kQ4_K || a.pair == 0, "tiled gemm: the SwiGLU pair is Q4_K only");
  RPG_CHECK(a.x.K % 256 == 0 && a.x.K >= 256, "tiled gemm: K = %d is not a multiple of 256", a.x.K);
  RPG_CHECK(a.ksplit >= 1 && a.ksplit <= a.x.K / 256, "tiled gemm: bad K split %d", a.ksplit);
  const int total = tiles * a.tiles_m;
  const int n_tail = a.tail_wg > 0 ? total - a.tail_wg : 0;
  if (a.tail_wg > 0)
    RPG_CHECK(a.pair && a.ksplit == 1 && a.tail_wg < total && a.x.K >= 512 &&
                  static_cast<int64_t>(n_tail) * 2 * kTiledTailFloats <= a.x.part_floats,
              "tiled gemm: bad tail split from workgroup %d of %d", a.tail_wg, total);
  const dim3 grid(static_cast<unsigned>(total + n_tail), static_cast<unsigned>(a.ksplit));
  if (type == kQ6_K)
    hipLaunchKernelGGL(TGemmKernel<kQ6_K>, grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(TGemmKernel<kQ4_K>, grid, dim3(kThreads), 0, s, a);
  HIP_CHECK(hipGetLastError());
  if (n_tail > 0) {
    hipLaunchKernelGGL(TailSwiGLUKernel, dim3(static_cast<unsigned>(n_tail), kTailSlices), dim3(256), 0, s, a);
    HIP_CHECK(hipGetLastError());
  }
}

}  // namespace k
}  // namespace rpg
