// Decode (one-token) matvec launches on the matrix cores, for Q4_K and Q6_K
// weights: one launch per projection (or per pair of projections); the
// arithmetic is described in mfma_dot.h.
//
// Work: a workgroup of NW waves takes NW / kw tiles; the kw waves of a tile
// split its super-blocks (part p takes the p-th of kw contiguous ranges) and
// add their sums in LDS in a fixed order. Weights are read row-major or from
// the tile-major decode copy (decode.h), where a wave streams contiguous
// bytes. The input is staged once per workgroup with the first batch of
// weight loads in flight meanwhile.

#include <hip/hip_runtime.h>

#include "common.h"
#include "decode.h"
#include "mfma_dot.h"

namespace rpg {
namespace k {

namespace {

using namespace mfma;

static_assert(kMaxNormK >= kDecodeNormMaxK, "the matrix-core launches' normed staging");

// The header (first 64 bytes) holds what the prologue reads before it knows
// its job, then each job's weights, tile count and type (what the first
// weight loads need): the prologue requests all of it at once, so the
// weights are requested after one round trip for the arguments, not two.
// The jobs' other fields follow, read while the weights are in flight.
struct MfmaArgs {
  const float* x;
  const float* norm_w;
  int32_t K;
  float eps;
  int32_t epi;
  int32_t kw_log2;   // log2 of the waves per tile
  int32_t zero_off;  // LDS byte offsets: records at 0, then the zero region,
  int32_t xg_off;    // the per-group (f_g, sum x), the cross-wave sums
  int32_t red_off;
  int32_t n_jobs;
  int32_t tiles0, tiles1;  // tiles of jobs 0 and 1
  int32_t* inc;            // counter the launch adds 1 to, or null
  const uint8_t* jw[3];    // job j's w
  int32_t jtiles[3];       // job j's tiles
  uint32_t jtype[3];       // job j's type
  DecodeJob job[3];
};
static_assert(offsetof(MfmaArgs, jw) <= 64, "the header fills one 64-byte line");
static_assert(offsetof(MfmaArgs, job) <= 128, "header and per-job weights in two 64-byte lines");

template <int NW, uint32_t T, bool kTiled>
__device__ __forceinline__ void RunTile(const Hdr& a, const DecodeJob& J, const uint8_t* jw, int tile, bool active,
                                        int part, uint8_t* lds, double* redd, XChunks<NW>& xc) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, g = lane >> 4;
  const bool pair = J.w2 != nullptr || J.pair != 0;
  const int R = pair ? 8 : 16;
  const bool second = pair && col >= 8;
  const int row = tile * R + (second ? col - 8 : col);
  const bool valid = active && row < J.rows;
  const int n_sb = a.K >> 8, kwl = a.kwl, kw = 1 << kwl;
  constexpr int BB = MUnit<T>::kBytes;
  // Tile-major: super-block sb of the tile is the 16-block chunk at
  // ((tile * n_sb + sb) * 16) * BB -- a wave-uniform address (scalar
  // registers) plus the lane's fixed offsets, so the loads need no per-batch
  // vector address arithmetic. Row-major: the lane's row, then BB per
  // super-block.
  const uint8_t* tbase = jw + static_cast<int64_t>(active ? tile : 0) * n_sb * 16 * BB;
  const uint8_t* rowp = (second ? J.w2 : J.w) + static_cast<int64_t>(valid ? row : 0) * J.row_bytes;
  // this wave's super-blocks: the contiguous range [lo, hi)
  const int lo = (part * n_sb) >> kwl, hi = ((part + 1) * n_sb) >> kwl;
  const int n_part = hi - lo;
  // this lane's digit row of its group in super-block 0 -- row (col & 3) of
  // the record when it sits on the diagonal (col / 4 == g), else zeros
  const int gb = MUnit<T>::GroupBase(g);
  const bool diag = (col >> 2) == g;
  const int abase = diag ? gb * 64 + 16 * (col & 3) : a.zero_off + 64 * g;
  const int astep = diag ? 16 * 64 : 0;
  const float2* xg = reinterpret_cast<const float2*>(lds + a.xg_off) + gb;
  auto sb_of = [&](int i) { return min(lo + i, hi - 1); };
  MUnit<T> ua[kNB], ub[kNB];
  const Rsrc rsrc = TileRsrc(tbase, n_sb * 16 * BB);
  auto load = [&](MUnit<T>* u, int bt) {
    if constexpr (kTiled) {
      const auto off = MUnit<T>::MakeOff(g, col);
#pragma unroll
      for (int b = 0; b < kNB; ++b) u[b].LoadT(rsrc, 16 * BB * sb_of(bt * kNB + b), off);
    } else {
#pragma unroll
      for (int b = 0; b < kNB; ++b) u[b].Load(rowp + static_cast<int64_t>(BB) * sb_of(bt * kNB + b), g, col);
    }
  };
  const float xscale = StageDigits<NW, T == kQ8T, true>(a, xc, lds, redd, [&]() { load(ua, 0); });
  float acc = 0.0f;
  auto comp = [&](const MUnit<T>* u, int bt) {
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      const int i = bt * kNB + b, sb = sb_of(i);
      const float r = UnitDot(u[b], lds + abase + astep * sb, xg + 16 * sb, g);
      acc += i < n_part ? r : 0.0f;
    }
  };
  if (active) {
    const int nb = (n_part + kNB - 1) / kNB;
    for (int bt = 0; bt < nb; bt += 2) {
      load(ub, bt + 1);
      comp(ua, bt);
      if (bt + 1 >= nb) break;
      load(ua, bt + 2);
      comp(ub, bt + 1);
    }
  }
  // lanes j, j + 16, j + 32, j + 48 hold row j's partials
  acc = AddXor16(acc);
  acc = AddXor32(acc);
  if (kw > 1) {
    float* red = reinterpret_cast<float*>(lds + a.red_off);
    if (lane < 16) red[16 * wave + lane] = acc;
    LdsBarrier();
    if (part != 0) return;
    float sum = red[16 * wave + col];
    for (int p = 1; p < kw; ++p) sum += red[16 * (wave + p) + col];
    acc = sum;
  }
  if (!active) return;
  if (a.norm_w != nullptr) acc *= xscale;  // the RMSNorm scale of the input
  if (pair) {
    const float up = __uint_as_float(Dpp<kRowRor8>(__float_as_uint(acc)));  // lanes 0..7 <- 8..15
    if (lane < 8 && valid) {
      // silu(g) * up with glibc-exact expf (reference src/kernels.h:82-92)
      const float sg = acc / __fadd_rn(1.0f, GlibcExpf(-acc));
      J.y[row] = __fmul_rn(sg, up);
    }
  } else if (lane < 16 && valid) {
    float* y = J.y + row;
    *y = a.epi == kAdd ? *y + acc : acc;
  }
}

// kTypes: bit 0 = Q4_K jobs present, bit 1 = Q6_K jobs present, bit 2 =
// every job reads a tile-major copy, bit 3 = Q8_0 jobs (tile-major, alone in
// their launch); NW waves.
template <int kTypes, int NW>
__global__ __launch_bounds__(64 * NW) void MatvecMfmaKernel(MfmaArgs a) {
  extern __shared__ __align__(256) uint8_t lds[];
  __shared__ double redd[NW];
  const int wave = threadIdx.x >> 6;
  // one round trip for the header and the jobs' weight pointers, tile
  // counts and types (a single asm holds them all, so the compiler requests
  // them together), then the input loads; the jobs' other fields arrive
  // while the weights are in flight
  Hdr h;
  h.norm_w = a.norm_w;
  h.K = a.K;
  h.epi = a.epi;
  h.kwl = a.kw_log2;
  h.zero_off = a.zero_off;
  h.xg_off = a.xg_off;
  h.red_off = a.red_off;
  h.eps = a.eps;
  const float* x = a.x;
  int n_jobs = a.n_jobs, tiles0 = a.tiles0, tiles1 = a.tiles1;
  const uint8_t *jw0 = a.jw[0], *jw1 = a.jw[1], *jw2 = a.jw[2];
  int jt0 = a.jtiles[0], jt1 = a.jtiles[1], jt2 = a.jtiles[2];
  uint32_t jy0 = a.jtype[0], jy1 = a.jtype[1], jy2 = a.jtype[2];
  asm volatile(""
               : "+s"(h.norm_w), "+s"(h.K), "+s"(h.epi), "+s"(h.kwl), "+s"(h.zero_off), "+s"(h.xg_off),
                 "+s"(h.red_off), "+s"(h.eps), "+s"(x), "+s"(n_jobs), "+s"(tiles0), "+s"(tiles1), "+s"(jw0),
                 "+s"(jw1), "+s"(jw2), "+s"(jt0), "+s"(jt1), "+s"(jt2), "+s"(jy0), "+s"(jy1), "+s"(jy2));
  XChunks<NW> xc;
  xc.Load(x, h.norm_w, h.K);
  // wave-uniform tile and part, in scalar registers
  constexpr int kNWLog2 = NW == 4 ? 2 : NW == 8 ? 3 : 4;
  int tile = __builtin_amdgcn_readfirstlane((static_cast<int>(blockIdx.x) << (kNWLog2 - h.kwl)) + (wave >> h.kwl));
  const int part = __builtin_amdgcn_readfirstlane(wave & ((1 << h.kwl) - 1));
  // jobs' tiles in order; a tile past the last job's is inactive
  int j = 0;
  if (n_jobs > 1 && tile >= tiles0) {
    tile -= tiles0;
    j = 1;
    if (n_jobs > 2 && tile >= tiles1) {
      tile -= tiles1;
      j = 2;
    }
  }
  const DecodeJob& J = a.job[j];
  const uint8_t* jw = j == 0 ? jw0 : j == 1 ? jw1 : jw2;
  const uint32_t jtype = j == 0 ? jy0 : j == 1 ? jy1 : jy2;
  const bool active = tile < (j == 0 ? jt0 : j == 1 ? jt1 : jt2);
  // kTypes bit 2: every job reads a tile-major copy (the decode step), so
  // the row-major paths are not compiled in (half the code to fetch)
  constexpr bool kTiledOnly = (kTypes & 4) != 0;
  auto q4 = [&]() {
    if (kTiledOnly || J.tiled) {
      RunTile<NW, kQ4_K, true>(h, J, jw, tile, active, part, lds, redd, xc);
    } else {
      if constexpr (!kTiledOnly) RunTile<NW, kQ4_K, false>(h, J, jw, tile, active, part, lds, redd, xc);
    }
  };
  auto q8 = [&]() {
    if constexpr (kTiledOnly) RunTile<NW, kQ8T, true>(h, J, jw, tile, active, part, lds, redd, xc);
  };
  auto q6 = [&]() {
    if (kTiledOnly || J.tiled) {
      RunTile<NW, kQ6T, true>(h, J, jw, tile, active, part, lds, redd, xc);
    } else {
      if constexpr (!kTiledOnly) RunTile<NW, kQ6_K, false>(h, J, jw, tile, active, part, lds, redd, xc);
    }
  };
  if constexpr ((kTypes & 8) != 0) {
    q8();  // Q8_0 launches hold Q8_0 jobs only
  } else if constexpr ((kTypes & 3) == 1) {
    q4();
  } else if constexpr ((kTypes & 3) == 2) {
    q6();
  } else {
    if (jtype == kQ4_K)
      q4();
    else
      q6();
  }
  // (nothing in the launch reads the counter)
  if (a.inc != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *a.inc += 1;
}

template <int kTypes, int NW>
void Launch(const MfmaArgs& a, unsigned blocks, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((MatvecMfmaKernel<kTypes, NW>), dim3(blocks), dim3(64 * NW), lds, s, a);
}

template <int NW>
void LaunchTypes(int types, const MfmaArgs& a, unsigned blocks, size_t lds, hipStream_t s) {
  switch (types) {
    case 1: Launch<1, NW>(a, blocks, lds, s); break;
    case 2: Launch<2, NW>(a, blocks, lds, s); break;
    case 3: Launch<3, NW>(a, blocks, lds, s); break;
    case 5: Launch<5, NW>(a, blocks, lds, s); break;
    case 6: Launch<6, NW>(a, blocks, lds, s); break;
    case 12: Launch<12, NW>(a, blocks, lds, s); break;
    default: Launch<7, NW>(a, blocks, lds, s); break;
  }
}

}  // namespace

bool DecodeMatvecMfma(const DecodeMatvecArgs& in, hipStream_t s) {
  const int K = in.K;
  if (K <= 0 || K % 256 != 0 || K > kMaxK) return false;
  if (in.norm_w != nullptr && K > kMaxNormK) return false;
  MfmaArgs a{};
  a.n_jobs = in.n_jobs;
  a.x = in.x;
  a.K = K;
  a.norm_w = in.norm_w;
  a.eps = in.eps;
  a.epi = in.epi;
  a.inc = in.inc;
  int types = 0, tiles = 0;
  bool all_tiled = true;
  for (int j = 0; j < in.n_jobs; ++j) {
    DecodeJob J = in.job[j];
    if (J.type != kQ4_K && J.type != kQ6_K && J.type != kQ8_0) return false;
    // Q8_0 runs from its tile-major copy, in launches of Q8_0 jobs only
    if (J.type == kQ8_0 && (!J.tiled || J.w2 != nullptr || (types & 3) != 0)) return false;
    if (J.type != kQ8_0 && (types & 8) != 0) return false;
    if (J.w2 != nullptr && (J.tiled || J.type2 != J.type || J.row_bytes2 != J.row_bytes)) return false;
    const int64_t rb = (K / 256) * (J.type == kQ4_K ? 144 : J.type == kQ6_K ? 210 : 272);
    RPG_CHECK(J.row_bytes == rb, "decode matvec: row bytes %lld do not match K = %d", (long long)J.row_bytes, K);
    RPG_CHECK(!J.pair || J.tiled, "decode matvec: a pair flag needs a tile-major copy");
    types |= J.type == kQ4_K ? 1 : J.type == kQ6_K ? 2 : 8;
    all_tiled = all_tiled && J.tiled != 0;
    J.rows_per_tile = J.w2 != nullptr || J.pair ? 8 : 16;
    J.tiles = static_cast<int32_t>(CeilDiv(J.rows, J.rows_per_tile));
    tiles += J.tiles;
    a.job[j] = J;
    a.jw[j] = J.w;
    a.jtiles[j] = J.tiles;
    a.jtype[j] = J.type;
  }
  // Waves per tile: a tile's super-blocks are split only until the launch
  // holds about `target` waves -- 900 for Q4_K / Q6_K, 400 for Q8_0, whose
  // four-digit staging makes every extra wave dearer (same-box sweeps of the
  // decode steps: more, shorter waves lose to the extra staging and
  // cross-wave sums; the 1.7B QKV launch at 8 waves per tile instead of 4
  // cost 2.8 % of the Q4_K_M token, the Q8_0 model's launches at 1200
  // waves 6.8 %; the 4B launches are the same at 900 and 1200).
  const int n_sb = K / 256;
  int kw = 1;
  const int target = (types & 8) != 0 ? 400 : 900;
  while (kw < 8 && 2 * kw <= n_sb && static_cast<int64_t>(tiles) * kw < target) kw *= 2;
  const int nw = kw < 4 ? 4 : kw;
  a.kw_log2 = kw == 1 ? 0 : kw == 2 ? 1 : kw == 4 ? 2 : 3;
  a.tiles0 = a.job[0].tiles;
  a.tiles1 = in.n_jobs > 1 ? a.job[1].tiles : 0;
  if (all_tiled) types |= 4;
  const int n_groups = K / 16;
  int off = n_groups * 64;  // digit records
  a.zero_off = off;
  off += kZeroBytes;
  a.xg_off = off;
  off += n_groups * 8;
  a.red_off = off;
  off += nw * 16 * 4;
  const size_t dyn = static_cast<size_t>(off);
  const unsigned blocks = static_cast<unsigned>(CeilDiv(tiles, nw / kw));
  switch (nw) {
    case 4: LaunchTypes<4>(types, a, blocks, dyn, s); break;
    case 8: LaunchTypes<8>(types, a, blocks, dyn, s); break;
    default: RPG_CHECK(false, "decode matvec: %d waves per workgroup", nw);
  }
  HIP_CHECK(hipGetLastError());
  return true;
}


namespace {

// One thread per 2 bytes of the copy (block sizes 144 and 210 are even).
__global__ __launch_bounds__(256) void TileMajorKernel(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
                                                       int64_t row_bytes, int32_t rows, int32_t n_sb, int32_t bb,
                                                       int64_t n_units, uint8_t* __restrict__ dst) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= n_units) return;
  const int64_t byte = 2 * u, blk = byte / bb;
  const int off = static_cast<int>(byte - blk * bb);
  const int r = static_cast<int>(blk & 15);
  const int64_t ts = blk >> 4, tile = ts / n_sb;
  const int sb = static_cast<int>(ts - tile * n_sb);
  int rr = r, so = off;  // row in the tile, offset in its source block
  if (bb == 272) {         // Q8_0: quants regrouped by MFMA, then the scales (mfma_dot.h MUnit<kQ8T>)
    const int o = static_cast<int>(byte - (blk & ~int64_t{15}) * bb);  // offset in the chunk
    if (o < kQ8Sc) {
      const int m = o >> 10, gg = (o >> 4) & 3;
      rr = (o >> 6) & 15;
      so = 34 * (2 * m + (gg >> 1)) + 2 + 16 * (gg & 1) + (o & 15);
    } else {
      rr = (o - kQ8Sc) >> 4;
      so = 34 * (((o - kQ8Sc) & 15) >> 1) + (o & 1);
    }
  } else if (bb == 210) {  // Q6_K: the chunk holds ql, qh, scales, d of its 16 blocks in turn
    const int o = static_cast<int>(byte - (blk & ~int64_t{15}) * bb);  // offset in the chunk
    if (o < kQ6Qh) rr = o >> 7, so = o & 127;
    else if (o < kQ6Sc) rr = (o - kQ6Qh) >> 6, so = 128 + ((o - kQ6Qh) & 63);
    else if (o < kQ6D) rr = (o - kQ6Sc) >> 4, so = 192 + ((o - kQ6Sc) & 15);
    else rr = (o - kQ6D) >> 1, so = 208 + ((o - kQ6D) & 1);
  }
  const int64_t row = b != nullptr ? tile * 8 + (rr & 7) : tile * 16 + rr;
  const uint8_t* src = b != nullptr && rr >= 8 ? b : a;
  uint16_t v = 0;
  if (row < rows) v = *reinterpret_cast<const uint16_t*>(src + row * row_bytes + static_cast<int64_t>(sb) * bb + so);
  *reinterpret_cast<uint16_t*>(dst + byte) = v;
}

}  // namespace

bool DecodeTileable(const MatRef& m) {
  return (m.type == kQ4_K || m.type == kQ6_K || m.type == kQ8_0) && m.cols > 0 && m.cols % 256 == 0 &&
         m.cols <= kMaxK && m.rows > 0;
}

bool BatchTileable(const MatRef& m) { return DecodeTileable(m); }

namespace {
int SuperBlockBytes(uint32_t type) { return type == kQ4_K ? 144 : type == kQ6_K ? 210 : 272; }
}  // namespace

int64_t TileMajorBytes(const MatRef& m, bool pair) {
  RPG_CHECK(DecodeTileable(m), "tile-major copy: unsupported matrix");
  const int64_t tiles = CeilDiv(m.rows, pair ? 8 : 16);
  return tiles * (m.cols / 256) * 16 * SuperBlockBytes(m.type);
}

void TileMajor(const MatRef& a, const MatRef* b, uint8_t* dst, hipStream_t s) {
  const bool pair = b != nullptr;
  RPG_CHECK(!pair || (b->type == a.type && b->rows == a.rows && b->cols == a.cols),
            "tile-major copy: a pair needs two matrices of one shape and type");
  const int64_t bytes = TileMajorBytes(a, pair);
  const int64_t units = bytes / 2;
  hipLaunchKernelGGL(TileMajorKernel, dim3(static_cast<unsigned>(CeilDiv(units, 256))), dim3(256), 0, s, a.w,
                     pair ? b->w : nullptr, a.row_bytes, a.rows, a.cols / 256, SuperBlockBytes(a.type), units,
                     dst);
  HIP_CHECK(hipGetLastError());
}

}  // namespace k
}  // namespace rpg
