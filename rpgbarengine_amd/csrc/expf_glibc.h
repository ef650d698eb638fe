// expf that returns glibc's bits, for host and device.
//
// The reference's softmax and SiLU call std::exp(float), i.e. glibc expf
// (reference src/kernels.h:73,85), and the sampler's probabilities must match
// it bit for bit. glibc's expf is not correctly rounded, so the device runs the
// same published algorithm: ARM optimized-routines expf (Szabolcs Nagy, 2017,
// shipped as glibc sysdeps/ieee754/flt-32/e_expf.c), in glibc's x86-64 FMA
// build, whose multiply-adds are fused:
//   z  = x * 32/ln2;  k = round-to-nearest(z) via the 1.5*2^52 shift;  r = z - k
//   2^(k/32) from a 32-entry table of 2^(i/32) bit patterns (minus i<<47)
//   y  = 2^(k/32) * (1 + C2 r + C1 r^2 + C0 r^3),  all in double, then -> float.
// The table is the correctly rounded 2^(i/32); the polynomial is the published
// minimax fit (every table entry and the polynomial are exercised by the
// exhaustive comparison below). Pinned by an exhaustive comparison against the
// host's glibc over all 2^32 inputs (oracle/checks/expf_check.cc, run by
// tests/test_cpu_oracle.py) and on the GPU over every 37th float in
// [-104, 0] and every 41st in [0, 89] (tests/test_gpu_kernels.py).

#ifndef RPG_HIP_EXPF_GLIBC_H_
#define RPG_HIP_EXPF_GLIBC_H_

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define RPG_HD __host__ __device__ __forceinline__
#else
#define RPG_HD inline
#endif

namespace rpg {

struct Exp2fTable {
  uint64_t tab[32];
};

RPG_HD double ExpfAsDouble(uint64_t u) {
  double d;
  memcpy(&d, &u, 8);
  return d;
}

RPG_HD uint64_t ExpfAsU64(double d) {
  uint64_t u;
  memcpy(&u, &d, 8);
  return u;
}

RPG_HD uint32_t ExpfAsU32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

RPG_HD float GlibcExpf(float x) {
  // tab[i] = bits(2^(i/32)) - (i << 47)
  constexpr uint64_t kTab[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
  };
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;

  const uint32_t ux = ExpfAsU32(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {  // |x| >= 88 or NaN
    if (ux == 0xff800000u) return 0.0f;  // -inf
    if (abstop >= 0x7f8) return x + x;   // +inf, NaN
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = static_cast<double>(x);
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = ExpfAsU64(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  uint64_t t = kTab[ki % 32];
  t += ki << 47;
  const double s = ExpfAsDouble(t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return static_cast<float>(y);
}

}  // namespace rpg

#endif  // RPG_HIP_EXPF_GLIBC_H_
