// exp for softmax weights on the hardware 2^x.
#pragma once

#include <hip/hip_runtime.h>

namespace rpg {

// exp(x) for x <= 0 as the hardware 2^y at y = x log2(e): the product's
// rounding moves the result by at most |x| 2^-24 relative (under 1.2e-6 for
// x >= -20; below that exp(x) < 2.1e-9 of the largest term of its sum), and
// exp(-inf) = 0. For attention weights, which only feed logits judged within
// a tolerance; glibc's expf (expf_glibc.h) would cost double arithmetic and
// a table load per call on the launch's critical path.
__device__ __forceinline__ float ExpSoft(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

}  // namespace rpg
