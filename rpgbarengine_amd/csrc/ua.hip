#include <hip/hip_runtime.h>
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef u32x2 u32x2a2 __attribute__((aligned(2)));
__global__ void K(const unsigned char* __restrict__ p, unsigned* y) {
  u32x2 v = *(const __attribute__((address_space(1))) u32x2a2*)(p + threadIdx.x * 210 + 2);
  y[threadIdx.x] = v.x + v.y;
}
