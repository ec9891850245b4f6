// Shared device helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace xtk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef short short8 __attribute__((ext_vector_type(8)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef unsigned int uint4v __attribute__((ext_vector_type(4)));
typedef unsigned int uint2v __attribute__((ext_vector_type(2)));

// Affine element offset of a tile origin: c0 + x*sx + y*sy + z*sz
// (the host folds tile coordinates, tile shape and memref strides into it).
struct TileOff {
  long long c0, sx, sy, sz;
  __device__ __forceinline__ long long at(int x, int y, int z) const {
    return c0 + (long long)x * sx + (long long)y * sy + (long long)z * sz;
  }
};

// Block id (x, y, z) of the grid point handled by linear index `b`, in the
// reference's z -> y -> x order (x fastest).
__device__ __forceinline__ void decode_block(int b, int gx, int gy, int& x, int& y, int& z) {
  x = b % gx;
  int t = b / gx;
  y = t % gy;
  z = t / gy;
}

// Scheduling fence: no instruction moves across it.  Placed after a batch of
// independent global loads, it keeps the compiler from hoisting arithmetic on
// the first load (and so a wait for it) above the remaining loads of the
// batch; every load of the batch is then in flight before the first wait.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ float wave_max(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace xtk
