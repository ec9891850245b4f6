// Measurement kernels for the benchmark's ceilings (include/xt_ceiling.h):
// a streaming copy, an empty kernel and an MFMA issue loop, and the hold
// kernel that keeps a stream busy while the host enqueues a timed run.  They
// compute nothing a tile program needs; bench.py times them beside the tile
// programs so that each roofline fraction can be read against what this GPU
// attains.
#include <hip/hip_runtime.h>

#include "../../include/xt_ceiling.h"
#include "kernels/common.h"

namespace {

using xtk::float4v;
using xtk::uint4v;

constexpr int kCopyU = 4;     // 16-byte vectors per thread per pass
constexpr int kCopyWgs = 512;  // workgroups walking the array (two per CU)
constexpr long long kOnePass = 1LL << 21;  // up to 32 MiB: one pass of a full grid

// Streaming copy: each pass of a thread issues its U loads before its first
// store.  Arrays of at most 32 MiB are copied in one pass of a full grid with
// two vectors a thread (for C1's 12.6 MB 3.2-3.5 us a launch, where 512
// walking workgroups took 3.8); larger ones in one pass with eight vectors a
// thread (256 MiB: 6.33 TB/s, against 6.28 for two and 6.24 for four vectors
// a thread, and 6.27-6.30 for 512 workgroups walking the array with four);
// arrays beyond one launch's grid by 512 workgroups walking the array.
template <int U>
__global__ __launch_bounds__(256) void copy_kernel(const float4v* __restrict__ src, float4v* __restrict__ dst,
                                                   long long n) {
  const long long stride = (long long)gridDim.x * 256 * U;
  for (long long base = (long long)blockIdx.x * 256 * U + threadIdx.x; base < n; base += stride) {
    float4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + u * 256;
      v[u] = i < n ? __builtin_nontemporal_load(src + i) : float4v{0.f, 0.f, 0.f, 0.f};
    }
    xtk::issue_fence();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + u * 256;
      if (i < n) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

__global__ __launch_bounds__(256) void noop_kernel() {}

// One wave that returns once `ticks` of the constant-rate wall clock have
// passed since it started; sleeping between reads keeps it off the issue
// ports.  The host bounds `ticks`, so every launch ends.
__global__ __launch_bounds__(64) void hold_kernel(unsigned long long ticks) {
  const unsigned long long t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int16v __attribute__((ext_vector_type(16)));
typedef int int4v __attribute__((ext_vector_type(4)));

template <int KIND>
__global__ __launch_bounds__(256, 2) void mfma_kernel(const uint4v* __restrict__ ops, float* __restrict__ out,
                                                      int iters) {
  constexpr int NACC = 8;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  uint4v a[NACC], b[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) {
    a[j] = ops[t * 16 + j];
    b[j] = ops[t * 16 + NACC + j];
  }
  typedef typename std::conditional<KIND == 2, int16v, float16v>::type acc_t;
  acc_t acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < NACC; ++j) {
      if constexpr (KIND == 0)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(xtk::half8, a[j]),
                                                        __builtin_bit_cast(xtk::half8, b[j]), acc[j], 0, 0, 0);
      else if constexpr (KIND == 1)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(xtk::bf16x8, a[j]),
                                                         __builtin_bit_cast(xtk::bf16x8, b[j]), acc[j], 0, 0, 0);
      else
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(int4v, a[j]), __builtin_bit_cast(int4v, b[j]),
                                                       acc[j], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NACC; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += (float)acc[j][v];
  out[t] = s;
}

}  // namespace

extern "C" {

int xt_ceiling_copy(const void* src, void* dst, size_t bytes, void* stream) {
  if (bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return hipErrorInvalidValue;
  const long long n = static_cast<long long>(bytes / 16);
  if (n < 1) return hipErrorInvalidValue;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (n <= kOnePass) {
    const long long wgs = (n + 511) / 512;
    hipLaunchKernelGGL(copy_kernel<2>, dim3(static_cast<unsigned>(wgs)), dim3(256), 0, s,
                       static_cast<const float4v*>(src), static_cast<float4v*>(dst), n);
    return hipGetLastError();
  }
  if (n < (1LL << 31)) {
    const long long wgs = (n + 2047) / 2048;
    hipLaunchKernelGGL(copy_kernel<8>, dim3(static_cast<unsigned>(wgs)), dim3(256), 0, s,
                       static_cast<const float4v*>(src), static_cast<float4v*>(dst), n);
    return hipGetLastError();
  }
  long long wgs = (n + 256 * kCopyU - 1) / (256 * kCopyU);
  if (wgs > kCopyWgs) wgs = kCopyWgs;
  hipLaunchKernelGGL(copy_kernel<kCopyU>, dim3(static_cast<unsigned>(wgs)), dim3(256), 0, s,
                     static_cast<const float4v*>(src), static_cast<float4v*>(dst), n);
  return hipGetLastError();
}

int xt_ceiling_noop(int workgroups, void* stream) {
  if (workgroups < 1 || (long long)workgroups * 256 >= (1LL << 32)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(noop_kernel, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream));
  return hipGetLastError();
}

int xt_ceiling_hold(unsigned microseconds, void* stream) {
  if (microseconds < 1 || microseconds > 1000000) return hipErrorInvalidValue;
  int dev = 0, khz = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return e;
  if (khz <= 0) return hipErrorInvalidValue;
  const unsigned long long ticks = static_cast<unsigned long long>(microseconds) * static_cast<unsigned>(khz) / 1000u;
  hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), ticks);
  return hipGetLastError();
}

int xt_ceiling_mfma(const void* operands, float* out, int workgroups, int iters, int kind, void* stream) {
  if (workgroups < 1 || workgroups > (1 << 20) || iters < 1 || !operands || !out ||
      reinterpret_cast<uintptr_t>(operands) % 16)
    return hipErrorInvalidValue;
  const dim3 grid(workgroups), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint4v* ops = static_cast<const uint4v*>(operands);
  if (kind == 0) hipLaunchKernelGGL(mfma_kernel<0>, grid, block, 0, s, ops, out, iters);
  else if (kind == 1) hipLaunchKernelGGL(mfma_kernel<1>, grid, block, 0, s, ops, out, iters);
  else if (kind == 2) hipLaunchKernelGGL(mfma_kernel<2>, grid, block, 0, s, ops, out, iters);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // extern "C"
