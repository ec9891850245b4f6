// Host-side launchers of the gfx950 kernels.  Each validates what its kernel
// assumes about the plan and the buffers (alignment, LDS budget) and returns
// hipErrorInvalidValue with `why` set instead of launching when it does not
// hold.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "../plan.h"

namespace xtk {

// A 1-D launch of `workgroups` groups of `threads` work-items.  The dispatch
// packet carries the grid size in work-items as a 32-bit count, so the product
// must stay below 2^32; the group count is also passed through int.
inline bool grid_fits(long long workgroups, int threads) {
  return workgroups >= 1 && workgroups <= 0x7fffffffLL && workgroups * threads < (1LL << 32);
}

// LDS per workgroup on gfx950.
constexpr int kMaxLds = 160 * 1024;

// Raises `kernel`'s dynamic-LDS limit to the full 160 KB on the current device,
// once per (kernel, device) and under a lock, so concurrent first launches
// cannot leave the limit below what a later launch needs.  A host-side
// attribute: launches recorded into a HIP graph afterwards only enqueue work.
inline hipError_t allow_full_lds(const void* kernel) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kernel, dev})) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
  if (e == hipSuccess) done.insert({kernel, dev});
  return e;
}

// Whether the GEMM and implicit-GEMM conv launchers may split K across
// workgroups whose f32 partial sums are added atomically (faster on launches
// of few tiles; the addition order, and so the last bits, vary between runs).
// XTILE_AMD_KSPLIT=0 in the environment turns it off (read at each launch,
// so a process may switch it between launches).
inline bool ksplit_allowed() {
  const char* v = std::getenv("XTILE_AMD_KSPLIT");
  return !(v && v[0] == '0' && v[1] == '\0');
}

// Blocks of the plan's grid, in 64 bits (three int32 axes).
inline long long grid_blocks(const xt::Plan& p) {
  return static_cast<long long>(p.grid[0]) * p.grid[1] * p.grid[2];
}

hipError_t launch_ew_binary(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);
hipError_t launch_row_softmax(const xt::Plan& p, void* const* bufs, hipStream_t s,
                              std::string& why);
hipError_t launch_gemm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);
hipError_t launch_conv2d(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);
hipError_t launch_conv2d_general(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);
// The implicit-GEMM conv kernel (conv_igemm.hip): false, with nothing
// launched, when the plan is outside what it takes; else `e` is the launch's status.
bool launch_conv2d_igemm(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e);
// The resident-image conv kernel (conv_image.hip), same contract.
bool launch_conv2d_image(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e);
// Whether a conv plan's Blocks tile images [0, grid[batch axis] * TB) x every
// output row, column and channel once in the output's natural NHWC
// addressing, with one filter whose origin is 16-byte aligned (`es` bytes an
// element); shared by the implicit-GEMM and resident-image kernels.
bool conv_blocks_cover_output(const xt::Plan& p, long long es);
// The few-input-channel conv kernel (conv_small.hip), same contract.
bool launch_conv2d_small(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e);
hipError_t launch_tilevm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);

// Fused tile programs (fused_jit.cpp): compile_fused fills fp.code from
// fp.source with hiprtc (or the code-object cache); launch_fused runs it.
bool compile_fused(xt::FusedPlan& fp, std::string& err);
hipError_t launch_fused(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);

}  // namespace xtk
