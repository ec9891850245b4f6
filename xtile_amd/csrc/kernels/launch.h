// Host-side launchers of the gfx950 kernels.  Each validates what its kernel
// assumes about the plan and the buffers (alignment, LDS budget) and returns
// hipErrorInvalidValue with `why` set instead of launching when it does not
// hold.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../plan.h"

namespace xtk {

// A 1-D launch of `workgroups` groups of `threads` work-items.  The dispatch
// packet carries the grid size in work-items as a 32-bit count, so the product
// must stay below 2^32; the group count is also passed through int.
inline bool grid_fits(long long workgroups, int threads) {
  return workgroups >= 1 && workgroups <= 0x7fffffffLL && workgroups * threads < (1LL << 32);
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
hipError_t launch_tilevm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);

// Fused tile programs (fused_jit.cpp): compile_fused fills fp.code from
// fp.source with hiprtc (or the code-object cache); launch_fused runs it.
bool compile_fused(xt::FusedPlan& fp, std::string& err);
hipError_t launch_fused(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why);

}  // namespace xtk
