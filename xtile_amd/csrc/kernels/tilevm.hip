// Tile interpreter: any f32 xt tile program without matmul / conv.
//
// The host lowers the Block's ops, in program order, into a straight-line
// list of tile instructions over LDS slots (plan.cpp, match_vm).  One
// 256-thread workgroup runs one Block: it walks the list (the same for every
// Block, passed by value), each instruction a loop over its elements with a
// barrier after it.  Values live in LDS only; every global tile is read once
// and written once.
//
// Semantics (the reference dialect, include/xt/XTOps.td and lib/xt/XTOps.cpp;
// the DSL tracer xtile/dsl.py):
//   * load / store: the tile at element offset coord * shape of its memref
//     (lib/xt/XTToNova.cpp:94-99), shared loads at their group leader's
//     coordinates (folded into the affine origin on the host);
//   * add / sub / mul: IEEE f32, the right operand broadcast along its dims of
//     extent 1 (xtile/dsl.py:754-759);
//   * exp, cos, sin, reciprocal, rsqrt, sigmoid, tanh, silu: elementwise, with
//     the textbook formulas 1/x, 1/sqrt(x), 1/(1+exp(-x)), x/(1+exp(-x));
//   * reduce_sum / reduce_max over axis 0 or 1 of a rank-2 tile, keeping the
//     reduced dim at 1 (lib/xt/XTOps.cpp:274-307);
//   * transpose (last two dims) and permute (out dim d = in dim perm[d]);
//     reshape is a renaming on the host (row-major data).
#include "common.h"
#include "launch.h"

#include <atomic>

namespace xtk {
namespace {

constexpr int VM_T = 256;
constexpr int VM_MAX_INST = 40;
constexpr int VM_MAX_ACC = 8;

enum : int { kLoad = 0, kStore = 1, kUnary = 2, kBinary = 3, kReduce = 4, kPermute = 5 };

struct VmI {
  int op, kind;
  int dst, a, b;   // LDS float offsets
  int d0, d1, d2;  // result dims (Reduce, Permute: source dims)
  int x0, x1, x2;  // Binary: rhs dims; Reduce: axis; Permute: perm
  Magic m2, m12;   // dividers of the dims the element loop decodes (d2, d1*d2)
  int e1, e2;      // those dims (Permute: the output's)
};

struct VmA {
  float* ptr;
  TileOff org;
  long long s0, s1, s2;
};

struct VmArgs {
  VmA acc[VM_MAX_ACC];
  VmI inst[VM_MAX_INST];
  int ninst;
  int gx, gy;
};

__device__ __forceinline__ void decode3(int e, const VmI& in, int& i0, int& i1, int& i2) {
  const int t = (int)udiv((unsigned)e, in.m2);
  i2 = e - t * in.e2;
  i0 = (int)udiv((unsigned)e, in.m12);
  i1 = t - i0 * in.e1;
}

__device__ __forceinline__ float vm_unary(int k, float x) {
#pragma clang fp contract(off)
  switch (k) {
    case 0: return expf(x);
    case 1: return cosf(x);
    case 2: return sinf(x);
    case 3: return 1.0f / x;
    case 4: return 1.0f / sqrtf(x);
    case 5: return 1.0f / (1.0f + expf(-x));
    case 6: return tanhf(x);
    default: return x * (1.0f / (1.0f + expf(-x)));
  }
}

__device__ __forceinline__ float vm_binary(int k, float a, float b) {
#pragma clang fp contract(off)
  return k == 0 ? a + b : k == 1 ? a - b : a * b;
}

__global__ __launch_bounds__(VM_T) void tilevm_kernel(VmArgs p) {
  extern __shared__ __attribute__((aligned(16))) float vmem[];
  int x, y, z;
  decode_block(blockIdx.x, p.gx, p.gy, x, y, z);
  const int tid = threadIdx.x;
  for (int k = 0; k < p.ninst; ++k) {
    const VmI& in = p.inst[k];
    const int n = in.d0 * in.d1 * in.d2;
    switch (in.op) {
      case kLoad: {
        const VmA& A = p.acc[in.kind];
        const float* src = A.ptr + A.org.at(x, y, z);
        for (int e = tid; e < n; e += VM_T) {
          int i0, i1, i2;
          decode3(e, in, i0, i1, i2);
          vmem[in.dst + e] = src[i0 * A.s0 + i1 * A.s1 + i2 * A.s2];
        }
        break;
      }
      case kStore: {
        const VmA& A = p.acc[in.kind];
        float* dst = A.ptr + A.org.at(x, y, z);
        for (int e = tid; e < n; e += VM_T) {
          int i0, i1, i2;
          decode3(e, in, i0, i1, i2);
          dst[i0 * A.s0 + i1 * A.s1 + i2 * A.s2] = vmem[in.a + e];
        }
        break;
      }
      case kUnary:
        for (int e = tid; e < n; e += VM_T) vmem[in.dst + e] = vm_unary(in.kind, vmem[in.a + e]);
        break;
      case kBinary:
        if (in.x0 == in.d0 && in.x1 == in.d1 && in.x2 == in.d2) {
          for (int e = tid; e < n; e += VM_T) vmem[in.dst + e] = vm_binary(in.kind, vmem[in.a + e], vmem[in.b + e]);
        } else {
          for (int e = tid; e < n; e += VM_T) {
            int i0, i1, i2;
            decode3(e, in, i0, i1, i2);
            const int bi = ((in.x0 == 1 ? 0 : i0) * in.x1 + (in.x1 == 1 ? 0 : i1)) * in.x2 + (in.x2 == 1 ? 0 : i2);
            vmem[in.dst + e] = vm_binary(in.kind, vmem[in.a + e], vmem[in.b + bi]);
          }
        }
        break;
      case kReduce: {
        const bool is_max = in.kind == 1;
        const int R = in.d1, C = in.d2;
        if (in.x0 == 1) {
          // one row per group of 16 lanes: lane j takes columns j, j+16, ...
          const int g = tid >> 4, j = tid & 15;
          for (int r = g; r < R; r += VM_T / 16) {
            float v = is_max ? -INFINITY : 0.0f;
            for (int c = j; c < C; c += 16) {
              const float t = vmem[in.a + r * C + c];
              v = is_max ? fmaxf(v, t) : v + t;
            }
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) {
              const float t = __shfl_xor(v, o, 16);
              v = is_max ? fmaxf(v, t) : v + t;
            }
            if (j == 0) vmem[in.dst + r] = v;
          }
        } else {
          for (int c = tid; c < C; c += VM_T) {
            float v = is_max ? -INFINITY : 0.0f;
            for (int r = 0; r < R; ++r) {
              const float t = vmem[in.a + r * C + c];
              v = is_max ? fmaxf(v, t) : v + t;
            }
            vmem[in.dst + c] = v;
          }
        }
        break;
      }
      default: {  // kPermute: out (j0, j1, j2) = in (i_perm)
        const int sd[3] = {in.d0, in.d1, in.d2};
        const int s1 = sd[2], s0 = sd[1] * sd[2];
        for (int e = tid; e < n; e += VM_T) {
          int j0, j1, j2;
          decode3(e, in, j0, j1, j2);
          int iv[3] = {0, 0, 0};
          iv[in.x0] = j0;
          iv[in.x1] = j1;
          iv[in.x2] = j2;
          vmem[in.dst + e] = vmem[in.a + iv[0] * s0 + iv[1] * s1 + iv[2]];
        }
        break;
      }
    }
    __syncthreads();
  }
}

}  // namespace

hipError_t launch_tilevm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  const xt::VmPlan& vm = p.vm;
  if (vm.inst.size() > (size_t)VM_MAX_INST || vm.access.size() > (size_t)VM_MAX_ACC) {
    why = "tile program too long for the interpreter";
    return hipErrorInvalidValue;
  }
  VmArgs a{};
  for (size_t k = 0; k < vm.access.size(); ++k) {
    const xt::VmAccess& acc = vm.access[k];
    a.acc[k].ptr = static_cast<float*>(bufs[acc.arg]);
    a.acc[k].org = TileOff{acc.addr.c0, acc.addr.sx, acc.addr.sy, acc.addr.sz};
    a.acc[k].s0 = acc.stride[0];
    a.acc[k].s1 = acc.stride[1];
    a.acc[k].s2 = acc.stride[2];
  }
  for (size_t k = 0; k < vm.inst.size(); ++k) {
    const xt::VmInst& in = vm.inst[k];
    VmI& o = a.inst[k];
    o.op = static_cast<int>(in.op);
    o.kind = in.kind;
    o.dst = in.dst;
    o.a = in.a;
    o.b = in.b;
    o.d0 = in.dims[0];
    o.d1 = in.dims[1];
    o.d2 = in.dims[2];
    o.x0 = in.aux[0];
    o.x1 = in.aux[1];
    o.x2 = in.aux[2];
    int e0 = o.d0, e1 = o.d1, e2 = o.d2;
    if (in.op == xt::VmOp::Permute) {
      const int sd[3] = {o.d0, o.d1, o.d2};
      e0 = sd[o.x0];
      e1 = sd[o.x1];
      e2 = sd[o.x2];
    }
    if ((long long)e0 * e1 * e2 >= 65536) {
      why = "tile interpreter values hold fewer than 65536 elements";
      return hipErrorInvalidValue;
    }
    o.e1 = e1;
    o.e2 = e2;
    o.m2 = udiv_magic((unsigned)e2);
    o.m12 = udiv_magic((unsigned)(e1 * e2));
  }
  a.ninst = static_cast<int>(vm.inst.size());
  a.gx = p.grid[0];
  a.gy = p.grid[1];
  const size_t lds = size_t(vm.lds_floats) * 4;
  static std::atomic<int> configured{0};
  if (static_cast<int>(lds) > configured.load()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(tilevm_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    configured.store(static_cast<int>(lds));
  }
  const long long blocks = (long long)p.grid[0] * p.grid[1] * p.grid[2];
  hipLaunchKernelGGL(tilevm_kernel, dim3((unsigned)blocks), dim3(VM_T), lds, s, a);
  return hipGetLastError();
}

}  // namespace xtk
