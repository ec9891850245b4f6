// Tile interpreter: any xt tile program of rank <= 3 tensors without conv.
//
// The host lowers the Block's ops, in program order, into a straight-line
// list of tile instructions over LDS slots (plan.cpp, match_vm).  One
// 256-thread workgroup runs one Block: it walks the list (the same for every
// Block, passed by value), each instruction a loop over its elements with a
// barrier after it.  Values live in LDS only, as f32 whatever their element
// type; every global tile is read once and written once.
//
// Semantics (the reference dialect, include/xt/XTOps.td and lib/xt/XTOps.cpp;
// the DSL tracer xtile/dsl.py):
//   * load / store: the tile at element offset coord * shape of its memref
//     (lib/xt/XTToNova.cpp:94-99), shared loads at their group leader's
//     coordinates (folded into the affine origin on the host).  Loads convert
//     f16 / bf16 / i8 exactly; stores round to nearest even (f16, bf16) or
//     round, saturate and map NaN to 0 (i8);
//   * add / sub / mul: IEEE f32, operands broadcast numpy-style along dims of
//     extent 1 (lib/xt/XTOps.cpp:104-145);
//   * exp, cos, sin, reciprocal, rsqrt, sigmoid, tanh, silu: elementwise, with
//     the textbook formulas 1/x, 1/sqrt(x), 1/(1+exp(-x)), x/(1+exp(-x));
//     ftoi rounds half to even and saturates to i8 (NaN -> 0); itof is the
//     identity on the held value (a renaming on the host);
//   * reduce_sum / reduce_max over axis 0 or 1 of a rank-2 tile, keeping the
//     reduced dim at 1 (lib/xt/XTOps.cpp:274-307);
//   * matmul / mma: [M,K] x [K,N] (+ acc) (lib/xt/XTOps.cpp:218-272); i8 x i8
//     sums in exact i32 and rounds to f32 once, as does the f32 result of an
//     exact sum; other types accumulate in f32;
//   * transpose (last two dims) and permute (out dim d = in dim perm[d]);
//     reshape is a renaming on the host (row-major data).
#include "common.h"
#include "launch.h"


namespace xtk {
namespace {

constexpr int VM_T = 256;
constexpr int VM_MAX_INST = 40;
constexpr int VM_MAX_ACC = 8;

enum : int { kLoad = 0, kStore = 1, kUnary = 2, kBinary = 3, kReduce = 4, kPermute = 5, kMatmul = 6 };
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2, kI8 = 3 };

// Kernel-argument form of one instruction (kernel arguments are limited to
// 4 KB, so dims travel as 16-bit values: every tile holds < 65536 elements).
struct VmI {
  int op, kind;
  int dst, a, b, c;               // LDS float offsets (c: mma accumulator, -1 none)
  unsigned short d[3];            // result dims (Reduce, Permute: source dims; Matmul: 1, M, N)
  unsigned short x[3];            // Binary: rhs dims; Reduce: axis; Permute: perm; Matmul: K, i8, -
  unsigned short l[3];            // Binary: lhs dims
  unsigned short e1, e2;          // dims the element loop decodes (Permute: the output's)
  Magic m2, m12;                  // dividers of e2 and e1*e2
};

struct VmA {
  void* ptr;
  TileOff org;
  long long s0, s1, s2;
  int elem;
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

// f32 -> f16 bits, IEEE round to nearest even (subnormals kept, overflow to
// inf, NaN to a quiet NaN of the same sign).
__device__ __forceinline__ unsigned short to_f16(float f) {
  const unsigned u = __float_as_uint(f);
  const unsigned sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (unsigned short)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (unsigned short)(sign | 0x7c00u);  // >= 65520 rounds past the largest half
  if (a < 0x38800000u)  // below 2^-14: a multiple of 2^-24, rounded to even
    return (unsigned short)(sign | (unsigned)rintf(__uint_as_float(a) * 16777216.0f));
  unsigned out = (((a >> 23) - 112u) << 10) | ((a >> 13) & 0x3ffu);
  const unsigned rem = a & 0x1fffu;
  out += (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) ? 1u : 0u;
  return (unsigned short)(sign | out);
}

__device__ __forceinline__ unsigned short to_bf16(float f) {
  const unsigned x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((x >> 16) | 0x40u);
  return (unsigned short)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

// float -> i8 value: NaN -> 0, round half to even, saturate
__device__ __forceinline__ float to_i8(float v) {
  if (v != v) return 0.0f;
  return fminf(fmaxf(rintf(v), -128.0f), 127.0f);
}

__device__ __forceinline__ float vm_read(const VmA& A, long long i) {
  switch (A.elem) {
    case kF32: return static_cast<const float*>(A.ptr)[i];
    case kF16: return static_cast<float>(static_cast<const _Float16*>(A.ptr)[i]);
    case kBF16: return __uint_as_float((unsigned)static_cast<const unsigned short*>(A.ptr)[i] << 16);
    default: return static_cast<float>(static_cast<const signed char*>(A.ptr)[i]);
  }
}

__device__ __forceinline__ void vm_write(const VmA& A, long long i, float v) {
  switch (A.elem) {
    case kF32: static_cast<float*>(A.ptr)[i] = v; break;
    case kF16: static_cast<unsigned short*>(A.ptr)[i] = to_f16(v); break;
    case kBF16: static_cast<unsigned short*>(A.ptr)[i] = to_bf16(v); break;
    default: static_cast<signed char*>(A.ptr)[i] = static_cast<signed char>(to_i8(v)); break;
  }
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
    case 7: return x * (1.0f / (1.0f + expf(-x)));
    default: return to_i8(x);
  }
}

__device__ __forceinline__ float vm_binary(int k, float a, float b) {
#pragma clang fp contract(off)
  return k == 0 ? a + b : k == 1 ? a - b : a * b;
}

__device__ __forceinline__ int bcast(const unsigned short (&s)[3], int i0, int i1, int i2) {
  return ((s[0] == 1 ? 0 : i0) * s[1] + (s[1] == 1 ? 0 : i1)) * s[2] + (s[2] == 1 ? 0 : i2);
}

__global__ __launch_bounds__(VM_T) void tilevm_kernel(VmArgs p) {
  extern __shared__ __attribute__((aligned(16))) float vmem[];
  int x, y, z;
  decode_block(blockIdx.x, p.gx, p.gy, x, y, z);
  const int tid = threadIdx.x;
  for (int k = 0; k < p.ninst; ++k) {
    const VmI& in = p.inst[k];
    const int n = in.d[0] * in.d[1] * in.d[2];
    switch (in.op) {
      case kLoad: {
        const VmA& A = p.acc[in.kind];
        const long long o = A.org.at(x, y, z);
        for (int e = tid; e < n; e += VM_T) {
          int i0, i1, i2;
          decode3(e, in, i0, i1, i2);
          vmem[in.dst + e] = vm_read(A, o + i0 * A.s0 + i1 * A.s1 + i2 * A.s2);
        }
        break;
      }
      case kStore: {
        const VmA& A = p.acc[in.kind];
        const long long o = A.org.at(x, y, z);
        for (int e = tid; e < n; e += VM_T) {
          int i0, i1, i2;
          decode3(e, in, i0, i1, i2);
          vm_write(A, o + i0 * A.s0 + i1 * A.s1 + i2 * A.s2, vmem[in.a + e]);
        }
        break;
      }
      case kUnary:
        for (int e = tid; e < n; e += VM_T) vmem[in.dst + e] = vm_unary(in.kind, vmem[in.a + e]);
        break;
      case kBinary: {
        const bool same_l = in.l[0] == in.d[0] && in.l[1] == in.d[1] && in.l[2] == in.d[2];
        const bool same_r = in.x[0] == in.d[0] && in.x[1] == in.d[1] && in.x[2] == in.d[2];
        if (same_l && same_r) {
          for (int e = tid; e < n; e += VM_T) vmem[in.dst + e] = vm_binary(in.kind, vmem[in.a + e], vmem[in.b + e]);
        } else {
          for (int e = tid; e < n; e += VM_T) {
            int i0, i1, i2;
            decode3(e, in, i0, i1, i2);
            const int ai = same_l ? e : bcast(in.l, i0, i1, i2);
            const int bi = same_r ? e : bcast(in.x, i0, i1, i2);
            vmem[in.dst + e] = vm_binary(in.kind, vmem[in.a + ai], vmem[in.b + bi]);
          }
        }
        break;
      }
      case kReduce: {
        const bool is_max = in.kind == 1;
        const int R = in.d[1], C = in.d[2];
        if (in.x[0] == 1) {
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
      case kMatmul: {
        // consecutive threads take consecutive columns of a row: the A value
        // is an LDS broadcast, the B row segment is contiguous
        const int N = in.d[2], K = in.x[0];
        const bool exact = in.x[1] != 0;
        for (int e = tid; e < n; e += VM_T) {
          const int i = e / N, j = e - (e / N) * N;
          const float* ar = vmem + in.a + i * K;
          const float* bc = vmem + in.b + j;
          float v;
          if (exact) {  // i8 x i8: |a*b| <= 2^14, the host bounds K so the i32 sum is exact
            int s = 0;
            for (int t = 0; t < K; ++t) s += (int)ar[t] * (int)bc[t * N];
            v = static_cast<float>(s);
          } else {
            v = 0.0f;
            for (int t = 0; t < K; ++t) v = fmaf(ar[t], bc[t * N], v);
          }
          if (in.c >= 0) v += vmem[in.c + e];
          vmem[in.dst + e] = v;
        }
        break;
      }
      default: {  // kPermute: out (j0, j1, j2) = in (i_perm)
        const int s1 = in.d[2], s0 = in.d[1] * in.d[2];
        for (int e = tid; e < n; e += VM_T) {
          int j0, j1, j2;
          decode3(e, in, j0, j1, j2);
          int iv[3] = {0, 0, 0};
          iv[in.x[0]] = j0;
          iv[in.x[1]] = j1;
          iv[in.x[2]] = j2;
          vmem[in.dst + e] = vmem[in.a + iv[0] * s0 + iv[1] * s1 + iv[2]];
        }
        break;
      }
    }
    __syncthreads();
  }
}

int elem_code(xt::Elem e) {
  switch (e) {
    case xt::Elem::F32: return kF32;
    case xt::Elem::F16: return kF16;
    case xt::Elem::BF16: return kBF16;
    case xt::Elem::I8: return kI8;
    default: return -1;
  }
}

}  // namespace

hipError_t launch_tilevm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  static_assert(sizeof(VmArgs) <= 4096, "kernel arguments are limited to 4 KB");
  const xt::VmPlan& vm = p.vm;
  if (vm.inst.size() > (size_t)VM_MAX_INST || vm.access.size() > (size_t)VM_MAX_ACC) {
    why = "tile program too long for the interpreter";
    return hipErrorInvalidValue;
  }
  VmArgs a{};
  for (size_t k = 0; k < vm.access.size(); ++k) {
    const xt::VmAccess& acc = vm.access[k];
    a.acc[k].ptr = bufs[acc.arg];
    a.acc[k].org = TileOff{acc.addr.c0, acc.addr.sx, acc.addr.sy, acc.addr.sz};
    a.acc[k].s0 = acc.stride[0];
    a.acc[k].s1 = acc.stride[1];
    a.acc[k].s2 = acc.stride[2];
    a.acc[k].elem = elem_code(acc.elem);
    if (a.acc[k].elem < 0) {
      why = "tile interpreter memrefs hold f32, f16, bf16 or i8";
      return hipErrorInvalidValue;
    }
  }
  for (size_t k = 0; k < vm.inst.size(); ++k) {
    const xt::VmInst& in = vm.inst[k];
    VmI& o = a.inst[k];
    o.op = static_cast<int>(in.op);
    o.kind = in.kind;
    o.dst = in.dst;
    o.a = in.a;
    o.b = in.b;
    o.c = in.c;
    for (int d = 0; d < 3; ++d) {
      if (in.dims[d] < 0 || in.dims[d] > 65535 || in.aux[d] < 0 || in.aux[d] > 65535 || in.lhs[d] < 0 ||
          in.lhs[d] > 65535) {
        why = "tile interpreter dims must lie in [0, 65535]";
        return hipErrorInvalidValue;
      }
      o.d[d] = (unsigned short)in.dims[d];
      o.x[d] = (unsigned short)in.aux[d];
      o.l[d] = (unsigned short)in.lhs[d];
    }
    int e0 = in.dims[0], e1 = in.dims[1], e2 = in.dims[2];
    if (in.op == xt::VmOp::Permute) {
      e0 = in.dims[in.aux[0]];
      e1 = in.dims[in.aux[1]];
      e2 = in.dims[in.aux[2]];
    }
    if ((long long)e0 * e1 * e2 >= 65536 || (long long)in.dims[0] * in.dims[1] * in.dims[2] >= 65536) {
      why = "tile interpreter values hold fewer than 65536 elements";
      return hipErrorInvalidValue;
    }
    o.e1 = (unsigned short)e1;
    o.e2 = (unsigned short)e2;
    o.m2 = udiv_magic((unsigned)(e2 > 0 ? e2 : 1));
    o.m12 = udiv_magic((unsigned)(e1 * e2 > 0 ? e1 * e2 : 1));
  }
  a.ninst = static_cast<int>(vm.inst.size());
  a.gx = p.grid[0];
  a.gy = p.grid[1];
  const size_t lds = size_t(vm.lds_floats) * 4;
  if (lds > size_t(kMaxLds)) {
    why = "tile program needs more than 160 KB of LDS";
    return hipErrorInvalidValue;
  }
  {
    hipError_t e = allow_full_lds(reinterpret_cast<const void*>(tilevm_kernel));
    if (e != hipSuccess) return e;
  }
  const long long blocks = grid_blocks(p);
  if (!grid_fits(blocks, VM_T)) {
    why = "tile program grid of " + std::to_string(blocks) + " Blocks exceeds one launch";
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(tilevm_kernel, dim3((unsigned)blocks), dim3(VM_T), lds, s, a);
  return hipGetLastError();
}

}  // namespace xtk
