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

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int int2v __attribute__((ext_vector_type(2)));

// A raw buffer descriptor (stride 0, `bytes` records): offsets at or past
// `bytes` read as zero.
__device__ __forceinline__ i32x4 raw_rsrc(const void* base, unsigned bytes = 0xFFFFFFFFu) {
  const unsigned long long b = reinterpret_cast<unsigned long long>(base);
  return i32x4{(int)(unsigned)b, (int)(unsigned)(b >> 32) & 0xFFFF, (int)bytes, 0x00020000};
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) unsigned char*)p);
}

// One 16-byte-per-lane LDS DMA: lane L's 16 bytes from rsrc at voff + soff
// land at LDS byte lds + 16 L (lanes off in exec write nothing).  Issued as
// inline assembly so that the compiler does not track it: kernels using it
// account for these loads themselves (explicit vmcnt waits before their
// barriers), where the compiler, which cannot tell LDS buffers apart
// reliably, would wait for every DMA in flight before the next LDS read.
// M0 carries the LDS address: an input bound to M0, so the compiler sets it
// once per DMA (and not at all when it already holds the address) instead of
// a save / set / restore around every instruction.
__device__ __forceinline__ void dma16(i32x4 rsrc, unsigned lds, unsigned voff, unsigned soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds) : "memory");
}

// s_waitcnt vmcnt(n) alone (gfx9 encoding: expcnt and lgkmcnt fields at
// their maxima), n < 64.
#define XTK_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x70 | 0xF00)

// The logical index of workgroup `id` of `n` when the 8 XCDs, which receive
// workgroups round-robin (id % 8), should each take a contiguous run of
// logical indices (the first n % 8 XCDs one more than the rest): a bijection
// on [0, n).
__device__ __forceinline__ int xcd_contiguous(int id, int n) {
  const int x = id & 7, j = id >> 3, per = n >> 3, rem = n & 7;
  return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + j;
}

// Affine element offset of a tile origin: c0 + x*sx + y*sy + z*sz
// (the host folds tile coordinates, tile shape and memref strides into it).
struct TileOff {
  long long c0, sx, sy, sz;
  __device__ __forceinline__ long long at(int x, int y, int z) const {
    return c0 + (long long)x * sx + (long long)y * sy + (long long)z * sz;
  }
};

struct Magic {
  unsigned m, k;
};

// n / d for n, d < 2^16 as umulhi(n, ceil(2^32 / d)) + (n & k), where k is
// all ones for d == 1 (m = 0) and zero otherwise, so there is no branch.
// Exact: with m*d = 2^32 + r (0 <= r < d) and n = q*d + s, n*m / 2^32 =
// q + (s + n*r / 2^32) / d and n*r < 2^32, so the fraction stays below 1.
__host__ __device__ __forceinline__ unsigned udiv(unsigned n, Magic m) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umulhi(n, m.m) + (n & m.k);
#else
  return unsigned((unsigned long long)n * m.m >> 32) + (n & m.k);
#endif
}

inline Magic udiv_magic(unsigned d) {
  return d == 1 ? Magic{0u, ~0u} : Magic{unsigned(((1ull << 32) + d - 1) / d), 0u};
}

// Exact n / d for 0 <= n < 2^31 and 1 <= d < 2^31 with one 64-bit multiply:
// with l = ceil(log2 d), s = 31 + l and m = ceil(2^s / d) <= 2^32, m*d = 2^s + e
// with 0 <= e < d <= 2^l, so n*m / 2^s = n/d + n*e / (d 2^s), and n*e < 2^s
// keeps the excess below 1/d: the floor is exact.  Replaces the ~30-instruction
// integer division sequence in kernel prologues.
struct Div31 {
  unsigned long long m;
  unsigned s;
  __host__ __device__ __forceinline__ unsigned operator()(unsigned n) const {
    return static_cast<unsigned>((n * m) >> s);
  }
};

inline Div31 div31(unsigned d) {
  unsigned l = 0;
  while ((1ull << l) < d) ++l;
  const unsigned s = 31 + l;
  return Div31{((1ull << s) + d - 1) / d, s};
}

// Linear Block index -> (x, y, z) for a grid of gx x gy x gz Blocks, either in
// the reference's z -> y -> x order (x fastest) or, when y_fastest, with y
// fastest (Blocks are independent, so any order gives the same result).
struct BlockDecode {
  Div31 dx, dy;
  int gx, gy;
  int y_fastest;
  __device__ __forceinline__ void operator()(int b, int& x, int& y, int& z) const {
    if (y_fastest) {
      const unsigned t = dy(static_cast<unsigned>(b));
      y = b - static_cast<int>(t) * gy;
      z = static_cast<int>(dx(t));
      x = static_cast<int>(t) - z * gx;
    } else {
      const unsigned t = dx(static_cast<unsigned>(b));
      x = b - static_cast<int>(t) * gx;
      z = static_cast<int>(dy(t));
      y = static_cast<int>(t) - z * gy;
    }
  }
};

inline BlockDecode block_decode(int gx, int gy, bool y_fastest) {
  return BlockDecode{div31(static_cast<unsigned>(gx)), div31(static_cast<unsigned>(gy)), gx, gy, y_fastest ? 1 : 0};
}

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

// One DPP step of wave_reduce: src from the lane `CTRL` names, or the
// reduction's identity where the source lane lies outside the row or the
// destination lane is masked off (bound_ctrl off keeps `old`).
template <bool IS_MAX, int CTRL, int RM, int BM>
__device__ __forceinline__ float dpp_or_identity(float src) {
  const float id = IS_MAX ? -__builtin_inff() : 0.0f;
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, id),
                                                               __builtin_bit_cast(int, src), CTRL, RM, BM, false));
}

// Max or sum over all 64 lanes of a wave (every lane active), returned to
// every lane.  DPP steps build an inclusive prefix that ends in lane 63:
// row_shr 1, 2, 3 of the inputs (each lane gets its four-lane group), row_shr
// 4 into banks 1-3 and row_shr 8 into banks 2-3 (each lane 15 of a row gets
// its row), row_bcast 15 into rows 1 and 3 and row_bcast 31 into rows 2 and
// 3 (lane 63 gets the wave); then lane 63 is read as a scalar.  Seven VALU
// operations with DPP operands, where a butterfly of __shfl_xor costs six
// ds_bpermute round trips through the LDS crossbar.
template <bool IS_MAX>
__device__ __forceinline__ float wave_reduce(float v) {
  auto op = [](float a, float b) { return IS_MAX ? fmaxf(a, b) : a + b; };
  float a = v;
  a = op(a, dpp_or_identity<IS_MAX, 0x111, 0xf, 0xf>(v));  // row_shr:1
  a = op(a, dpp_or_identity<IS_MAX, 0x112, 0xf, 0xf>(v));  // row_shr:2
  a = op(a, dpp_or_identity<IS_MAX, 0x113, 0xf, 0xf>(v));  // row_shr:3
  a = op(a, dpp_or_identity<IS_MAX, 0x114, 0xf, 0xe>(a));  // row_shr:4, banks 1-3
  a = op(a, dpp_or_identity<IS_MAX, 0x118, 0xf, 0xc>(a));  // row_shr:8, banks 2-3
  a = op(a, dpp_or_identity<IS_MAX, 0x142, 0xa, 0xf>(a));  // row_bcast:15, rows 1, 3
  a = op(a, dpp_or_identity<IS_MAX, 0x143, 0xc, 0xf>(a));  // row_bcast:31, rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 63));
}

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32): two instructions
// where expf takes eleven.  The product x * log2 e is rounded once, so the
// result's relative error is at most |x| 2^-24 plus exp2's own (one ulp):
// below 5.3e-6 wherever e^x is a normal float (x >= -87.3), and exactly 1
// at x = 0, 0 at -inf, NaN at NaN.  Results below FLT_MIN may flush to 0.
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
}

__device__ __forceinline__ float wave_max(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace xtk
