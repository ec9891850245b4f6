// Pieces shared by the two generators of compiled tile programs: the
// register-resident fused kernel (fused.cpp) and the LDS-staged kernel
// (staged.cpp).  Host code; the strings are HIP source.
#pragma once

#include <string>

#include "plan.h"

namespace xt {

// Types and conversions every generated kernel starts with.
inline const char* fused_preamble() {
  static const char* k = R"(
typedef float xf4 __attribute__((ext_vector_type(4)));
typedef float xf2 __attribute__((ext_vector_type(2)));
typedef _Float16 xh4 __attribute__((ext_vector_type(4)));
typedef _Float16 xh2 __attribute__((ext_vector_type(2)));
typedef unsigned short xu4 __attribute__((ext_vector_type(4)));
typedef unsigned short xu2 __attribute__((ext_vector_type(2)));
typedef signed char xc4 __attribute__((ext_vector_type(4)));
typedef signed char xc2 __attribute__((ext_vector_type(2)));
struct FusedArgs { void* p[8]; };
template <bool MX, int C, int RM, int BM>
__device__ __forceinline__ float xdpp(float s) {
  const float id = MX ? -__builtin_huge_valf() : 0.0f;
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, id), __builtin_bit_cast(int, s),
                                                               C, RM, BM, false));
}
template <bool MX>
__device__ __forceinline__ float xwred(float v) {
  auto op = [](float a, float b) { return MX ? fmaxf(a, b) : a + b; };
  float a = v;
  a = op(a, xdpp<MX, 0x111, 0xf, 0xf>(v));
  a = op(a, xdpp<MX, 0x112, 0xf, 0xf>(v));
  a = op(a, xdpp<MX, 0x113, 0xf, 0xf>(v));
  a = op(a, xdpp<MX, 0x114, 0xf, 0xe>(a));
  a = op(a, xdpp<MX, 0x118, 0xf, 0xc>(a));
  a = op(a, xdpp<MX, 0x142, 0xa, 0xf>(a));
  a = op(a, xdpp<MX, 0x143, 0xc, 0xf>(a));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 63));
}
__device__ __forceinline__ float xbf(unsigned short u) { return __uint_as_float((unsigned)u << 16); }
__device__ __forceinline__ unsigned short xto_f16(float f) {
  const unsigned u = __float_as_uint(f);
  const unsigned sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (unsigned short)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (unsigned short)(sign | 0x7c00u);
  if (a < 0x38800000u) return (unsigned short)(sign | (unsigned)rintf(__uint_as_float(a) * 16777216.0f));
  unsigned out = (((a >> 23) - 112u) << 10) | ((a >> 13) & 0x3ffu);
  const unsigned rem = a & 0x1fffu;
  out += (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) ? 1u : 0u;
  return (unsigned short)(sign | out);
}
__device__ __forceinline__ unsigned short xto_bf16(float f) {
  const unsigned x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((x >> 16) | 0x40u);
  return (unsigned short)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float xto_i8(float v) {
  if (v != v) return 0.0f;
  return fminf(fmaxf(rintf(v), -128.0f), 127.0f);
}
)";
  return k;
}

// The f32 formula of a unary op with its operand written as X (the tile
// interpreter's semantics, kernels/tilevm.hip:vm_unary).
inline const char* unary_expr(int k) {
  switch (static_cast<VmUnary>(k)) {
    case VmUnary::Exp: return "expf(X)";
    case VmUnary::Cos: return "cosf(X)";
    case VmUnary::Sin: return "sinf(X)";
    case VmUnary::Recip: return "1.0f / (X)";
    case VmUnary::Rsqrt: return "1.0f / sqrtf(X)";
    case VmUnary::Sigmoid: return "1.0f / (1.0f + expf(-(X)))";
    case VmUnary::Tanh: return "tanhf(X)";
    case VmUnary::Silu: return "(X) * (1.0f / (1.0f + expf(-(X))))";
    default: return "xto_i8(X)";
  }
}

inline std::string replace_x(const char* pattern, const std::string& x) {
  std::string s(pattern), out;
  for (char ch : s) {
    if (ch == 'X') out += x;
    else out += ch;
  }
  return out;
}

}  // namespace xt
