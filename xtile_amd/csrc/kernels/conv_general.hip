// xt.load_conv2d for every tile shape the planner accepts: the generic
// implicit-GEMM path behind the band and persistent kernels (conv.hip).
//
// Semantics (lib/xt/XTOps.cpp:43-90, lib/xt/XTToNova.cpp:110-142,353-437): the
// Block's output tile [TB, TH, TW, TC] at batch b0 = idx_b*TB, rows oh0 =
// idx_h*TH, columns ow0 = idx_w*TW holds
//   out[b, i, j, o] = sum_{kh,kw,c} src[b0+b, (oh0+i)*sh - pad_top + kh*dh,
//                                       (ow0+j)*sw - pad_left + kw*dw, c] * f[kh, kw, c, o]
// for the first TC of the filter's Cout channels, with source elements
// outside the image read as zero.  The channel tile coordinate is 0 (the
// source holds exactly the filter's input channels).
//
// GEMM view per Block: M = TB*TH*TW pixels, N = TC, K = KH*KW*Cin in the
// filter's (kh, kw, c) order.  A wave owns one 32 x 32 output tile and runs
// v_mfma_f32_32x32x16_{f16,bf16} (f32 sums) or v_mfma_i32_32x32x32_i8 (exact
// i32 sums, rounded to f32 once when stored).  Per K step a lane holds 16
// bytes of K for its pixel row (l % 32) and the same K positions for its
// filter column; which K positions a lane's bytes stand for does not matter
// to the product as long as both operands agree, so lane half l / 32 takes
// K [s*KS + 16/es * (l/32), +16/es).
//   * A: when Cin * esize is a multiple of 16 those K positions are 16
//     contiguous bytes of one pixel (one 16-byte load); otherwise the lane
//     gathers them element by element, crossing taps.
//   * B: one load per K position, consecutive lanes on consecutive Cout
//     columns (coalesced); the filter is small and stays in the caches.
//   * Out-of-image pixels, K past the end, pixel rows past M and columns past
//     TC read as zero; rows past M and columns past TC are not stored.
// No LDS and no barriers: waves are independent and a wave with no pixels
// exits at once.
#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

enum { kGenF16 = 0, kGenBF16 = 1, kGenI8 = 2 };
typedef int gen_int4 __attribute__((ext_vector_type(4)));
typedef int gen_int16 __attribute__((ext_vector_type(16)));
typedef float gen_float16 __attribute__((ext_vector_type(16)));

struct GenArgs {
  const unsigned char* src;
  const unsigned char* filt;
  unsigned char* out;
  TileOff tf, to;  // filter / output tile origins (elements)
  long long image_elems;  // H * W * Cin
  int H, W, C;
  int KH, KW, CO, TC;
  int TH, TW;
  int pad_t, pad_l, sh, sw, dh, dw;
  int cb_axis, ch_axis, cw_axis, cb_val, ch_val, cw_val, TB;
  int out_H, out_W, out_C;
  int gx, gy;
  int M, K, steps;
  int mgroups, ntiles;  // workgroups per Block = mgroups * ntiles (4 M tiles per workgroup)
};

template <int ELEM>
struct GenAcc {
  typedef gen_float16 type;
};
template <>
struct GenAcc<kGenI8> {
  typedef gen_int16 type;
};

template <int ELEM>
__device__ __forceinline__ typename GenAcc<ELEM>::type gen_mfma(gen_int4 a, gen_int4 b,
                                                               typename GenAcc<ELEM>::type c) {
  if constexpr (ELEM == kGenI8)
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  else if constexpr (ELEM == kGenBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}

// f32 -> bf16, round to nearest even, NaN kept quiet.
__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f) {
  const unsigned x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((x >> 16) | 0x40u);
  return (unsigned short)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ int pick(int axis, int val, int x, int y, int z) {
  return axis < 0 ? val : axis == 0 ? x : axis == 1 ? y : z;
}

// Advance a (c, kw, kh) K position by `d` channels.
__device__ __forceinline__ void advance(int& c, int& kw, int& kh, int d, int C, int KW) {
  c += d;
  while (c >= C) {
    c -= C;
    if (++kw == KW) {
      kw = 0;
      ++kh;
    }
  }
}

template <int ELEM, bool VEC, bool OUT_BF16>
__global__ __launch_bounds__(256) void conv2d_general_kernel(GenArgs p) {
  constexpr int ES = ELEM == kGenI8 ? 1 : 2;  // bytes per element
  constexpr int KL = 16 / ES;                 // K positions per lane per step
  constexpr int KS = 2 * KL;                  // K positions per step
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per_block = p.mgroups * p.ntiles;
  const int blk = blockIdx.x / per_block;
  const int r = blockIdx.x - blk * per_block;
  const int mg = r / p.ntiles, nt = r - mg * p.ntiles;
  const int mt = mg * 4 + wave;
  if (mt * 32 >= p.M) return;
  int x, y, z;
  decode_block(blk, p.gx, p.gy, x, y, z);
  const int b0 = pick(p.cb_axis, p.cb_val, x, y, z) * p.TB;
  const int oh0 = pick(p.ch_axis, p.ch_val, x, y, z) * p.TH;
  const int ow0 = pick(p.cw_axis, p.cw_val, x, y, z) * p.TW;
  const int lr = lane & 31, hi = lane >> 5;
  const int HW = p.TH * p.TW;

  // this lane's pixel row of A
  const int m = mt * 32 + lr;
  const bool mvalid = m < p.M;
  int pb = 0, pi = 0, pj = 0;
  if (mvalid) {
    pb = m / HW;
    const int rem = m - pb * HW;
    pi = rem / p.TW;
    pj = rem - pi * p.TW;
  }
  const unsigned char* img = p.src + (long long)(b0 + pb) * p.image_elems * ES;
  const int ih0 = (oh0 + pi) * p.sh - p.pad_t, iw0 = (ow0 + pj) * p.sw - p.pad_l;

  // this lane's filter column of B
  const int n = nt * 32 + lr;
  const bool nvalid = n < p.TC;
  const unsigned char* fcol = p.filt + (p.tf.at(x, y, z) + (nvalid ? n : 0)) * ES;
  const long long frow = (long long)p.CO * ES;

  int c = 0, kw = 0, kh = 0;
  advance(c, kw, kh, hi * KL, p.C, p.KW);
  typename GenAcc<ELEM>::type acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0;

  for (int s = 0; s < p.steps; ++s) {
    const int k0 = s * KS + hi * KL;
    gen_int4 a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
    if constexpr (VEC) {
      const int ih = ih0 + kh * p.dh, iw = iw0 + kw * p.dw;
      if (mvalid && k0 < p.K && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
        a = *reinterpret_cast<const gen_int4*>(img + (((long long)ih * p.W + iw) * p.C + c) * ES);
    } else {
      int cc = c, ckw = kw, ckh = kh;
#pragma unroll
      for (int e = 0; e < KL; ++e) {
        const int ih = ih0 + ckh * p.dh, iw = iw0 + ckw * p.dw;
        if (mvalid && k0 + e < p.K && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W) {
          const long long off = ((long long)ih * p.W + iw) * p.C + cc;
          const unsigned v = ES == 1 ? (unsigned)img[off] : (unsigned)reinterpret_cast<const unsigned short*>(img)[off];
          a[e * ES / 4] |= (int)(v << (8 * ((e * ES) & 3)));
        }
        if (++cc == p.C) {
          cc = 0;
          if (++ckw == p.KW) {
            ckw = 0;
            ++ckh;
          }
        }
      }
    }
#pragma unroll
    for (int e = 0; e < KL; ++e) {
      if (nvalid && k0 + e < p.K) {
        const unsigned char* f = fcol + (long long)(k0 + e) * frow;
        const unsigned v = ES == 1 ? (unsigned)*f : (unsigned)*reinterpret_cast<const unsigned short*>(f);
        b[e * ES / 4] |= (int)(v << (8 * ((e * ES) & 3)));
      }
    }
    acc = gen_mfma<ELEM>(a, b, acc);
    advance(c, kw, kh, KS, p.C, p.KW);
  }

  // D = A x B: lane l holds column 32*nt + l%32; register v holds pixel row
  // 8*(v/4) + 4*(l/32) + v%4 of the tile.
  if (!nvalid) return;
  const long long obase = p.to.at(x, y, z) + n;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int mm = mt * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
    if (mm < p.M) {
      const int bb = mm / HW;
      const int rem = mm - bb * HW;
      const int ii = rem / p.TW, jj = rem - ii * p.TW;
      const long long off = obase + (((long long)bb * p.out_H + ii) * p.out_W + jj) * p.out_C;
      // an i8 sum is an exact i32, rounded to f32 once (nearest even)
      const float val = static_cast<float>(acc[v]);
      if constexpr (OUT_BF16)
        reinterpret_cast<unsigned short*>(p.out)[off] = f32_to_bf16_rne(val);
      else
        reinterpret_cast<float*>(p.out)[off] = val;
    }
  }
}

template <int ELEM, bool VEC, bool OUT_BF16>
hipError_t launch_gen_t(const GenArgs& a, unsigned wgs, hipStream_t s) {
  hipLaunchKernelGGL((conv2d_general_kernel<ELEM, VEC, OUT_BF16>), dim3(wgs), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int ELEM>
hipError_t launch_gen_e(const GenArgs& a, bool vec, bool out_bf16, unsigned wgs, hipStream_t s) {
  if (vec) return out_bf16 ? launch_gen_t<ELEM, true, true>(a, wgs, s) : launch_gen_t<ELEM, true, false>(a, wgs, s);
  return out_bf16 ? launch_gen_t<ELEM, false, true>(a, wgs, s) : launch_gen_t<ELEM, false, false>(a, wgs, s);
}

}  // namespace

hipError_t launch_conv2d_general(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  const xt::ConvPlan& c = p.conv;
  const bool i8 = c.elem == xt::Elem::I8;
  const long long es = i8 ? 1 : 2;
  const long long K = c.KH * c.KW * c.C;
  const long long M = c.TB * c.TH * c.TW;
  // i32 sums of |i8 x i8| <= 2^14 stay exact below 2^31
  if (i8 && K >= (1LL << 17)) {
    why = "i8 conv2d reduction (KH*KW*Cin) must stay below 131072 for exact i32 sums";
    return hipErrorInvalidValue;
  }
  if (K >= (1LL << 30) || M >= (1LL << 30) || c.H * c.W >= (1LL << 31) || c.TW >= (1LL << 30)) {
    why = "conv2d tile or image too large for the generic kernel";
    return hipErrorInvalidValue;
  }
  const long long mtiles = (M + 31) / 32, mgroups = (mtiles + 3) / 4, ntiles = (c.TC + 31) / 32;
  const long long blocks = (long long)p.grid[0] * p.grid[1] * p.grid[2];
  const long long wgs = blocks * mgroups * ntiles;
  if (wgs >= (1LL << 24)) {
    why = "conv2d grid too large for the generic kernel (2^24 workgroups)";
    return hipErrorInvalidValue;
  }
  GenArgs a{};
  a.src = static_cast<const unsigned char*>(bufs[c.src_arg]);
  a.filt = static_cast<const unsigned char*>(bufs[c.filt_arg]);
  a.out = static_cast<unsigned char*>(bufs[c.out_arg]);
  a.tf = TileOff{c.filt_addr.c0, c.filt_addr.sx, c.filt_addr.sy, c.filt_addr.sz};
  a.to = TileOff{c.out_addr.c0, c.out_addr.sx, c.out_addr.sy, c.out_addr.sz};
  a.image_elems = c.H * c.W * c.C;
  a.H = (int)c.H;
  a.W = (int)c.W;
  a.C = (int)c.C;
  a.KH = (int)c.KH;
  a.KW = (int)c.KW;
  a.CO = (int)c.CO;
  a.TC = (int)c.TC;
  a.TB = (int)c.TB;
  a.TH = (int)c.TH;
  a.TW = (int)c.TW;
  a.pad_t = (int)c.pad_top;
  a.pad_l = (int)c.pad_left;
  a.sh = (int)c.stride_h;
  a.sw = (int)c.stride_w;
  a.dh = (int)c.dil_h;
  a.dw = (int)c.dil_w;
  a.cb_axis = c.cb.axis;
  a.ch_axis = c.ch.axis;
  a.cw_axis = c.cw.axis;
  a.cb_val = (int)c.cb.value;
  a.ch_val = (int)c.ch.value;
  a.cw_val = (int)c.cw.value;
  a.out_H = (int)c.out_H;
  a.out_W = (int)c.out_W;
  a.out_C = (int)c.out_C;
  a.gx = p.grid[0];
  a.gy = p.grid[1];
  a.M = (int)M;
  a.K = (int)K;
  const long long KS = 32 / es;
  a.steps = (int)((K + KS - 1) / KS);
  a.mgroups = (int)mgroups;
  a.ntiles = (int)ntiles;
  // one 16-byte load per lane and step needs whole 16-byte channel runs
  const bool vec = (c.C * es) % 16 == 0 && reinterpret_cast<uintptr_t>(a.src) % 16 == 0;
  const bool out_bf16 = c.out_elem == xt::Elem::BF16;
  const unsigned n = static_cast<unsigned>(wgs);
  if (i8) return launch_gen_e<kGenI8>(a, vec, out_bf16, n, s);
  if (c.elem == xt::Elem::BF16) return launch_gen_e<kGenBF16>(a, vec, out_bf16, n, s);
  return launch_gen_e<kGenF16>(a, vec, out_bf16, n, s);
}

}  // namespace xtk
