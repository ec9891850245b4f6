// xt.load_conv2d as an implicit GEMM on the gfx950 matrix cores.
//
// Semantics (lib/xt/XTToNova.cpp:110-142,353-437; lib/nova/NovaOps.cpp:46-59):
// for the output tile of one Block at (b, oh0 = idx_h*TH, ow0 = idx_w*TW)
//   out[oh, ow, o] = sum_{kh,kw,c} src[b, oh*sh - pad_top + kh*dh,
//                                      ow*sw - pad_left + kw*dw, c] * f[kh, kw, c, o]
// with source elements outside [0,H) x [0,W) read as zero.  That is exactly the
// reference's halo slice: load rows [max(ideal,0), min(ideal+rf, H)) and pad the
// clamped parts with zeros.
//
// GEMM view per workgroup: M = TH*TW output pixels, N = Cout, K = KH*KW*Cin.
//   * The whole filter (K x Cout) is staged once per workgroup in LDS,
//     transposed to Cout-major rows with K contiguous (the MFMA B operand
//     layout).  It is the `shared = 2` tile of the reference kernel
//     (kernels/conv2d.py:19-24): every Block reads the same filter.
//   * The receptive-field halo of the tile (rf_h x rf_w x Cin, NHWC so channels
//     are contiguous) is staged in LDS with zero fill outside the image; every
//     (tap, 32-channel) K-step then reads 16-byte channel runs per pixel.
//   * 4 waves; each owns up to 4 of the 16-pixel M tiles at a time and all
//     Cout/16 N tiles, so each B fragment read from LDS feeds 4 MFMAs.
#include <atomic>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

struct ConvArgs {
  const unsigned short* src;
  const unsigned short* filt;
  float* out;
  TileOff tf, to;
  int N, H, W, C;
  int KH, KW, CO;
  int TH, TW;
  int pad_t, pad_l, sh, sw, dh, dw;
  int cb_axis, ch_axis, cw_axis;
  int cb_val, ch_val, cw_val;
  int out_W, out_C;
  int gx, gy;
  int rf_h, rf_w;
  int cpad;  // LDS pitch of one halo pixel (Cin + 8)
  int kpad;  // LDS pitch of one filter row (K + 8)
};

template <bool BF16>
__device__ __forceinline__ float4v mfma16(short8 a, short8 b, float4v c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

__device__ __forceinline__ int coord(int axis, int val, int x, int y, int z) {
  return axis < 0 ? val : axis == 0 ? x : axis == 1 ? y : z;
}

template <int NT, bool BF16>
__global__ __launch_bounds__(256) void conv2d_kernel(ConvArgs p) {
  constexpr int MT = 4;  // M tiles per wave per round
  extern __shared__ __attribute__((aligned(16))) unsigned short lds[];
  unsigned short* Fs = lds;
  unsigned short* Is = lds + p.CO * p.kpad;

  int x, y, z;
  decode_block(blockIdx.x, p.gx, p.gy, x, y, z);
  const int n = coord(p.cb_axis, p.cb_val, x, y, z);
  const int oh0 = coord(p.ch_axis, p.ch_val, x, y, z) * p.TH;
  const int ow0 = coord(p.cw_axis, p.cw_val, x, y, z) * p.TW;
  const int ih0 = oh0 * p.sh - p.pad_t;
  const int iw0 = ow0 * p.sw - p.pad_l;
  const int tid = threadIdx.x;
  const int K = p.KH * p.KW * p.C;

  // 1. filter -> LDS, transposed by 4(k) x 8(cout) register blocks
  {
    const unsigned short* F = p.filt + p.tf.at(x, y, z);
    const int kgroups = K / 4;
    const int nsub = kgroups * (p.CO / 8);
    for (int sb = tid; sb < nsub; sb += 256) {
      const int kg = sb % kgroups, cg = sb / kgroups;
      const int k0 = kg * 4, c0 = cg * 8;
      uint4v r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[i] = *reinterpret_cast<const uint4v*>(F + (long long)(k0 + i) * p.CO + c0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2v even, odd;
        even.x = (r[0][j] & 0xFFFFu) | (r[1][j] << 16);
        even.y = (r[2][j] & 0xFFFFu) | (r[3][j] << 16);
        odd.x = (r[0][j] >> 16) | (r[1][j] & 0xFFFF0000u);
        odd.y = (r[2][j] >> 16) | (r[3][j] & 0xFFFF0000u);
        *reinterpret_cast<uint2v*>(&Fs[(c0 + 2 * j) * p.kpad + k0]) = even;
        *reinterpret_cast<uint2v*>(&Fs[(c0 + 2 * j + 1) * p.kpad + k0]) = odd;
      }
    }
  }
  // 2. receptive-field halo -> LDS, zero outside the image
  {
    const int cv = p.C / 8;
    const int total = p.rf_h * p.rf_w * cv;
    const unsigned short* S = p.src + (long long)n * p.H * p.W * p.C;
    for (int v = tid; v < total; v += 256) {
      const int c8 = v % cv;
      const int pix = v / cv;
      const int r = pix / p.rf_w, c = pix - r * p.rf_w;
      const int ih = ih0 + r, iw = iw0 + c;
      uint4v val = {0u, 0u, 0u, 0u};
      if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
        val = *reinterpret_cast<const uint4v*>(S + ((long long)ih * p.W + iw) * p.C + c8 * 8);
      *reinterpret_cast<uint4v*>(&Is[pix * p.cpad + c8 * 8]) = val;
    }
  }
  __syncthreads();

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  const int M = p.TH * p.TW;
  const int nmt = (M + 15) / 16;
  float* O = p.out + p.to.at(x, y, z);

  for (int mt0 = wave * MT; mt0 < nmt; mt0 += 4 * MT) {
    float4v acc[MT][NT];
    int base[MT];
    bool valid[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int pix = (mt0 + i) * 16 + lrow;
      valid[i] = (mt0 + i) < nmt && pix < M;
      const int ph = valid[i] ? pix / p.TW : 0;
      const int pw = valid[i] ? pix - ph * p.TW : 0;
      base[i] = ph * p.sh * p.rf_w + pw * p.sw;
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};
    }
    for (int kh = 0; kh < p.KH; ++kh)
      for (int kw = 0; kw < p.KW; ++kw) {
        const int tap = kh * p.dh * p.rf_w + kw * p.dw;
        const int kbase = (kh * p.KW + kw) * p.C;
        for (int cc = 0; cc < p.C; cc += 32) {
          short8 bfr[NT];
#pragma unroll
          for (int j = 0; j < NT; ++j)
            bfr[j] = *reinterpret_cast<const short8*>(&Fs[(j * 16 + lrow) * p.kpad + kbase + cc + lk]);
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            short8 af = *reinterpret_cast<const short8*>(&Is[(base[i] + tap) * p.cpad + cc + lk]);
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[i][j] = mfma16<BF16>(af, bfr[j], acc[i][j]);
          }
        }
      }
    // D layout: lane holds pixel rows 4*(lane/16)+v of the M tile, column lane%16.
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (mt0 + i >= nmt) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int pix = (mt0 + i) * 16 + (lane >> 4) * 4 + v;
        if (pix >= M) continue;
        const int ph = pix / p.TW, pw = pix - (pix / p.TW) * p.TW;
        float* orow = O + ((long long)ph * p.out_W + pw) * p.out_C;
#pragma unroll
        for (int j = 0; j < NT; ++j) orow[j * 16 + lrow] = acc[i][j][v];
      }
    }
  }
}

TileOff to_off(const xt::TileAddr& a) { return TileOff{a.c0, a.sx, a.sy, a.sz}; }

// Raises the kernel's dynamic-LDS limit once (a host-side attribute, so later
// launches - including ones recorded into a HIP graph - only enqueue work).
template <int NT, bool BF16>
hipError_t launch_conv_t(const ConvArgs& a, dim3 grid, size_t lds, hipStream_t s) {
  static std::atomic<int> configured{0};
  auto fn = conv2d_kernel<NT, BF16>;
  if (static_cast<int>(lds) > configured.load()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    configured.store(static_cast<int>(lds));
  }
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_conv2d(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  const xt::ConvPlan& c = p.conv;
  ConvArgs a;
  a.src = static_cast<const unsigned short*>(bufs[c.src_arg]);
  a.filt = static_cast<const unsigned short*>(bufs[c.filt_arg]);
  a.out = static_cast<float*>(bufs[c.out_arg]);
  a.tf = to_off(c.filt_addr);
  a.to = to_off(c.out_addr);
  a.N = (int)c.N;
  a.H = (int)c.H;
  a.W = (int)c.W;
  a.C = (int)c.C;
  a.KH = (int)c.KH;
  a.KW = (int)c.KW;
  a.CO = (int)c.CO;
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
  a.out_W = (int)c.out_W;
  a.out_C = (int)c.out_C;
  a.gx = p.grid[0];
  a.gy = p.grid[1];
  a.rf_h = (a.TH - 1) * a.sh + a.dh * (a.KH - 1) + 1;
  a.rf_w = (a.TW - 1) * a.sw + a.dw * (a.KW - 1) + 1;
  a.cpad = a.C + 8;
  const int K = a.KH * a.KW * a.C;
  a.kpad = K + 8;
  const int nt = a.CO / 16;
  if (a.C % 32 || a.CO % 16 || !(nt == 1 || nt == 2 || nt == 4 || nt == 8)) {
    why = "conv2d kernel needs Cin % 32 == 0 and Cout in {16, 32, 64, 128}";
    return hipErrorInvalidValue;
  }
  for (const void* ptr : {(const void*)a.src, (const void*)a.filt, (const void*)a.out})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) {
      why = "conv2d buffers must be 16-byte aligned";
      return hipErrorInvalidValue;
    }
  if (a.tf.c0 % 8 || a.tf.sx % 8 || a.tf.sy % 8 || a.tf.sz % 8) {
    why = "conv2d filter tile must start on a 16-byte boundary";
    return hipErrorInvalidValue;
  }
  size_t lds = (size_t(a.CO) * a.kpad + size_t(a.rf_h) * a.rf_w * a.cpad) * 2;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int max_lds = 0;
  e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return e;
  if (lds > size_t(max_lds)) {
    why = "conv2d tile needs " + std::to_string(lds) + " bytes of LDS; the device allows " +
          std::to_string(max_lds) + " (use a smaller output tile)";
    return hipErrorInvalidValue;
  }
  dim3 grid(p.grid[0] * p.grid[1] * p.grid[2]), block(256);
  const bool bf16 = c.elem == xt::Elem::BF16;
#define XT_CONV(NTV, BFV) e = launch_conv_t<NTV, BFV>(a, grid, lds, s)
  switch (nt) {
    case 1: if (bf16) XT_CONV(1, true); else XT_CONV(1, false); break;
    case 2: if (bf16) XT_CONV(2, true); else XT_CONV(2, false); break;
    case 4: if (bf16) XT_CONV(4, true); else XT_CONV(4, false); break;
    default: if (bf16) XT_CONV(8, true); else XT_CONV(8, false); break;
  }
#undef XT_CONV
  return e;
}

}  // namespace xtk
