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
// GEMM view: M = output pixels, N = Cout, K = KH*KW*Cin.
//   * Persistent grid: one workgroup per CU walks work units of UR output rows
//     (UR divides the Block's TH; a Block is TH/UR units).  Blocks are
//     independent (README.md:85-89), so this is a scheduling choice.
//   * The whole filter (K x Cout) is staged once per workgroup in LDS,
//     transposed to Cout-major rows with K contiguous (the MFMA B operand
//     layout).  It is the `shared = 2` tile of the reference kernel
//     (kernels/conv2d.py:19-24): every Block reads the same filter.
//   * The receptive-field halo of a unit (rf_h x rf_w x Cin, NHWC so channels
//     are contiguous) lives in one of two LDS buffers, zero-filled outside the
//     image.  The next unit's halo is loaded into registers while the current
//     unit computes, then written to the other buffer; one barrier per unit.
//   * Waves take the unit's 16-pixel M tiles round-robin and all Cout/16 N
//     tiles, v_mfma_f32_16x16x32_{f16,bf16}; each B fragment read from LDS
//     feeds every M tile of the wave.
//   * Outputs are written once and never re-read: non-temporal stores.
#include <algorithm>
#include <atomic>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr int HV = 12;  // halo 16-byte vectors per thread per unit (at most)
constexpr int MT = 2;   // M tiles per wave per round
constexpr int FB = 4;   // filter sub-blocks per thread per batch

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
  int UR;               // output rows per work unit
  int units_per_block;  // TH / UR
  int total_units;
  int rf_h, rf_w;       // receptive field of one unit
  int cpad;             // LDS pitch of one halo pixel (Cin + 8)
  int kpad;             // LDS pitch of one filter row (K + 8)
  int halo_vecs;        // rf_h * rf_w * Cin / 8
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

struct Unit {
  const unsigned short* S;  // image base of the unit's batch entry
  int ih0, iw0;             // top-left source coordinate of the halo
  float* O;                 // output origin of the unit
};

__device__ __forceinline__ Unit unit_of(const ConvArgs& p, int u) {
  const int blk = u / p.units_per_block;
  const int sub = u - blk * p.units_per_block;
  int x, y, z;
  decode_block(blk, p.gx, p.gy, x, y, z);
  const int n = coord(p.cb_axis, p.cb_val, x, y, z);
  const int oh0 = coord(p.ch_axis, p.ch_val, x, y, z) * p.TH + sub * p.UR;
  const int ow0 = coord(p.cw_axis, p.cw_val, x, y, z) * p.TW;
  Unit t;
  t.S = p.src + (long long)n * p.H * p.W * p.C;
  t.ih0 = oh0 * p.sh - p.pad_t;
  t.iw0 = ow0 * p.sw - p.pad_l;
  t.O = p.out + p.to.at(x, y, z) + (long long)sub * p.UR * p.out_W * p.out_C;
  return t;
}

// Halo of unit `t` -> registers.  Every load is issued (out-of-range vectors
// read the image base and are zeroed), so the whole halo is one round trip.
__device__ __forceinline__ void load_halo(const ConvArgs& p, const Unit& t, int tid, uint4v (&hv)[HV]) {
  const int cv = p.C / 8;
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int v = tid + i * 256;
    const int vc = v < p.halo_vecs ? v : 0;
    const int c8 = vc % cv;
    const int pix = vc / cv;
    const int r = pix / p.rf_w, c = pix - r * p.rf_w;
    const int ih = t.ih0 + r, iw = t.iw0 + c;
    const bool inside = v < p.halo_vecs && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    const unsigned short* addr = inside ? t.S + ((long long)ih * p.W + iw) * p.C + c8 * 8 : t.S;
    const uint4v val = *reinterpret_cast<const uint4v*>(addr);
    hv[i] = inside ? val : uint4v{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void store_halo(const ConvArgs& p, unsigned short* Is, int tid,
                                           const uint4v (&hv)[HV]) {
  const int cv = p.C / 8;
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int v = tid + i * 256;
    if (v < p.halo_vecs) {
      const int c8 = v % cv;
      const int pix = v / cv;
      *reinterpret_cast<uint4v*>(&Is[pix * p.cpad + c8 * 8]) = hv[i];
    }
  }
}

// Filter -> LDS, transposed by 4(k) x 8(cout) register blocks; FB blocks per
// thread per batch, all of a batch's loads issued before the first use.
__device__ __forceinline__ void stage_filter(const ConvArgs& p, const unsigned short* F,
                                             unsigned short* Fs, int tid) {
  const int K = p.KH * p.KW * p.C;
  const int kgroups = K / 4;
  const int nsub = kgroups * (p.CO / 8);
  for (int base = tid; base < nsub; base += 256 * FB) {
    uint4v r[FB][4];
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const int sb = base + b * 256;
      const int sbc = sb < nsub ? sb : 0;
      const int kg = sbc % kgroups, cg = sbc / kgroups;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[b][i] = *reinterpret_cast<const uint4v*>(F + (long long)(kg * 4 + i) * p.CO + cg * 8);
    }
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const int sb = base + b * 256;
      if (sb >= nsub) continue;
      const int kg = sb % kgroups, cg = sb / kgroups;
      const int k0 = kg * 4, c0 = cg * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2v even, odd;
        even.x = (r[b][0][j] & 0xFFFFu) | (r[b][1][j] << 16);
        even.y = (r[b][2][j] & 0xFFFFu) | (r[b][3][j] << 16);
        odd.x = (r[b][0][j] >> 16) | (r[b][1][j] & 0xFFFF0000u);
        odd.y = (r[b][2][j] >> 16) | (r[b][3][j] & 0xFFFF0000u);
        *reinterpret_cast<uint2v*>(&Fs[(c0 + 2 * j) * p.kpad + k0]) = even;
        *reinterpret_cast<uint2v*>(&Fs[(c0 + 2 * j + 1) * p.kpad + k0]) = odd;
      }
    }
  }
}

template <int NT, bool BF16>
__device__ __forceinline__ void compute_unit(const ConvArgs& p, const Unit& t,
                                             const unsigned short* Fs, const unsigned short* Is,
                                             int tid) {
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  const int M = p.UR * p.TW;
  const int nmt = (M + 15) / 16;
  // wave w owns M tiles w, w+4, w+8, ...; MT of them per round
  for (int mt0 = wave; mt0 < nmt; mt0 += 4 * MT) {
    float4v acc[MT][NT];
    int base[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int pix = (mt0 + 4 * i) * 16 + lrow;
      const bool valid = (mt0 + 4 * i) < nmt && pix < M;
      const int ph = valid ? pix / p.TW : 0;
      const int pw = valid ? pix - ph * p.TW : 0;
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
            const short8 af = *reinterpret_cast<const short8*>(&Is[(base[i] + tap) * p.cpad + cc + lk]);
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[i][j] = mfma16<BF16>(af, bfr[j], acc[i][j]);
          }
        }
      }
    // D layout: lane holds pixel rows 4*(lane/16)+v of the M tile, column lane%16.
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (mt0 + 4 * i >= nmt) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int pix = (mt0 + 4 * i) * 16 + (lane >> 4) * 4 + v;
        if (pix >= M) continue;
        const int ph = pix / p.TW, pw = pix - (pix / p.TW) * p.TW;
        float* orow = t.O + ((long long)ph * p.out_W + pw) * p.out_C;
#pragma unroll
        for (int j = 0; j < NT; ++j) __builtin_nontemporal_store(acc[i][j][v], &orow[j * 16 + lrow]);
      }
    }
  }
}

template <int NT, bool BF16>
__global__ __launch_bounds__(256, 1) void conv2d_kernel(ConvArgs p) {
  extern __shared__ __attribute__((aligned(16))) unsigned short lds[];
  unsigned short* Fs = lds;
  const int halo_elems = p.rf_h * p.rf_w * p.cpad;
  unsigned short* Is0 = lds + p.CO * p.kpad;
  unsigned short* Is1 = Is0 + halo_elems;
  const int tid = threadIdx.x;

  int u = blockIdx.x;  // the host launches at most total_units workgroups
  uint4v hv[HV];
  Unit cur = unit_of(p, u);
  load_halo(p, cur, tid, hv);  // in flight while the filter is staged
  {
    // The filter tile is the whole filter array (checked by the planner), so
    // every Block - and every unit of this workgroup - uses the same origin.
    int x, y, z;
    decode_block(u / p.units_per_block, p.gx, p.gy, x, y, z);
    stage_filter(p, p.filt + p.tf.at(x, y, z), Fs, tid);
  }
  store_halo(p, Is0, tid, hv);
  __syncthreads();
  int buf = 0;
  for (; u < p.total_units; u += gridDim.x) {
    const int un = u + gridDim.x;
    Unit next = cur;
    if (un < p.total_units) {
      next = unit_of(p, un);
      load_halo(p, next, tid, hv);
    }
    compute_unit<NT, BF16>(p, cur, Fs, buf ? Is1 : Is0, tid);
    if (un < p.total_units) store_halo(p, buf ? Is0 : Is1, tid, hv);
    __syncthreads();
    buf ^= 1;
    cur = next;
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
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int max_lds = 0, cus = 0;
  e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  // Largest work unit (rows dividing TH) whose double-buffered halo fits.
  const size_t filt_bytes = size_t(a.CO) * a.kpad * 2;
  size_t lds = 0;
  a.UR = 0;
  for (int ur = a.TH; ur >= 1; --ur) {
    if (a.TH % ur) continue;
    const int rf_h = (ur - 1) * a.sh + a.dh * (a.KH - 1) + 1;
    const int rf_w = (a.TW - 1) * a.sw + a.dw * (a.KW - 1) + 1;
    const int halo_vecs = rf_h * rf_w * (a.C / 8);
    const size_t need = filt_bytes + 2 * size_t(rf_h) * rf_w * a.cpad * 2;
    if (halo_vecs <= 256 * HV && need <= size_t(max_lds)) {
      a.UR = ur;
      a.rf_h = rf_h;
      a.rf_w = rf_w;
      a.halo_vecs = halo_vecs;
      lds = need;
      break;
    }
  }
  if (a.UR == 0) {
    why = "conv2d tile row (" + std::to_string(a.TW) + " pixels x " + std::to_string(a.C) +
          " channels) with a " + std::to_string(a.CO) + "x" + std::to_string(K) +
          " filter does not fit the LDS budget; use a narrower tile";
    return hipErrorInvalidValue;
  }
  a.units_per_block = a.TH / a.UR;
  const long long units = (long long)p.grid[0] * p.grid[1] * p.grid[2] * a.units_per_block;
  if (units > 0x7fffffff) {
    why = "conv2d grid too large";
    return hipErrorInvalidValue;
  }
  a.total_units = static_cast<int>(units);
  const int nwg = static_cast<int>(std::min<long long>(units, cus > 0 ? cus : 256));
  dim3 grid(nwg);
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
