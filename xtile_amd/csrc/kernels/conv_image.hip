// xt.load_conv2d with each image resident in LDS: the path for deep layers
// (small images, many channels) whose filter is too large for the band
// kernel's LDS-resident filter, where the implicit GEMM (conv_igemm.hip)
// would gather every input pixel once per tap through the CU's address unit.
//
// Semantics (lib/xt/XTOps.cpp:43-90, lib/xt/XTToNova.cpp:110-142,353-437):
//   out[n, oh, ow, o] = sum_{kh,kw,c} src[n, oh*sh - pad_t + kh*dh,
//                                         ow*sw - pad_l + kw*dw, c] * f[kh, kw, c, o]
// with source elements outside the image read as zero.  Taken when the
// Blocks tile the whole output (every output channel, one filter), f16 /
// bf16 sources with Cin a multiple of 64 and Cout a multiple of 32, a 3-wide
// filter, 128 to 256 output pixels an image, the image's channels fit in
// LDS beside the filter stages, and at least a quarter of the CUs' worth of
// workgroups (measurements at the launcher).
//
//   * One workgroup per (image, 32 output channels): N * Cout / 32
//     workgroups (32 x 14^2 x 256 -> 256: 256, one a CU).  The image reaches
//     LDS once, in sub-chunks of 64 channels (128 bytes a pixel, pixels 144
//     bytes apart: 16 consecutive pixels' 16-byte reads fall in distinct bank
//     groups); the filter's 32 columns stream through four stage buffers,
//     one filter row of taps (KW taps x 64 channels x 32 columns, 12 KB) a
//     stage.  LDS DMA bytes a workgroup: the image (padded to 144-byte
//     pixels) plus 32 filter columns, ~260 KB for the layer above, against
//     ~885 KB for an implicit-GEMM tile of 64 pixels x 128 channels.
//   * Four MFMA waves (one a SIMD) split K: wave w takes channels 16w ..
//     16w + 15 of every sub-chunk at every tap, all M tiles of 32 pixels
//     (v_mfma_f32_32x32x16_{f16,bf16}, f32 sums), so each filter fragment is
//     read once and the SIMDs carry equal work.  A fragments by ds_read_b128
//     at the tap's source pixel (a 256-byte zero block for taps outside the
//     image and pixels past the image), B fragments by ds_read_b64_tr_b16
//     from 64-byte filter rows.  The four partial sums meet through LDS at
//     the end and leave as 4-byte lanes, 32 lanes a 128-byte output run.
//   * Four more waves only issue the DMA (a wave blocks in DMA issue until
//     the CU's address unit takes each instruction): sub-chunk j of the
//     image in the slot of its first stage, every stage's filter rows three
//     stages ahead.
//   * Measured on 32 x 14^2 x 256 -> 256 (one call, 2000 launches each):
//     13.3 us against 15.7 for the implicit GEMM's 64 x 128 tiles (13.7
//     with three stage buffers).  What measured slower: two MFMA waves a
//     SIMD (tiles split 4 + 3; 14.5 us: fewer cycles, but the clock fell
//     from ~2.38 to ~2.17 GHz under the denser matrix work at lower socket
//     power), a ring of three sub-chunk regions with six filter buffers,
//     first fragments of each stage read during the stage before it, tap
//     validity precomputed per tile (no change).
//
// Every output pixel's f32 sum is a different grouping of the same terms as
// the other conv kernels' (four channel-interleaved partial sums added at
// the end); Blocks are independent (README.md:85-89).
#include <algorithm>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr unsigned kImOutOfRange = 0x80000000u;  // the input and the filter are < 2 GiB
constexpr int kImPitch = 144;                    // LDS bytes a pixel: 128 of channels, 16 of padding
constexpr int kImNS = 4;                         // filter stage buffers (three slots in flight)
typedef float float16v_t __attribute__((ext_vector_type(16)));

struct ImArgs {
  const unsigned char* src;   // NHWC input
  const unsigned char* filt;  // [K][CO], K in (kh, kw, c) order
  float* out;                 // [N * OH * OW][CO]
  unsigned src_bytes, filt_bytes;
  int H, W, C, KH, CO;
  int OW, P;  // output row length, output pixels an image
  int pad_t, pad_l, sh, sw, dh, dw;
  int nsub;    // 64-channel sub-chunks: C / 64
  int nh;      // DMA instructions a sub-chunk: ceil(H * W / 7)
  int region;  // LDS bytes a sub-chunk: nh * 1008 + 16
  int ntile;   // channel tiles of 32: CO / 32
  int nwg;     // N * ntile
  Div31 d_ow;
};

template <int ELEM>
__device__ __forceinline__ float16v_t im_mfma(uint4v a, uint4v b, float16v_t c) {
  if constexpr (ELEM == 1)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}

// ELEM 0: f16, 1: bf16.  MT: M tiles of 32 output pixels an image (P <= 32 MT).
// KW: filter width (taps a stage).
template <int ELEM, int MT, int KW>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_image_kernel(ImArgs p) {
  constexpr int FST = KW * 4096;  // filter stage: KW taps x 64 rows x 64 bytes
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup -> (image, channel tile); the XCDs take contiguous runs, so the
  // channel tiles of an image meet in one L2
  const int L = xcd_contiguous(blockIdx.x, p.nwg);
  const int n = L / p.ntile;
  const int n0 = (L - n * p.ntile) * 32;
  const int zero_off = p.nsub * p.region;   // 256 bytes of zeros
  const int fbuf_off = zero_off + 256;      // kImNS filter stages
  const int ns = p.nsub * p.KH;             // stages: (sub-chunk, filter row)

  if (wave >= 4) {
    // loader wave lw: a quarter of each slot's DMA instructions.  Slot s =
    // stage s's filter rows (KW instructions a wave) plus, when s opens
    // sub-chunk j, the image's channels 64 j .. 64 j + 63.
    const int lw = wave - 4;
    const i32x4 rs = raw_rsrc(p.src, p.src_bytes), rf = raw_rsrc(p.filt, p.filt_bytes);
    const unsigned ldf = (unsigned)p.CO * 2u;
    // image: instruction u fills pixels 7u .. 7u + 6, lane l pixel 7u + l / 9
    // and 16-byte chunk l % 9 (chunk 8 is the padding: its lane reads zeros;
    // lane 63 writes the next instruction's first chunk with the same bytes
    // that instruction writes there)
    const int hp = lane / 9, hc = lane - 9 * (lane / 9);
    const unsigned img = (unsigned)n * (unsigned)(p.H * p.W) * (unsigned)p.C * 2u;
    const int HW = p.H * p.W;
    // filter: instruction u (0 .. 4 KW - 1) fills rows 16 (u % 4) .. + 15 of tap u / 4
    const unsigned vb = (unsigned)(lane >> 2) * ldf + (unsigned)n0 * 2u + (unsigned)(lane & 3) * 16u;
    int sj = 0, skh = 0;  // the next slot's (sub-chunk, filter row)
    auto issue = [&](int s) {
      if (skh == 0) {
        const int hbase = sj * p.region;
        const unsigned cbase = img + (unsigned)(sj * 128 + hc * 16);
        for (int u = lw; u < p.nh; u += 4) {
          const int pix = 7 * u + hp;
          const bool in = pix < HW && hc < 8;
          dma16(rs, lds_addr(smem + hbase + u * 1008), in ? cbase + (unsigned)pix * (unsigned)p.C * 2u : kImOutOfRange, 0);
        }
      }
      unsigned char* const F = smem + fbuf_off + (s % kImNS) * FST;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        const int u = lw * KW + k, kw = u >> 2, rq = u & 3;
        const unsigned row = (unsigned)((skh * KW + kw) * p.C + sj * 64 + rq * 16);
        dma16(rf, lds_addr(F + kw * 4096 + rq * 1024), vb, row * ldf);
      }
      if (++skh == p.KH) {
        skh = 0;
        ++sj;
      }
    };
    issue(0);
    if (ns > 1) issue(1);
    if (ns > 2) issue(2);
    for (int s = 0; s < ns; ++s) {
      // slots s + 1 and s + 2 (issued after slot s) hold at least KW
      // instructions of this wave each, and DMA results arrive in issue
      // order, so vmcnt <= 2 KW means slot s has landed
      if (s + 2 < ns) XTK_WAIT_VM(2 * KW);
      else if (s + 1 < ns) XTK_WAIT_VM(KW);
      else XTK_WAIT_VM(0);
      asm volatile("s_barrier" ::: "memory");
      // into stage s - 1's buffer: every MFMA wave is past barrier s
      if (s + 3 < ns) issue(s + 3);
    }
  } else {
    // MFMA wave w = wave: channels 16 w .. 16 w + 15 of each sub-chunk
    const int lrow = lane & 31, hi = lane >> 5;
    if (wave == 0 && lane < 16)
      *reinterpret_cast<uint4v*>(smem + zero_off + lane * 16) = uint4v{0u, 0u, 0u, 0u};
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zero block is written before barrier 0
    // A: pixel row lrow of M tile i at its source origin (ih0, iw0); its
    // chunk 2 w + hi of a sub-chunk lies at pb + tap offset
    int ih0[MT], iw0[MT], pb[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = 32 * i + lrow;
      if (m < p.P) {
        const int oh = (int)p.d_ow((unsigned)m), ow = m - oh * p.OW;
        ih0[i] = oh * p.sh - p.pad_t;
        iw0[i] = ow * p.sw - p.pad_l;
      } else {
        ih0[i] = -(1 << 28);  // never inside the image
        iw0[i] = 0;
      }
      pb[i] = (ih0[i] * p.W + iw0[i]) * kImPitch + (2 * wave + hi) * 16;
    }
    // B: a 16-lane group of ds_read_b64_tr_b16 covers four 64-byte filter
    // rows; lane (g, li) reads K row 8 (g / 2) + 4 h + li / 4 of the wave's
    // 16 and columns 16 (g % 2) + 4 (li % 4) .. + 3
    int boff[2];
    {
      const int g = lane >> 4, li = lane & 15;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        boff[h] = (16 * wave + 8 * (g >> 1) + 4 * h + (li >> 2)) * 64 + (16 * (g & 1) + 4 * (li & 3)) * 2;
    }
    float16v_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;
    typedef __attribute__((address_space(3))) unsigned char lds_t;
    const unsigned zaddr = lds_addr(smem + zero_off);
    int j = 0, kh = 0;
    for (int s = 0; s < ns; ++s) {
      asm volatile("s_barrier" ::: "memory");
      const unsigned hb = lds_addr(smem + j * p.region);
      lds_t* const F = (lds_t*)(smem + fbuf_off + (s % kImNS) * FST);
      const int dih = kh * p.dh;
      // fragments of K step kw + 1 are read before the MFMAs of step kw
      // (one MFMA wave a SIMD: no other wave hides the LDS latency)
      auto read_a = [&](int kw, uint4v* af) {
        const int diw = kw * p.dw;
        const unsigned toff = hb + (unsigned)((dih * p.W + diw) * kImPitch);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const bool in = ((unsigned)(ih0[i] + dih) < (unsigned)p.H) & ((unsigned)(iw0[i] + diw) < (unsigned)p.W);
          const unsigned a = in ? toff + (unsigned)pb[i] : zaddr;
          af[i] = *reinterpret_cast<const uint4v __attribute__((address_space(3)))*>(a);
        }
      };
      uint4v bf[KW], af[2][MT];
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) {
        const uint2v l2 = __builtin_bit_cast(
            uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        reinterpret_cast<short4v __attribute__((address_space(3)))*>(F + kw * 4096 + boff[0])));
        const uint2v h2 = __builtin_bit_cast(
            uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        reinterpret_cast<short4v __attribute__((address_space(3)))*>(F + kw * 4096 + boff[1])));
        bf[kw] = uint4v{l2[0], l2[1], h2[0], h2[1]};
      }
      read_a(0, af[0]);
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) {
        // the fence keeps step kw + 1's reads ahead of step kw's MFMAs (the
        // scheduler would sink each read down to its MFMA)
        if (kw + 1 < KW) read_a(kw + 1, af[(kw + 1) & 1]);
        issue_fence();
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i] = im_mfma<ELEM>(af[kw & 1][i], bf[kw], acc[i]);
      }
      if (++kh == p.KH) {
        kh = 0;
        ++j;
      }
    }
    __syncthreads();  // every wave is done with the image and the filter stages
    // the wave's partial sums: register group q (v = 4 q .. 4 q + 3) of tile i
    // at ((wave MT + i) 4 + q) KB + 16 lane
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4v*>(smem + ((wave * MT + i) * 4 + q) * 1024 + lane * 16) =
            float4v{acc[i][4 * q], acc[i][4 * q + 1], acc[i][4 * q + 2], acc[i][4 * q + 3]};
  }
  if (wave >= 4) __syncthreads();  // the loaders' side of the barrier above
  __syncthreads();
  // D = A x B per 32 x 32 tile: lane l holds channel l % 32 and register v
  // pixel row 8 (v / 4) + 4 (l / 32) + v % 4.  Each group of four registers
  // is summed over the four waves' partials and stored by all eight waves.
  for (int g = tid; g < MT * 256; g += 512) {
    const int i = g >> 8, q = (g >> 6) & 3, l = g & 63;
    const unsigned char* const src = smem + (i * 4 + q) * 1024 + l * 16;
    float4v sum = *reinterpret_cast<const float4v*>(src);
#pragma unroll
    for (int w = 1; w < 4; ++w) sum += *reinterpret_cast<const float4v*>(src + w * MT * 4096);
    const int r0 = 32 * i + 8 * q + 4 * (l >> 5);
    float* const o = p.out + ((long long)n * p.P + r0) * p.CO + n0 + (l & 31);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (r0 + e < p.P) __builtin_nontemporal_store(sum[e], o + (long long)e * p.CO);
  }
}

template <int ELEM, int KW>
hipError_t launch_im(const ImArgs& a, int mt, size_t lds, hipStream_t s) {
  const void* fn = nullptr;
  switch (mt) {
#define XT_IM(MTV) \
  case MTV: fn = reinterpret_cast<const void*>(conv_image_kernel<ELEM, MTV, KW>); break
    XT_IM(1); XT_IM(2); XT_IM(3); XT_IM(4); XT_IM(5); XT_IM(6); XT_IM(7); XT_IM(8);
#undef XT_IM
    default: return hipErrorInvalidValue;
  }
  hipError_t e = allow_full_lds(fn);
  if (e != hipSuccess) return e;
  switch (mt) {
#define XT_IM(MTV) \
  case MTV: hipLaunchKernelGGL((conv_image_kernel<ELEM, MTV, KW>), dim3(a.nwg), dim3(512), lds, s, a); break
    XT_IM(1); XT_IM(2); XT_IM(3); XT_IM(4); XT_IM(5); XT_IM(6); XT_IM(7); XT_IM(8);
#undef XT_IM
  }
  return hipGetLastError();
}

}  // namespace

bool launch_conv2d_image(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e) {
  // XTILE_AMD_CONV_IMAGE=0 keeps these shapes on the implicit GEMM; =1 takes
  // this kernel also for small images and few workgroups (tests)
  const char* env = std::getenv("XTILE_AMD_CONV_IMAGE");
  if (env && env[0] == '0') return false;
  const bool force = env && env[0] == '1';
  const xt::ConvPlan& c = p.conv;
  if (c.elem != xt::Elem::F16 && c.elem != xt::Elem::BF16) return false;
  if (c.out_elem != xt::Elem::F32 || c.TC != c.CO || c.C % 64 || c.CO % 32 || c.KW != 3) return false;
  if (!conv_blocks_cover_output(p, 2)) return false;
  const long long HW = c.H * c.W, P = c.out_H * c.out_W;
  if (P > 256 || P < 1) return false;
  // the Blocks cover images [0, gB TB)
  const long long images = p.grid[c.cb.axis] * c.TB;
  const long long src_bytes = images * HW * c.C * 2;
  const long long filt_bytes = c.KH * c.KW * c.C * c.CO * 2;
  if (src_bytes >= (1LL << 31) || filt_bytes >= (1LL << 31)) return false;
  const long long nh = (HW + 6) / 7;
  const long long region = nh * 1008 + 16;
  const long long nsub = c.C / 64;
  const long long mt = (P + 31) / 32;
  const long long lds = std::max(nsub * region + 256 + kImNS * 3 * 4096, 16 * mt * 1024);
  if (lds > kMaxLds) return false;
  // Taken for images of at least four M tiles (128 outputs) and at least a
  // quarter of the CUs' worth of workgroups.  Measured (HIP graphs of 100
  // launches, inputs L2-resident), implicit GEMM / this kernel: 32 x 14^2 x
  // 256 -> 256 16.2 / 13.0 us, 64 x 14^2 x 256 32.3 / 23.4, 8 x 14^2 x 256
  // (64 workgroups) 12.6 / 10.7, 32 x 14^2 x 128 -> 128 9.6 / 7.7, 32 x
  // 12^2 x 256 14.4 / 10.9; but 7 x 7 images (49 outputs: each workgroup
  // streams its filter columns for few pixels) 32 x 7^2 x 512 -> 512 21.2 /
  // 22.1, 64 x 7^2 x 512 27.9 / 37.7, 32 x 7^2 x 1024 60.8 / 89.7.
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  const long long nwg = images * (c.CO / 32);
  if ((!force && (mt < 4 || nwg * 4 < cus)) || !grid_fits(nwg, 512)) return false;
  const unsigned char* src = static_cast<const unsigned char*>(bufs[c.src_arg]);
  const unsigned char* filt = static_cast<const unsigned char*>(bufs[c.filt_arg]) + c.filt_addr.c0 * 2;
  float* out = static_cast<float*>(bufs[c.out_arg]);
  for (const void* ptr : {(const void*)src, (const void*)filt, (const void*)out})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) return false;
  ImArgs a;
  a.src = src;
  a.filt = filt;
  a.out = out;
  a.src_bytes = static_cast<unsigned>(src_bytes);
  a.filt_bytes = static_cast<unsigned>(filt_bytes);
  a.H = (int)c.H;
  a.W = (int)c.W;
  a.C = (int)c.C;
  a.KH = (int)c.KH;
  a.CO = (int)c.CO;
  a.OW = (int)c.out_W;
  a.P = (int)P;
  a.pad_t = (int)c.pad_top;
  a.pad_l = (int)c.pad_left;
  a.sh = (int)c.stride_h;
  a.sw = (int)c.stride_w;
  a.dh = (int)c.dil_h;
  a.dw = (int)c.dil_w;
  a.nsub = (int)nsub;
  a.nh = (int)nh;
  a.region = (int)region;
  a.ntile = (int)(c.CO / 32);
  a.nwg = (int)nwg;
  a.d_ow = div31((unsigned)c.out_W);
  e = c.elem == xt::Elem::BF16 ? launch_im<1, 3>(a, (int)mt, (size_t)lds, s) : launch_im<0, 3>(a, (int)mt, (size_t)lds, s);
  return true;
}

}  // namespace xtk
