// xt.load_conv2d with few input channels (Cin * 2 bytes below 16 or not a
// multiple of 16: the RGB stem of a CNN, Cin = 1 .. 7) as an implicit GEMM
// over an input patch staged in LDS, for f16 / bf16 sources and an f32 result.
//
// Semantics (lib/xt/XTOps.cpp:43-90, lib/xt/XTToNova.cpp:110-142,353-437):
//   out[n, oh, ow, o] = sum_{kh,kw,c} src[n, oh*sh - pad_t + kh*dh,
//                                         ow*sw - pad_l + kw, c] * f[kh, kw, c, o]
// (column dilation 1), source elements outside the image read as zero.  Used
// when the Blocks tile the whole output with one filter and every output
// channel (any batch tile), like the implicit-GEMM kernel (conv_igemm.hip),
// whose 16-byte channel runs these channel counts do not have.
//
//   * For a fixed kh, the (kw, c) terms of a pixel are KW * Cin consecutive
//     source elements of one input row (column dilation 1), and f[kh] is
//     KW * Cin consecutive filter rows (HWIO).  So K runs kh by kh in runs of
//     KP = KW * Cin rounded up to 16 (one v_mfma_f32_32x32x16 step each 16);
//     the padding positions take zero filter rows and zeroed source values.
//   * A workgroup computes 128 consecutive output pixels of one output row
//     against 64 output channels, four waves of 32 pixels x 64 channels (two
//     32 x 32 tiles).  It stages the KH input rows its pixels read (128 sw +
//     KW - 1 columns of Cin channels, zeros outside the image) and the filter's
//     64 columns (KH * KP rows, zero past each kh's KW * Cin) in LDS once, then
//     runs every K step from LDS: source fragments as 2-byte reads at the
//     pixel's patch position, filter fragments by ds_read_b64_tr_b16.
//   * Results: a half-wave stores one 128-byte run of 32 channels per
//     accumulator register (non-temporal); pixels past the row and channels
//     past Cout are not stored.
#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

typedef float sc_f16v __attribute__((ext_vector_type(16)));

struct ScArgs {
  const unsigned short* src;  // NHWC input
  const unsigned short* filt; // [KH*KW*C][CO]
  float* out;                 // [N][OH][OW][CO]
  unsigned src_bytes, filt_bytes;
  int H, W, C, KH, KW, CO;
  int OH, OW;
  int pad_t, pad_l, sh, sw, dh;
  int run;      // KW * C: consecutive source elements of one kh
  int kp;       // run rounded up to 16
  int pw;       // patch columns: 127 * sw + KW
  int chunks;   // 128-pixel chunks per output row
  int ntiles;   // 64-channel tiles
  Div31 d_prow; // / patch row pitch (pw * C rounded up to 8)
  Div31 d_kp;   // / kp
};

template <bool BF16, bool BIG>
__global__ __launch_bounds__(256) void conv2d_small_kernel(ScArgs p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char sm[];
  typedef __attribute__((address_space(3))) unsigned char lds_t;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int L = blockIdx.x;
  const int nt = L % p.ntiles;
  L /= p.ntiles;
  const int ch = L % p.chunks;
  L /= p.chunks;
  const int oh = L % p.OH;
  const int n = L / p.OH;
  const int ow0 = ch * 128, n0 = nt * 64;

  // patch [KH rows][pw * C elements] of f16 / bf16, then the filter tile
  // [KH * kp rows][64 channels] (128-byte rows, chunk c of row k at
  // c ^ 2 ((k / 2) % 2) so a transposing read's four rows hit distinct banks).
  // Each thread issues U loads before it writes any of them to LDS, so that
  // their latencies overlap.
  const int prow = p.pw * p.C;                       // elements per patch row
  const int prow_pad = (prow + 7) & ~7;              // 16-byte multiple
  unsigned short* patch = reinterpret_cast<unsigned short*>(sm);
  unsigned char* ftile = sm + (size_t)p.KH * prow_pad * 2;
  const int iw_lo = ow0 * p.sw - p.pad_l;
  // a patch row's elements inside the image: columns [0, W), a range of j
  const int jlo = max(0, -iw_lo) * p.C, jhi = min(prow, (p.W - iw_lo) * p.C);
  const long long img = (long long)n * p.H;
  const int total = p.KH * prow_pad;
  // buffer loads: an offset at or past the buffer's size (kOor) reads zero,
  // so no load sits behind a branch and all U are in flight together
  constexpr unsigned kOor = 0x80000000u;  // both buffers are below 2 GiB
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(p.src), (short)0, (int)p.src_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rf =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(p.filt), (short)0, (int)p.filt_bytes, 0x00020000);
  // rounds of U patch elements and UF filter pieces a thread, every load of a
  // round issued before the round's LDS writes (BIG: one round for the
  // 7 x 7 stem, where the LDS already holds the workgroups a CU to four)
  constexpr int U = BIG ? 24 : 8, UF = BIG ? 8 : 2;
  const int ftotal = p.KH * p.kp * 8;  // 16-byte pieces: 8 per 64-channel row
  for (int r = 0; r * 256 * U < total || r * 256 * UF < ftotal; ++r) {
    unsigned short v[U];
    uint4v w[UF];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = tid + 256 * (r * U + u);
      const int kh = (int)p.d_prow((unsigned)e), j = e - kh * prow_pad;
      const int ih = oh * p.sh - p.pad_t + kh * p.dh;
      const bool in = e < total && j >= jlo && j < jhi && (unsigned)ih < (unsigned)p.H;
      v[u] = __builtin_amdgcn_raw_buffer_load_b16(
          rs, in ? (unsigned)(((img + ih) * p.W + iw_lo) * p.C + j) * 2u : kOor, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < UF; ++u) {
      const int e = tid + 256 * (r * UF + u), k = e >> 3, q = e & 7;
      const int kh = (int)p.d_kp((unsigned)k), j = k - kh * p.kp;
      const bool in = e < ftotal && j < p.run && n0 + 8 * q < p.CO;
      w[u] = __builtin_amdgcn_raw_buffer_load_b128(rf, in ? (unsigned)((kh * p.run + j) * p.CO + n0 + 8 * q) * 2u : kOor,
                                                   0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = tid + 256 * (r * U + u);
      if (e < total) patch[e] = v[u];
    }
#pragma unroll
    for (int u = 0; u < UF; ++u) {
      const int e = tid + 256 * (r * UF + u), k = e >> 3, q = e & 7;
      if (e < ftotal) *reinterpret_cast<uint4v*>(ftile + k * 128 + ((q ^ (2 * ((k >> 1) & 1))) << 4)) = w[u];
    }
  }
  __syncthreads();

  // this wave's 32 pixels: lane l % 32; K positions 8 (l / 32) .. + 7 of a step
  const int lr = lane & 31, hi = lane >> 5;
  const int g = lane >> 4, li = lane & 15;
  sc_f16v acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[t][v] = 0.f;
  const int px = wave * 32 + lr;                  // pixel within the chunk
  const int pbase = px * p.sw * p.C;              // its first element in a patch row
  // filter fragment offsets (N tile j, read h) in a step's first row block
  int boff[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = 8 * (g >> 1) + 4 * h + (li >> 2);
      const int cb = (t * 32 + 16 * (g & 1) + 4 * (li & 3)) * 2;
      boff[t][h] = k * 128 + (((cb >> 4) ^ (2 * ((k >> 1) & 1))) << 4) + (cb & 15);
    }
  for (int kh = 0; kh < p.KH; ++kh) {
    const unsigned short* prow_p = patch + kh * prow_pad + pbase;
    for (int j0 = 0; j0 < p.kp; j0 += 16) {
      // source fragment: 8 consecutive elements of the run (zero past it)
      unsigned a32[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + 8 * hi + 2 * e;
        const unsigned lo = j < p.run ? prow_p[j] : 0u;
        const unsigned up = j + 1 < p.run ? prow_p[j + 1] : 0u;
        a32[e] = lo | (up << 16);
      }
      const uint4v a = {a32[0], a32[1], a32[2], a32[3]};
      lds_t* const f = (lds_t*)(ftile + (kh * p.kp + j0) * 128);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint2v l2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                         reinterpret_cast<short4v __attribute__((address_space(3)))*>(
                                                             f + boff[t][0])));
        const uint2v h2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                         reinterpret_cast<short4v __attribute__((address_space(3)))*>(
                                                             f + boff[t][1])));
        const uint4v b = {l2[0], l2[1], h2[0], h2[1]};
        if constexpr (BF16)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                           acc[t], 0, 0, 0);
        else
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b),
                                                          acc[t], 0, 0, 0);
      }
    }
  }

  // D = A x B: lane l holds channel 32 t + l % 32 of N tile t, register v
  // pixel 8 (v / 4) + 4 (l / 32) + v % 4 of the wave's 32
  float* const orow = p.out + (((long long)n * p.OH + oh) * p.OW) * p.CO;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int co = n0 + t * 32 + lr;
    if (co >= p.CO) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int ow = ow0 + wave * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
      if (ow < p.OW) __builtin_nontemporal_store(static_cast<float>(acc[t][v]), orow + (long long)ow * p.CO + co);
    }
  }
}

}  // namespace

bool launch_conv2d_small(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e) {
  const xt::ConvPlan& c = p.conv;
  if (c.elem != xt::Elem::F16 && c.elem != xt::Elem::BF16) return false;
  if (c.out_elem != xt::Elem::F32 || c.TC != c.CO || c.dil_w != 1 || c.C * 2 % 16 == 0 || c.CO % 8) return false;
  if (c.cb.axis < 0 || c.ch.axis < 0 || c.cw.axis < 0 || c.cb.axis == c.ch.axis || c.cb.axis == c.cw.axis ||
      c.ch.axis == c.cw.axis)
    return false;
  // the Blocks tile images [0, gB TB) x every output row and column once, in
  // the output's natural NHWC addressing, with one filter
  const long long gB = p.grid[c.cb.axis], gH = p.grid[c.ch.axis], gW = p.grid[c.cw.axis];
  if (gH * c.TH != c.out_H || gW * c.TW != c.out_W || c.out_C != c.CO) return false;
  auto step = [&](const xt::TileAddr& t, int axis) { return axis == 0 ? t.sx : axis == 1 ? t.sy : t.sz; };
  const long long plane = c.out_H * c.out_W * c.out_C;
  if (c.out_addr.c0 != 0 || (gB > 1 && step(c.out_addr, c.cb.axis) != c.TB * plane) ||
      (gH > 1 && step(c.out_addr, c.ch.axis) != c.TH * c.out_W * c.out_C) ||
      (gW > 1 && step(c.out_addr, c.cw.axis) != c.TW * c.out_C))
    return false;
  if (c.filt_addr.sx || c.filt_addr.sy || c.filt_addr.sz || c.filt_addr.c0 % 8) return false;
  const long long images = gB * c.TB;
  const long long run = c.KW * c.C, kp = (run + 15) / 16 * 16;
  const long long pw = 127 * c.stride_w + c.KW;
  const long long prow_pad = (pw * c.C + 7) / 8 * 8;
  const size_t lds = (size_t)(c.KH * prow_pad * 2 + c.KH * kp * 128);
  if (lds > size_t(kMaxLds) || images > c.N) return false;
  const long long chunks = (c.out_W + 127) / 128, ntiles = (c.CO + 63) / 64;
  const long long wgs = images * c.out_H * chunks * ntiles;
  const long long src_bytes = images * c.H * c.W * c.C * 2, filt_bytes = c.KH * run * c.CO * 2;
  if (!grid_fits(wgs, 256) || src_bytes >= (1LL << 31) || filt_bytes >= (1LL << 31)) return false;
  const unsigned short* src = static_cast<const unsigned short*>(bufs[c.src_arg]);
  const unsigned short* filt = static_cast<const unsigned short*>(bufs[c.filt_arg]) + c.filt_addr.c0;
  float* out = static_cast<float*>(bufs[c.out_arg]);
  if (reinterpret_cast<uintptr_t>(filt) % 16) return false;
  ScArgs a;
  a.src = src;
  a.filt = filt;
  a.out = out;
  a.src_bytes = (unsigned)src_bytes;
  a.filt_bytes = (unsigned)filt_bytes;
  a.H = (int)c.H;
  a.W = (int)c.W;
  a.C = (int)c.C;
  a.KH = (int)c.KH;
  a.KW = (int)c.KW;
  a.CO = (int)c.CO;
  a.OH = (int)c.out_H;
  a.OW = (int)c.out_W;
  a.pad_t = (int)c.pad_top;
  a.pad_l = (int)c.pad_left;
  a.sh = (int)c.stride_h;
  a.sw = (int)c.stride_w;
  a.dh = (int)c.dil_h;
  a.run = (int)run;
  a.kp = (int)kp;
  a.pw = (int)pw;
  a.chunks = (int)chunks;
  a.ntiles = (int)ntiles;
  a.d_prow = div31((unsigned)prow_pad);
  a.d_kp = div31((unsigned)kp);
  // four workgroups a CU or fewer by LDS: the register-heavy one-round staging
  const bool big = lds * 5 > size_t(kMaxLds);
  const bool bf = c.elem == xt::Elem::BF16;
  auto k = bf ? (big ? conv2d_small_kernel<true, true> : conv2d_small_kernel<true, false>)
              : (big ? conv2d_small_kernel<false, true> : conv2d_small_kernel<false, false>);
  hipLaunchKernelGGL(k, dim3((unsigned)wgs), dim3(256), lds, s, a);
  e = hipGetLastError();
  return true;
}

}  // namespace xtk
