// xt.load_conv2d with few input channels (Cin * esize not a multiple of 16:
// the RGB stem of a CNN; any Cin whose row of channels is not a whole number
// of 16-byte pieces: 3, 5, 12, 20 ... for f16 / bf16, 3, 12, 15 ... for i8) as an
// implicit GEMM over an input patch staged in LDS, for f16 / bf16 / i8 sources
// and an f32 result.
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
//     KP = KW * Cin rounded up to the MFMA depth KS (16 for
//     v_mfma_f32_32x32x16_{f16,bf16}, 32 for v_mfma_i32_32x32x32_i8); the
//     padding positions take zero filter rows and zeroed source values.
//   * A workgroup computes 128 consecutive output pixels of one output row
//     against 64 output channels, four waves of 32 pixels x 64 channels (two
//     32 x 32 tiles).  It stages the KH input rows its pixels read (127 sw +
//     KW columns of Cin channels, zeros outside the image) and the filter's
//     64 columns (KH * KP rows, zero past each kh's KW * Cin) in LDS once, then
//     runs every K step from LDS: source fragments as element reads at the
//     pixel's patch position, filter fragments by ds_read_b64_tr_b16 / _b8.
//   * With one channel tile, the patch in one round and enough output rows
//     (the 7 x 7 stem), three workgroups a CU walk the tasks instead
//     (TASKS): filter tile and K table staged once, the next task's patch
//     loads in flight behind the current task, every patch piece's row and
//     position known at compile time, patch rows one slot per piece apart
//     (no range check before a write).  The one-workgroup-a-task form spent
//     most of its time issuing the staging's index arithmetic (~545
//     instructions a round, three rounds a wave): C8 38.1 -> 31.8 us; the
//     stores as buffer stores against the output row (a pixel past the row
//     is past the buffer: no compare and branch a store) and the unchecked
//     patch writes, 1019 -> 592 instructions a task: 25.9 us.
//   * i8: exact i32 sums, rounded to f32 once at the store.
//   * Results: a half-wave stores one 128-byte run of 32 channels per
//     accumulator register (non-temporal buffer stores against the output
//     row); pixels past the row and channels past Cout fall outside the
//     buffer and are not stored.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

typedef float sc_f16v __attribute__((ext_vector_type(16)));
typedef int sc_i16v __attribute__((ext_vector_type(16)));

enum { kScF16 = 0, kScBF16 = 1, kScI8 = 2 };

struct ScArgs {
  const unsigned char* src;   // NHWC input
  const unsigned char* filt;  // [KH*KW*C][CO]
  float* out;                 // [N][OH][OW][CO]
  unsigned src_bytes, filt_bytes;
  int H, W, C, KH, KW, CO;
  int OH, OW;
  int pad_t, pad_l, sh, sw, dh;
  int run;      // KW * C: consecutive source elements of one kh
  int K;        // KH * run: the reduction length
  int kp;       // K rounded up to the MFMA depth
  int pw;       // patch columns: 127 * sw + KW
  int npr;      // 256-element pieces a patch row
  int chunks;   // 128-pixel chunks per output row
  int ntiles;   // 64-channel tiles
  int nwg;      // workgroups
  int ntask;    // TASKS: images * OH * chunks (one channel tile)
};

// TASKS: the workgroup walks output-row tasks (one 64-channel tile, the
// patch in one round of loads, NPR 256-element pieces a patch row) instead
// of taking one: the filter tile and the K table are staged once, the next
// task's patch loads are issued as soon as the current patch is in LDS (they
// land behind the current task's K loop and stores), and each piece's patch
// row and position are compile-time constants (the counters of the one-task
// staging cost ~25 scalar instructions a piece).
template <int ELEM, bool BIG, bool TASKS = false, int NPR = 0>
__global__ __launch_bounds__(256, TASKS ? 3 : BIG ? 4 : 1) void conv2d_small_kernel(ScArgs p) {
  constexpr bool I8 = ELEM == kScI8;
  constexpr int ES = I8 ? 1 : 2;       // element bytes
  constexpr int KS = I8 ? 32 : 16;     // MFMA depth
  constexpr int FR = 64 * ES;          // filter tile row bytes
  constexpr int PPR = FR / 16;         // 16-byte pieces a filter row
  constexpr int RPR = 256 / PPR;       // filter rows a round of one piece a thread
  extern __shared__ __attribute__((aligned(16))) unsigned char sm[];
  typedef __attribute__((address_space(3))) unsigned char lds_t;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // LDS: the patch [KH rows][pw * C elements], the filter tile [kp rows][64
  // channels] (K = (kh, kw, c) in HWIO row order, zero rows past K; FR-byte
  // rows, 16-byte chunk c of row k at c ^ fsw(k) so that a transposing read's
  // rows hit distinct banks: 128-byte rows XOR 2 ((k / 2) % 2), 64-byte rows
  // XOR (k / 4) % 2), and T[k], the byte offset of K index k in a pixel's
  // patch window (kh * row pitch + (k - kh * run)) * esize.
  auto fsw = [](int k) { return I8 ? (k >> 2) & 1 : 2 * ((k >> 1) & 1); };
  const int prow = p.pw * p.C;                                 // elements per patch row
  // patch row pitch: a 16-byte multiple; with TASKS every piece's slot (no
  // piece needs a range check before its write)
  const int prow_pad = TASKS ? 256 * NPR : (prow + 16 / ES - 1) & ~(16 / ES - 1);
  unsigned char* const patch = sm;
  unsigned char* const ftile = sm + p.KH * prow_pad * ES;
  unsigned short* const T = reinterpret_cast<unsigned short*>(ftile + p.kp * FR);
  for (int k = tid; k < p.kp; k += 256) {
    const int kh = k / p.run;
    T[k] = k < p.K ? (unsigned short)((kh * prow_pad + k - kh * p.run) * ES) : 0;
  }
  const int nrow = p.KH * p.npr;       // 256-element patch pieces
  // buffer loads: an offset at or past the buffer's size (kOor) reads zero,
  // so no load sits behind a branch and a round's loads are in flight together
  constexpr unsigned kOor = 0x80000000u;  // both buffers are below 2 GiB
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(p.src), (short)0, (int)p.src_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rf =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(p.filt), (short)0, (int)p.filt_bytes, 0x00020000);
  // rounds of U patch pieces and UF filter pieces a thread, every load of a
  // round issued before the round's LDS writes (BIG: one round for the 7 x 7
  // stem, where the LDS already holds the workgroups a CU to four).  Piece t
  // of the patch is row t / npr, elements 256 (t % npr) + tid: the row's
  // image row and offset are the same for every thread.
  constexpr int U = BIG ? 28 : 12, UF = BIG ? 5 : 2;
  const int fq = tid % PPR, fk0 = tid / PPR;  // this thread's filter piece column, first row
  // this wave's 32 pixels: lane l % 32; K positions (KS / 2) (l / 32) .. + KS / 2 - 1 of a step
  const int lr = lane & 31, hi = lane >> 5;
  const int g = lane >> 4, li = lane & 15;
  typedef typename std::conditional<I8, sc_i16v, sc_f16v>::type acc_t;
  acc_t acc[2];
  const int px = wave * 32 + lr;                                // pixel within the chunk
  const unsigned char* const pwin = patch + px * p.sw * p.C * ES;  // its patch window
  // filter fragment offsets (N tile t, read h) in a step's first row block
  int boff[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int k, cb;
      if constexpr (I8) {
        k = 16 * (g >> 1) + 8 * h + (li >> 1);
        cb = t * 32 + 16 * (g & 1) + 8 * (li & 1);
      } else {
        k = 8 * (g >> 1) + 4 * h + (li >> 2);
        cb = (t * 32 + 16 * (g & 1) + 4 * (li & 3)) * 2;
      }
      boff[t][h] = k * FR + (((cb >> 4) ^ fsw(k)) << 4) + (cb & 15);
    }
  const int nsteps = p.kp / KS;
  // one K step: the lane's KS / 2 source elements through T (GUARD: the last
  // step, whose positions past K read as zero), two MFMAs
  auto step = [&](int s, auto guard) {
    constexpr bool G = decltype(guard)::value;
    const int k0 = s * KS + (KS / 2) * hi;
    unsigned a32[4];
    if constexpr (I8) {
      const uint4v t0 = *reinterpret_cast<const uint4v*>(T + k0);
      const uint4v t1 = *reinterpret_cast<const uint4v*>(T + k0 + 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned tw0 = e < 2 ? t0[2 * e] : t1[2 * e - 4], tw1 = e < 2 ? t0[2 * e + 1] : t1[2 * e - 3];
        const unsigned o[4] = {tw0 & 0xffffu, tw0 >> 16, tw1 & 0xffffu, tw1 >> 16};
        unsigned word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          unsigned x = pwin[o[b]];
          if (G && k0 + 4 * e + b >= p.K) x = 0;
          word |= x << (8 * b);
        }
        a32[e] = word;
      }
    } else {
      const uint4v t0 = *reinterpret_cast<const uint4v*>(T + k0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        unsigned lo = *reinterpret_cast<const unsigned short*>(pwin + (t0[e] & 0xffffu));
        unsigned up = *reinterpret_cast<const unsigned short*>(pwin + (t0[e] >> 16));
        if (G && k0 + 2 * e >= p.K) lo = 0;
        if (G && k0 + 2 * e + 1 >= p.K) up = 0;
        a32[e] = lo | (up << 16);
      }
    }
    const uint4v a = {a32[0], a32[1], a32[2], a32[3]};
    lds_t* const f = (lds_t*)(ftile + s * KS * FR);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      uint2v l2, h2;
      if constexpr (I8) {
        l2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                                            reinterpret_cast<int2v __attribute__((address_space(3)))*>(f + boff[t][0])));
        h2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                                            reinterpret_cast<int2v __attribute__((address_space(3)))*>(f + boff[t][1])));
      } else {
        l2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                            reinterpret_cast<short4v __attribute__((address_space(3)))*>(f + boff[t][0])));
        h2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                            reinterpret_cast<short4v __attribute__((address_space(3)))*>(f + boff[t][1])));
      }
      const uint4v b = {l2[0], l2[1], h2[0], h2[1]};
      if constexpr (I8)
        acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b),
                                                       acc[t], 0, 0, 0);
      else if constexpr (ELEM == kScBF16)
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                         acc[t], 0, 0, 0);
      else
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b),
                                                        acc[t], 0, 0, 0);
    }
  };
  // one task's K loop and stores, after its patch and the filter tile are in LDS
  auto compute_store = [&](int n, int oh, int ow0, int n0) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[t][v] = 0;
    for (int s = 0; s + 1 < nsteps; ++s) step(s, std::false_type{});
    step(nsteps - 1, std::true_type{});

    // D = A x B: lane l holds channel 32 t + l % 32 of N tile t, register v
    // pixel 8 (v / 4) + 4 (l / 32) + v % 4 of the wave's 32.  Buffer stores
    // against the output row: a pixel past OW is past the buffer's records
    // and is dropped, a channel past Cout gets an offset past them.
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        p.out + (((long long)n * p.OH + oh) * p.OW) * p.CO, (short)0, p.OW * p.CO * 4, 0x00020000);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int co = n0 + t * 32 + lr;
      const unsigned lbase = co < p.CO ? (unsigned)(((ow0 + wave * 32 + 4 * hi) * p.CO + co) * 4) : kOor;
#pragma unroll
      for (int v = 0; v < 16; ++v)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(static_cast<float>(acc[t][v])), ro,
                                              lbase + (unsigned)((8 * (v >> 2) + (v & 3)) * p.CO * 4), 0, 2);
    }
  };

  if constexpr (!TASKS) {
    // workgroup -> (image, output row, pixel chunk, channel tile); with a
    // multiple of 8 workgroups the 8 XCDs (dispatched round-robin) receive
    // contiguous runs of output rows, which share their input rows in one L2
    int L = blockIdx.x;
    if ((p.nwg & 7) == 0) L = (L & 7) * (p.nwg >> 3) + (L >> 3);
    const int nt = L % p.ntiles;
    L /= p.ntiles;
    const int ch = L % p.chunks;
    L /= p.chunks;
    const int oh = L % p.OH;
    const int n = L / p.OH;
    const int ow0 = ch * 128, n0 = nt * 64;

    const int iw_lo = ow0 * p.sw - p.pad_l;
    // a patch row's elements inside the image: columns [0, W), a range of j
    const int jlo = max(0, -iw_lo) * p.C, jhi = min(prow, (p.W - iw_lo) * p.C);
    int kh_t = 0, i_t = 0;                      // piece t's row and position, t = r U + u
    for (int r = 0; r * U < nrow || r * UF * RPR < p.kp; ++r) {
      unsigned short v[U];
      int dst[U];
      uint4v w[UF];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int ih = oh * p.sh - p.pad_t + kh_t * p.dh;
        const int j = tid + 256 * i_t;
        const int rowoff = ((n * p.H + ih) * p.W + iw_lo) * p.C;
        const bool in = r * U + u < nrow && (unsigned)ih < (unsigned)p.H && j >= jlo && j < jhi;
        const unsigned off = in ? (unsigned)(rowoff + j) * ES : kOor;
        if constexpr (I8)
          v[u] = __builtin_amdgcn_raw_buffer_load_b8(rs, off, 0, 0);
        else
          v[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
        dst[u] = r * U + u < nrow && j < prow_pad ? kh_t * prow_pad + j : -1;
        if (++i_t == p.npr) {
          i_t = 0;
          ++kh_t;
        }
      }
#pragma unroll
      for (int u = 0; u < UF; ++u) {
        const int k = fk0 + RPR * (r * UF + u);
        const bool in = k < p.K && n0 + fq * (16 / ES) < p.CO;
        w[u] = __builtin_amdgcn_raw_buffer_load_b128(rf, in ? (unsigned)(k * p.CO + n0 + fq * (16 / ES)) * ES : kOor,
                                                     0, 0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (dst[u] >= 0) {
          if constexpr (I8)
            patch[dst[u]] = (unsigned char)v[u];
          else
            reinterpret_cast<unsigned short*>(patch)[dst[u]] = v[u];
        }
      }
#pragma unroll
      for (int u = 0; u < UF; ++u) {
        const int k = fk0 + RPR * (r * UF + u);
        if (k < p.kp) *reinterpret_cast<uint4v*>(ftile + k * FR + ((fq ^ fsw(k)) << 4)) = w[u];
      }
    }
    __syncthreads();
    compute_store(n, oh, ow0, n0);
  } else {
    // the filter tile (channels 0 .. 63), rounds of UF pieces a thread
    for (int r = 0; r * UF * RPR < p.kp; ++r) {
      uint4v w[UF];
#pragma unroll
      for (int u = 0; u < UF; ++u) {
        const int k = fk0 + RPR * (r * UF + u);
        const bool in = k < p.K && fq * (16 / ES) < p.CO;
        w[u] = __builtin_amdgcn_raw_buffer_load_b128(rf, in ? (unsigned)(k * p.CO + fq * (16 / ES)) * ES : kOor, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < UF; ++u) {
        const int k = fk0 + RPR * (r * UF + u);
        if (k < p.kp) *reinterpret_cast<uint4v*>(ftile + k * FR + ((fq ^ fsw(k)) << 4)) = w[u];
      }
    }
    // tasks (image, output row, pixel chunk): each XCD (workgroups reach the
    // 8 XCDs round-robin; the grid is a multiple of 8) takes a contiguous
    // range of them, its G / 8 workgroups the range's tasks j, j + G / 8, ...
    // (neighbouring rows, which share input rows, in one L2 at once)
    const int ntask = p.ntask, gx = (int)(gridDim.x >> 3), xcd = blockIdx.x & 7;
    const int tend = (int)((long long)(xcd + 1) * ntask / 8);
    int task = (int)((long long)xcd * ntask / 8) + (int)(blockIdx.x >> 3);
    // the patch of one task: piece u (patch row u / NPR, elements 256 (u %
    // NPR) + tid) in register v[u]; rows past KH load nothing
    static_assert(NPR >= 1 && NPR <= U, "pieces a patch row");
    constexpr int KHM = U / NPR;  // patch rows one round holds
    unsigned short v[U];
    auto load_patch = [&](int t) {
      const int ch = t % p.chunks, r = t / p.chunks, oh = r % p.OH, n = r / p.OH;
      const int iw_lo = ch * 128 * p.sw - p.pad_l;
      const int jlo = max(0, -iw_lo) * p.C, jhi = min(prow, (p.W - iw_lo) * p.C);
      const int ih0 = oh * p.sh - p.pad_t;
#pragma unroll
      for (int kh = 0; kh < KHM; ++kh) {
        const int ih = ih0 + kh * p.dh;
        const bool row_in = kh < p.KH && (unsigned)ih < (unsigned)p.H;
        const int rowoff = ((n * p.H + ih) * p.W + iw_lo) * p.C;
#pragma unroll
        for (int i = 0; i < NPR; ++i) {
          const int j = tid + 256 * i;
          const bool in = row_in && j >= jlo && j < jhi;
          const unsigned off = in ? (unsigned)(rowoff + j) * ES : kOor;
          if constexpr (I8)
            v[kh * NPR + i] = __builtin_amdgcn_raw_buffer_load_b8(rs, off, 0, 0);
          else
            v[kh * NPR + i] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
        }
      }
    };
    if (task < tend) load_patch(task);
    while (task < tend) {
#pragma unroll
      for (int kh = 0; kh < KHM; ++kh)
        if (kh < p.KH) {
#pragma unroll
          for (int i = 0; i < NPR; ++i) {
            if constexpr (I8)
              patch[kh * prow_pad + tid + 256 * i] = (unsigned char)v[kh * NPR + i];
            else
              reinterpret_cast<unsigned short*>(patch)[kh * prow_pad + tid + 256 * i] = v[kh * NPR + i];
          }
        }
      __syncthreads();  // the patch (and, the first time, the filter tile and T) in LDS
      const int next = task + gx;
      if (next < tend) load_patch(next);
      const int ch = task % p.chunks, r = task / p.chunks;
      compute_store(r / p.OH, r % p.OH, ch * 128, 0);
      task = next;
      if (task < tend) __syncthreads();  // every wave is done with the patch
    }
  }
}

template <int E>
hipError_t launch_sc(bool big, int tasks_npr, long long wgs, size_t lds, hipStream_t s, const ScArgs& a) {
  // the task walk stages with the one-round constants (28 patch pieces a
  // thread), NPR of them a patch row
  auto kern = tasks_npr == 1   ? conv2d_small_kernel<E, true, true, 1>
              : tasks_npr == 2 ? conv2d_small_kernel<E, true, true, 2>
              : tasks_npr == 3 ? conv2d_small_kernel<E, true, true, 3>
              : tasks_npr == 4 ? conv2d_small_kernel<E, true, true, 4>
              : big            ? conv2d_small_kernel<E, true>
                               : conv2d_small_kernel<E, false>;
  const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(kern));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(256), lds, s, a);
  return hipGetLastError();
}

}  // namespace

bool launch_conv2d_small(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e) {
  const xt::ConvPlan& c = p.conv;
  const bool i8 = c.elem == xt::Elem::I8;
  if (c.elem != xt::Elem::F16 && c.elem != xt::Elem::BF16 && !i8) return false;
  const long long es = i8 ? 1 : 2, ks = i8 ? 32 : 16, fr = 64 * es;
  // 16-byte filter pieces: Cout * esize a multiple of 16
  if (c.out_elem != xt::Elem::F32 || c.TC != c.CO || c.dil_w != 1 || c.C * es % 16 == 0 || c.CO * es % 16) return false;
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
  if (c.filt_addr.sx || c.filt_addr.sy || c.filt_addr.sz || c.filt_addr.c0 * es % 16) return false;
  const long long images = gB * c.TB;
  const long long run = c.KW * c.C, K = c.KH * run, kp = (K + ks - 1) / ks * ks;
  const long long pw = 127 * c.stride_w + c.KW;
  const long long prow_pad = (pw * c.C * es + 15) / 16 * 16 / es;
  // patch, filter tile and the K table (16-bit byte offsets into the patch)
  const size_t lds = (size_t)(c.KH * prow_pad * es + kp * fr + kp * 2);
  if (c.KH * prow_pad * es >= 65536) return false;
  if (lds > size_t(kMaxLds) || images > c.N) return false;
  const long long chunks = (c.out_W + 127) / 128, ntiles = (c.CO + 63) / 64;
  const long long wgs = images * c.out_H * chunks * ntiles;
  const long long src_bytes = images * c.H * c.W * c.C * es, filt_bytes = c.KH * run * c.CO * es;
  if (!grid_fits(wgs, 256) || src_bytes >= (1LL << 31) || filt_bytes >= (1LL << 31)) return false;
  const unsigned char* src = static_cast<const unsigned char*>(bufs[c.src_arg]);
  const unsigned char* filt = static_cast<const unsigned char*>(bufs[c.filt_arg]) + c.filt_addr.c0 * es;
  float* out = static_cast<float*>(bufs[c.out_arg]);
  if (reinterpret_cast<uintptr_t>(filt) % 16 || reinterpret_cast<uintptr_t>(src) % es) return false;
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
  a.K = (int)K;
  a.kp = (int)kp;
  a.pw = (int)pw;
  a.npr = (int)((prow_pad + 255) / 256);
  a.chunks = (int)chunks;
  a.ntiles = (int)ntiles;
  a.nwg = (int)wgs;
  // four workgroups a CU or fewer by LDS: the register-heavy one-round staging
  const bool big = lds * 5 > size_t(kMaxLds);
  // One channel tile, the patch in one round of loads and enough tasks
  // (output-row chunks): three workgroups a CU (a multiple of 8; the next
  // patch's registers leave room for three) walk them,
  // the filter staged once per workgroup and the next task's patch in flight
  // behind the current task.
  const long long ntask = images * c.out_H * chunks;
  // (patch rows 256 * npr elements apart: three workgroups' LDS a CU, byte
  // offsets into the patch below 2^16 for the K table)
  const size_t lds_tasks = (size_t)(c.KH * 256 * a.npr * es + kp * fr + kp * 2);
  const bool tasks = ntiles == 1 && a.npr <= 4 && c.KH * a.npr <= 28 && ntask >= 2048 &&
                     c.KH * 256 * a.npr * es < 65536 && 3 * lds_tasks <= size_t(kMaxLds);
  if (tasks) {
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 2)
      cus = 256;
    a.ntask = (int)ntask;
    a.nwg = (int)(std::min<long long>(ntask, 3LL * cus) & ~7LL);
  }
  const long long grid = tasks ? a.nwg : wgs;
  const int tasks_npr = tasks ? a.npr : 0;
  const size_t lds_launch = tasks ? lds_tasks : lds;
  if (i8)
    e = launch_sc<kScI8>(big, tasks_npr, grid, lds_launch, s, a);
  else if (c.elem == xt::Elem::BF16)
    e = launch_sc<kScBF16>(big, tasks_npr, grid, lds_launch, s, a);
  else
    e = launch_sc<kScF16>(big, tasks_npr, grid, lds_launch, s, a);
  return true;
}

}  // namespace xtk
