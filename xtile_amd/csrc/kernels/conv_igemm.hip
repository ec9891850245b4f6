// xt.load_conv2d as an implicit GEMM whose operands reach LDS by DMA: the path
// for filters too large for the LDS-resident filter of the band and
// persistent kernels (conv.hip), e.g. 3x3 convolutions with 128 or more input
// and output channels.
//
// Semantics (lib/xt/XTOps.cpp:43-90, lib/xt/XTToNova.cpp:110-142,353-437):
//   out[n, oh, ow, o] = sum_{kh,kw,c} src[n, oh*sh - pad_t + kh*dh,
//                                         ow*sw - pad_l + kw*dw, c] * f[kh, kw, c, o]
// with source elements outside the image read as zero.  Used when the Blocks
// tile the whole output (TB images per Block, every output channel, one
// filter) and Cin * esize, Cout * esize are multiples of 16, so the launch is
// one GEMM:
//   M = N*OH*OW output pixels (NHWC order: the output is C[M][CO]),
//   N = CO, K = KH*KW*Cin in the filter's (kh, kw, c) order (B = f as
//   [K][CO], row-major HWIO).
// Every output pixel sums its K terms in the same order as the other conv
// kernels; Blocks are independent (README.md:85-89), so the regrouping is a
// scheduling choice.
//
//   * Workgroup tiles of 128 pixels x 128 channels (Cout a multiple of 128)
//     or 256 x 64, four waves of 64 x 64 (2 x 2 tiles of
//     v_mfma_f32_32x32x16_{f16,bf16}, f32 sums, or v_mfma_i32_32x32x32_i8,
//     exact i32 sums rounded to f32 once); 64 or 80 KB of LDS, so two
//     workgroups share a CU and one's barrier waits are the other's MFMA time.
//     Deep layers, whose 128 x 128 tiles would fill at most half the CUs,
//     take 64 x 128 tiles of four 32 x 64 waves with 128-byte stages (96 KB)
//     and eight more waves that only issue the DMA (below).
//   * A K stage is KB = 64 (or 128) bytes of one tap's channels in every
//     pixel row (32 f16 / bf16 or 64 i8 channels a 64-byte stage; a tap's
//     last stage is padded with zeros when Cin is not a multiple of that, and
//     a channel tile past Cout reads zeros and is not stored):
//     A [BM rows][KB] is an im2col gather done by the DMA itself: lane L of
//     A instruction i fetches 16 bytes of pixel row (1024 / KB) i + L / (KB /
//     16) at the tap's source position, or, outside the image (padding) or
//     past M, an offset past the buffer's end, which the DMA writes as zeros.
//     B [KB / esize k][BN esize B] holds the stage's filter rows for BN
//     output channels.
//   * LDS layouts as in the DMA GEMM (gemm.hip): A row r keeps its 16-byte
//     chunk c at c ^ ((r / (256 / KB)) % (KB / 16)), B row k at c ^
//     ig_bsw(k); A fragments are
//     ds_read_b128, B fragments ds_read_b64_tr_b16 / _tr_b8 (K-contiguous
//     lanes from the channel-contiguous filter rows).
//   * Four stages in LDS, three in flight (the pipeline is described at the
//     loop).
//   * Results: a half-wave stores one 128-byte run of 32 channels per
//     accumulator register (non-temporal); rows past M are not stored.
//   * When the tiles fill at most half the CUs (deep layers: few pixels, many
//     channels), f16 / bf16 tiles split K into ranges of whole stages, one
//     workgroup each, whose partial sums are added atomically into the
//     zero-filled output (so the f32 addition order, and the last bits,
//     vary between runs; i8 is never split and stays exact).
//   * Measured (one MI355X, 30 launches, inputs not rotated): 3 x 3, stride 1,
//     batch 32: 28 x 28 x 128 -> 128 18.3 us (405 TFLOP/s; 161 us on the
//     generic kernel before), 14 x 14 x 256 -> 256 29.7 us (256 us), 7 x 7 x
//     512 -> 512 53.4 us (341 us; 52 workgroups for 256 CUs); 1 x 1 56 x 56 x
//     256 -> 64 16.5 us (the per-unit kernel: 19.7).  C4's shape runs on the
//     band kernel: this one re-reads every input pixel once per tap from L2
//     and took 17.3 us there against 13.0.
#include <algorithm>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr unsigned kIgOutOfRange = 0x80000000u;  // the input and the filter are < 2 GiB
typedef float float16v_t __attribute__((ext_vector_type(16)));

struct IgArgs {
  const unsigned char* src;   // NHWC input
  const unsigned char* filt;  // [K][CO]
  float* out;                 // [M][CO]
  unsigned src_bytes, filt_bytes;
  int H, W, C, KW, CO;
  int OH, OW;
  int pad_t, pad_l, sh, sw, dh, dw;
  int M;        // N * OH * OW
  int stages;   // stages of KB bytes of one tap's channels (64 or 128)
  int cs;       // stages per tap: C * esize / KB, rounded up
  int ntiles;   // channel tiles: CO / BN
  int tiles;    // ceil(M / BM) * ntiles
  int ksplit;   // K ranges per tile (1: one workgroup per tile)
  int kstages;  // the shortest K range: range r covers stages [r S / ksplit, (r + 1) S / ksplit)
  int nwg;      // tiles * ksplit
  int rot;      // 1: a whole-K tile walks its stages from (pixel tile % stages), wrapping
  Div31 d_ohw, d_ow;
};

enum { kIgF16 = 0, kIgBF16 = 1, kIgI8 = 2 };
typedef int int16v_t __attribute__((ext_vector_type(16)));

// f16 / bf16 accumulate in f32; i8 in i32 (exact), rounded to f32 once when stored
template <int ELEM>
struct IgAcc {
  typedef float16v_t type;
};
template <>
struct IgAcc<kIgI8> {
  typedef int16v_t type;
};

template <int ELEM>
__device__ __forceinline__ typename IgAcc<ELEM>::type ig_mfma(uint4v a, uint4v b, typename IgAcc<ELEM>::type c) {
  if constexpr (ELEM == kIgI8)
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0,
                                                 0, 0);
  else if constexpr (ELEM == kIgBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}

// B row k (BR = BN * esize bytes) keeps its 16-byte chunk c at c ^ ig_bsw(k),
// so that the rows one 16-lane group of a transposing read covers fall in
// distinct bank groups of the 256-byte bank window.  16-bit: four rows of 32
// bytes (ds_read_b64_tr_b16); rows of 256 bytes XOR 4 (k % 4), of 128 bytes
// XOR 2 ((k / 2) % 2).  8-bit: eight rows of 16 bytes (ds_read_b64_tr_b8);
// rows of 128 bytes XOR (k / 2) % 4, of 64 bytes XOR (k / 4) % 2.
template <int ES, int BR>
__device__ __forceinline__ int ig_bsw(int k) {
  if constexpr (ES == 2) return BR == 256 ? 4 * (k & 3) : 2 * ((k >> 1) & 1);
  else return BR == 128 ? (k >> 1) & 3 : (k >> 2) & 1;
}

// BM x BN workgroup tiles, four waves in a WGM x (4 / WGM) layout of WTM x
// WTN wave tiles: (BM, BN) = (128, 128) with 2 x 2 waves of 64 x 64, (256,
// 64) with 4 x 1, or (64, 128) with 2 x 2 waves of 32 x 64.  A K stage is KBY
// bytes of one tap's channels (64, or 128 for the 64 x 128 tiles).
//
// LW > 0: LW more waves, 4 .. 3 + LW, that only issue the DMA, while waves
// 0-3 only read fragments and run the MFMAs.  A wave waits in issue until
// the CU's address unit takes each DMA instruction (~50 B/clk a CU for these
// gathers), so with one wave per SIMD doing both, a deep layer's stage spent
// ~470 cycles issuing its DMA and then ~455 on its fragments and MFMAs, one
// after the other (s_memtime stamps, 32 x 14^2 x 256 -> 256); split, the two
// run side by side and a stage takes ~740 (18.8 -> 17.5 us; four loader
// waves 17.9).  Reading each stage's fragments during the previous stage's
// MFMAs, or two K groups of 64 x 64 waves that halve the filter-fragment
// reads, measured slower on top of it.
template <int ELEM, int BM, int BN, int WTM = 64, int WTN = 64, int KBY = 64, int LW = 0, int NSTAGES = 4>
__global__ __launch_bounds__(64 * (4 + LW), LW == 0 && NSTAGES * KBY * (BM + BN) <= 80 * 1024 ? 2 : 1) void conv_igemm_kernel(IgArgs p) {
  // stages in LDS (64 or 80 KB, two workgroups a CU): five, or a pipeline
  // that also read each stage's fragments during the previous stage's MFMAs
  // and spread the DMA over them, measured slower on 3 x 3 convs with 128 to
  // 512 channels (e.g. 28 x 28 x 128: 18.3 us with this loop at four stages,
  // 19.2 at five, 21.1 / 23.2 pipelined); eight stages (one workgroup a CU)
  // left 32 x 14^2 x 256 -> 256 unchanged (29.0 / 30.4 us)
  constexpr int NS = NSTAGES;
  static_assert(NS == 4 || (LW > 0 && NS >= 3 && NS <= 5), "stages in LDS");
  constexpr int ES = ELEM == kIgI8 ? 1 : 2;  // bytes per element
  // a stage is KB bytes of K (KB / esize channels of one tap); a K step of
  // the MFMAs is 32 bytes (KSR filter rows), KSTEPS of them a stage.  A DMA
  // instruction fills RA pixel rows of CA 16-byte chunks; a row keeps its
  // chunk c at c ^ ((r / SWD) % CA), so that the 16 rows one 16-lane group
  // of a fragment read covers fall in distinct bank groups of the 256-byte
  // bank window.
  constexpr int KB = KBY, AB = BM * KB, BR = BN * ES, KR = KB / ES, KSR = 32 / ES, KSTEPS = KB / 32;
  constexpr int RA = 1024 / KB, CA = KB / 16, SWD = 256 / KB;
  constexpr int STAGE = AB + KR * BR;  // 16, 20 or 24 KB
  // whole-K results staged through LDS for 16-byte stores (below): with
  // loader waves, when the tile's results fit the stage buffers
  constexpr bool STAGED = LW > 0 && BM * (BN * 4 + 32) <= NS * STAGE;
  typedef typename IgAcc<ELEM>::type acc_t;
  constexpr int WGM = BM / WTM, WGN = 4 / WGM;
  static_assert(WGM * WGN == 4 && BN == WTN * WGN, "wave layout");
  constexpr int MI = WTM / 32, NI = WTN / 32;
  constexpr int DW = LW ? LW : 4;            // waves sharing the DMA
  constexpr int PA = BM * KB / (1024 * DW);  // A DMA instructions per DMA wave and stage (RA rows each)
  constexpr int PB = BN * KB / (1024 * DW);  // B DMA instructions per DMA wave and stage
  constexpr int PER = PA + PB;               // DMA instructions per DMA wave and stage
  static_assert(PA * 1024 * DW == BM * KB && PB * 1024 * DW == BN * KB, "DMA share");
  constexpr int CPR = BR / 16, RPI = 1024 / BR;  // B chunks per row, rows per DMA instruction
  typedef __attribute__((address_space(3))) unsigned char lds_t;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * STAGE];
  auto buf = [&](int q) { return smem + (q % NS) * STAGE; };

  // workgroup -> (K range, pixel tile, channel tile).  Workgroups are dealt
  // to the 8 XCDs round-robin (id % 8); each XCD takes a contiguous run of
  // the logical order (the first nwg % 8 XCDs one more), so the channel tiles
  // of a pixel tile and neighbouring pixel tiles share input rows and filter
  // columns in one L2.  (Without it a deep layer's whole input and filter,
  // 4.4 MB for 32 x 14^2 x 256 -> 256, passed through every XCD's 4 MB L2.)
  int L = xcd_contiguous(blockIdx.x, p.nwg);
  const int kr = L / p.tiles;
  L -= kr * p.tiles;
  const int mt = L / p.ntiles;
  const int m0 = mt * BM, n0 = (L - mt * p.ntiles) * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the wave's share of the DMA (every wave's, or a loader wave's)
  const int dw = LW ? wave - 4 : wave;
  const int wm = wave / WGN, wn = wave % WGN;

  const i32x4 ra = raw_rsrc(p.src, p.src_bytes), rb = raw_rsrc(p.filt, p.filt_bytes);
  const unsigned ldb = (unsigned)(p.CO * ES);

  // A: this wave's instruction PA wave + q covers pixel rows RA (PA wave + q)
  // + lane / CA; the lane fetches global chunk (lane % CA) ^ ((row / SWD) %
  // CA) of the stage's KB bytes, which lands at LDS chunk lane % CA of its row.
  int ih0[PA], iw0[PA];
  unsigned abase[PA];
  // channel of the lane's 16 bytes within a stage (a stage past the last
  // channel reads zeros: channels are padded to whole stages per tap)
  int ach[PA];
  {
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      const int arow_q = RA * (PA * dw + q) + lane / CA;
      const unsigned gc = (unsigned)((lane % CA) ^ ((arow_q / SWD) & (CA - 1)));
      ach[q] = (int)gc * (16 / ES);
      const int pix = m0 + arow_q;
      if (pix < p.M) {
        const int n = (int)p.d_ohw((unsigned)pix);
        const int rem = pix - n * p.OH * p.OW;
        const int oh = (int)p.d_ow((unsigned)rem);
        const int ow = rem - oh * p.OW;
        ih0[q] = oh * p.sh - p.pad_t;
        iw0[q] = ow * p.sw - p.pad_l;
        // the pixel's (possibly out-of-image) origin; valid taps add a
        // non-negative offset that brings the sum inside the image
        abase[q] = (unsigned)(((n * p.H + ih0[q]) * p.W + iw0[q]) * p.C) * (unsigned)ES + gc * 16u;
      } else {
        ih0[q] = -(1 << 30);  // never inside the image
        iw0[q] = 0;
        abase[q] = 0;
      }
    }
  }
  // B: instruction PB wave + q covers filter rows RPI (PB wave + q) + lane /
  // CPR; the lane at LDS chunk lane % CPR of row k fetches global chunk
  // (lane % CPR) ^ ig_bsw(k), and ig_bsw(k) depends on lane / CPR only.
  const unsigned vb = (unsigned)(lane / CPR) * ldb + (unsigned)(n0 * ES) +
                      (unsigned)(((lane % CPR) ^ ig_bsw<ES, BR>(lane / CPR)) << 4);
  // Channel limits: A instruction q's lane reads channels c0 + ach[q] .. of
  // a stage whose first channel is c0, B instruction q's lane filter row c0
  // + RPI (PB wave + q) + lane / CPR; each is in range while c0 is below its
  // limit (a stage past the last channel, or a column past Cout, reads zeros)
  int alim[PA], blim[PB];
#pragma unroll
  for (int q = 0; q < PA; ++q) alim[q] = p.C - ach[q];
  {
    const bool bcol = n0 * ES + (((lane % CPR) ^ ig_bsw<ES, BR>(lane / CPR)) << 4) < p.CO * ES;
#pragma unroll
    for (int q = 0; q < PB; ++q) blim[q] = bcol ? p.C - RPI * (PB * dw + q) - lane / CPR : -(1 << 30);
  }

  // DMA state of the next stage to load: its tap (kh, kw), its channel
  // stage lcc within the tap (first channel c0 = lcc KR), the tap's source
  // offset soff, filter row krow = tap C + c0, and whether each A
  // instruction's pixel is inside the image at this tap (recomputed only
  // when the tap changes; the stages of one tap differ by KB bytes of
  // source and KR filter rows).
  // this workgroup's stages [s_begin, s_begin + ns)
  const int s_begin = (int)((long long)kr * p.stages / p.ksplit);
  // With rot (whole-K tiles only), pixel tile mt starts its walk at stage mt
  // % stages and wraps: the workgroups of one XCD, which run in step, then
  // ask for different filter rows at any one time instead of all sending
  // the same lines' requests to the same L2 channels (c9: 17.5 -> 16.4 us;
  // a start per workgroup rather than per pixel tile 16.6, since the two
  // channel tiles of a pixel tile share its input rows).  The sum over the
  // stages is the same; the order of the f32 additions is not.
  int lst = s_begin + (p.rot ? mt % p.stages : 0);
  int lcc = lst % p.cs, lkw = lst / p.cs, lkh;
  lkh = lkw / p.KW;
  lkw -= lkh * p.KW;
  unsigned soff = 0;
  int krow = 0;
  bool ain[PA];
  auto tap_begin = [&]() {
    const int dih = lkh * p.dh, diw = lkw * p.dw;
    soff = (unsigned)((dih * p.W + diw) * p.C * ES + lcc * KB);
    krow = (lkh * p.KW + lkw) * p.C + lcc * KR;
#pragma unroll
    for (int q = 0; q < PA; ++q)
      ain[q] = ((unsigned)(ih0[q] + dih) < (unsigned)p.H) & ((unsigned)(iw0[q] + diw) < (unsigned)p.W);
  };
  tap_begin();
  const unsigned bstep = (unsigned)RPI * ldb;  // filter bytes between B instructions
  auto dma_stage = [&](unsigned char* S) {
    const int c0 = lcc * KR;  // the stage's first channel
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      const bool in = ain[q] & (c0 < alim[q]);
      dma16(ra, lds_addr(S + (PA * dw + q) * 1024), in ? abase[q] + soff : kIgOutOfRange, 0);
    }
    const unsigned sb = (unsigned)(krow + RPI * PB * dw) * ldb;
#pragma unroll
    for (int q = 0; q < PB; ++q)
      dma16(rb, lds_addr(S + AB + (PB * dw + q) * 1024), c0 < blim[q] ? vb : kIgOutOfRange, sb + q * bstep);
    // the next stage: the next KR channels of this tap, or the next tap
    if (++lst == p.stages) {
      // past the last stage: wrap to the first (only a rotated walk has
      // stages left to load then)
      lst = 0;
      lcc = 0;
      lkw = 0;
      lkh = 0;
      tap_begin();
    } else if (++lcc == p.cs) {
      lcc = 0;
      if (++lkw == p.KW) {
        lkw = 0;
        ++lkh;
      }
      tap_begin();
    } else {
      soff += KB;
      krow += KR;
    }
  };

  // fragment offsets (as in the DMA GEMM): A row r at r * KB, chunk c at
  // c ^ ((r / SWD) % CA); B tile j, read h at boff[j][h] in the stage's first
  // K step, KSR rows further for each later one
  const int lrow = lane & 31, hi = lane >> 5;
  int arow[MI], asw[MI], boff[NI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int r = wm * WTM + i * 32 + lrow;
    arow[i] = r * KB;
    asw[i] = (r / SWD) & (CA - 1);
  }
  {
    const int g = lane >> 4, li = lane & 15;
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int k, cb;
        if constexpr (ES == 2) {
          k = 8 * (g >> 1) + 4 * h + (li >> 2);
          cb = (wn * WTN + j * 32 + 16 * (g & 1) + 4 * (li & 3)) * 2;
        } else {
          k = 16 * (g >> 1) + 8 * h + (li >> 1);
          cb = wn * WTN + j * 32 + 16 * (g & 1) + 8 * (li & 1);
        }
        boff[j][h] = AB + k * BR + (((cb >> 4) ^ ig_bsw<ES, BR>(k)) << 4) + (cb & 15);
      }
  }
  acc_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  auto compute = [&](const unsigned char* S) {
    uint4v af[KSTEPS][MI], bf[KSTEPS][NI];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
        af[ks][i] = *reinterpret_cast<const uint4v*>(S + arow[i] + (((ks * 2 + hi) ^ asw[i]) << 4));
      lds_t* const f = (lds_t*)(S + ks * KSR * BR);
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        uint2v l2, h2;
        if constexpr (ES == 2) {
          l2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                              reinterpret_cast<short4v __attribute__((address_space(3)))*>(f + boff[j][0])));
          h2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                              reinterpret_cast<short4v __attribute__((address_space(3)))*>(f + boff[j][1])));
        } else {
          l2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                                              reinterpret_cast<int2v __attribute__((address_space(3)))*>(f + boff[j][0])));
          h2 = __builtin_bit_cast(uint2v, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                                              reinterpret_cast<int2v __attribute__((address_space(3)))*>(f + boff[j][1])));
        }
        bf[ks][j] = uint4v{l2[0], l2[1], h2[0], h2[1]};
      }
    }
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = ig_mfma<ELEM>(af[ks][i], bf[ks][j], acc[i][j]);
  };

  // NS - 1 stages in flight.  Before the barrier of stage s each wave waits
  // (vmcnt) for its own DMA of stage s only (s + 1 .. s + NS - 2 may stay in
  // flight); after it every wave's DMA of stage s has landed and every wave
  // is done with stage s - 1, whose buffer then receives stage s + NS - 1.
  // The barriers are bare s_barriers: __syncthreads' release fence would wait
  // for every DMA in flight.
  const int ns = (int)((long long)(kr + 1) * p.stages / p.ksplit) - s_begin;
  if (LW && wave >= 4) {
    // loader wave: barrier s follows its own DMA of stage s (stages s + 1
    // .. s + NS - 2 may stay in flight) and frees stage s - 1's buffer for
    // stage s + NS - 1.  As many barriers as the MFMA waves; then, for a
    // whole-K tile, its share of the stores below.
#pragma unroll
    for (int q = 0; q < NS - 1; ++q)
      if (q < ns) dma_stage(buf(q));
    int s = 0;
    for (; s + NS - 2 < ns; ++s) {
      XTK_WAIT_VM((NS - 2) * PER);
      asm volatile("s_barrier" ::: "memory");
      if (s + NS - 1 < ns) dma_stage(buf(s + NS - 1));
    }
    // the last NS - 2 stages: fewer later stages in flight
    for (; s < ns; ++s) {
      if (NS > 3 && s + 2 < ns) XTK_WAIT_VM(2 * PER);
      else if (s + 1 < ns) XTK_WAIT_VM(PER);
      else XTK_WAIT_VM(0);
      asm volatile("s_barrier" ::: "memory");
    }
    if (!STAGED || p.ksplit > 1) return;
  } else if constexpr (LW > 0) {
    // MFMA wave: after barrier s, stage s has landed
    for (int s = 0; s < ns; ++s) {
      asm volatile("s_barrier" ::: "memory");
      compute(buf(s));
    }
  } else {
    static_assert(NS == 4, "the loops below keep two later stages in flight");
#pragma unroll
    for (int q = 0; q < NS - 1; ++q)
      if (q < ns) dma_stage(buf(q));
    int s = 0;
    // steady state: stages s + 1 and s + 2 of this wave stay in flight
    for (; s + 2 < ns; ++s) {
      XTK_WAIT_VM(2 * PER);
      asm volatile("s_barrier" ::: "memory");
      if (s + NS - 1 < ns) dma_stage(buf(s + NS - 1));
      compute(buf(s));
    }
    // the last two stages (no DMA left to issue)
    for (; s < ns; ++s) {
      if (s + 1 < ns) XTK_WAIT_VM(PER);
      else XTK_WAIT_VM(0);
      asm volatile("s_barrier" ::: "memory");
      compute(buf(s));
    }
  }

  // D = A x B per 32 x 32 tile: lane l holds channel l % 32 of tile j and
  // register v pixel row 8 (v / 4) + 4 (l / 32) + v % 4 of tile i
  if constexpr (STAGED) {
    if (p.ksplit == 1) {
      // A whole-K tile's results go through LDS ([BM rows][BN f32], rows OP
      // bytes apart: the two half-waves' rows r and r + 4 fall 32 banks
      // apart) and leave as 16-byte non-temporal lanes from all 4 + LW
      // waves: a quarter of the store instructions of 4-byte lanes from
      // the four MFMA waves (c9: 1.8 us of stores after the K loop).
      constexpr int OP = BN * 4 + 32;
      static_assert(BM * OP <= NS * STAGE && (4 * (OP / 4)) % 64 == 32, "staging rows");
      float* const st = reinterpret_cast<float*>(smem);
      __syncthreads();  // every wave is done with the stage buffers
      if (wave < 4) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int row = wm * WTM + i * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
              const float x = static_cast<float>(acc[i][j][v]);
              st[row * (OP / 4) + wn * WTN + j * 32 + lrow] = x;
            }
      }
      __syncthreads();
      constexpr int PR = BN / 4;  // 16-byte pieces a row
      for (int k = tid; k < BM * PR; k += 64 * (4 + LW)) {
        const int row = k / PR, c4 = k - row * PR;
        // Cout is a multiple of 8 (16-byte filter rows), so a piece that
        // starts below Cout ends below it
        if (m0 + row < p.M && n0 + 4 * c4 < p.CO)
          __builtin_nontemporal_store(*reinterpret_cast<const float4v*>(st + row * (OP / 4) + 4 * c4),
                                      reinterpret_cast<float4v*>(p.out + (long long)(m0 + row) * p.CO + n0 + 4 * c4));
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int col = n0 + wn * WTN + j * 32 + lrow;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
        // through a scalar (a bit-cast of an ext_vector element lvalue reads
        // element 0); an i8 sum is an exact i32, rounded to f32 once
        const float x = static_cast<float>(acc[i][j][v]);
        if (row >= p.M || col >= p.CO) continue;
        float* const o = p.out + (long long)row * p.CO + col;
        // K split: the ranges' partial sums meet in the zero-filled output
        // (f16 / bf16 only; the order of the additions varies)
        if (p.ksplit > 1) __hip_atomic_fetch_add(o, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else __builtin_nontemporal_store(x, o);
      }
    }
}

// Zero-fills n floats (a kernel, not hipMemsetAsync, so that a captured graph
// replays it correctly).
__global__ __launch_bounds__(256) void ig_zero_kernel(float4v* __restrict__ o, long long n4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) __builtin_nontemporal_store(float4v{0.f, 0.f, 0.f, 0.f}, o + i);
}

}  // namespace

bool conv_blocks_cover_output(const xt::Plan& p, long long es) {
  const xt::ConvPlan& c = p.conv;
  if (c.cb.axis < 0 || c.ch.axis < 0 || c.cw.axis < 0 || c.cb.axis == c.ch.axis || c.cb.axis == c.cw.axis ||
      c.ch.axis == c.cw.axis)
    return false;
  // the Blocks tile images [0, gB) x every output row and column once, in the
  // output's natural NHWC addressing, with one filter
  const long long gB = p.grid[c.cb.axis], gH = p.grid[c.ch.axis], gW = p.grid[c.cw.axis];
  if (gH * c.TH != c.out_H || gW * c.TW != c.out_W || c.out_C != c.CO) return false;
  auto step = [&](const xt::TileAddr& t, int axis) { return axis == 0 ? t.sx : axis == 1 ? t.sy : t.sz; };
  // a Block holds TB images: the Blocks cover images [0, gB TB)
  const long long plane = c.out_H * c.out_W * c.out_C;
  if (c.out_addr.c0 != 0 || (gB > 1 && step(c.out_addr, c.cb.axis) != c.TB * plane) ||
      (gH > 1 && step(c.out_addr, c.ch.axis) != c.TH * c.out_W * c.out_C) ||
      (gW > 1 && step(c.out_addr, c.cw.axis) != c.TW * c.out_C))
    return false;
  return !(c.filt_addr.sx || c.filt_addr.sy || c.filt_addr.sz || (c.filt_addr.c0 * es) % 16);
}

bool launch_conv2d_igemm(const xt::Plan& p, void* const* bufs, hipStream_t s, hipError_t& e) {
  const xt::ConvPlan& c = p.conv;
  const bool i8 = c.elem == xt::Elem::I8;
  if (c.elem != xt::Elem::F16 && c.elem != xt::Elem::BF16 && !i8) return false;
  const long long es = i8 ? 1 : 2;
  // a K stage is 64 bytes of one tap's channels (the last stage of a tap
  // padded with zeros), read in 16-byte pieces: Cin * esize and Cout * esize
  // multiples of 16
  if (c.out_elem != xt::Elem::F32 || c.TC != c.CO || (c.C * es) % 16 || (c.CO * es) % 16) return false;
  if (!conv_blocks_cover_output(p, es)) return false;
  const long long gB = p.grid[c.cb.axis];
  // the source batch entries the Blocks read: images [0, gB) of an NHWC tensor
  const long long src_bytes = gB * c.TB * c.H * c.W * c.C * es;
  const long long K = c.KH * c.KW * c.C;
  const long long filt_bytes = K * c.CO * es;
  const long long M = gB * c.TB * c.out_H * c.out_W;
  if (src_bytes >= (1LL << 31) || filt_bytes >= (1LL << 31) || M >= (1LL << 31) || c.out_H * c.out_W >= (1LL << 31))
    return false;
  const unsigned char* src = static_cast<const unsigned char*>(bufs[c.src_arg]);
  const unsigned char* filt = static_cast<const unsigned char*>(bufs[c.filt_arg]) + c.filt_addr.c0 * es;
  float* out = static_cast<float*>(bufs[c.out_arg]);
  for (const void* ptr : {(const void*)src, (const void*)filt, (const void*)out})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) return false;
  IgArgs a;
  a.src = src;
  a.filt = filt;
  a.out = out;
  a.src_bytes = static_cast<unsigned>(src_bytes);
  a.filt_bytes = static_cast<unsigned>(filt_bytes);
  a.H = (int)c.H;
  a.W = (int)c.W;
  a.C = (int)c.C;
  a.KW = (int)c.KW;
  a.CO = (int)c.CO;
  a.OH = (int)c.out_H;
  a.OW = (int)c.out_W;
  a.pad_t = (int)c.pad_top;
  a.pad_l = (int)c.pad_left;
  a.sh = (int)c.stride_h;
  a.sw = (int)c.stride_w;
  a.dh = (int)c.dil_h;
  a.dw = (int)c.dil_w;
  a.M = (int)M;
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  // 128 x 128 tiles when Cout allows, else 256 x 64.  When the 128 x 128
  // tiles would fill at most half the CUs (deep layers) and a tap's channels
  // are whole 128-byte stages: 64 x 128 tiles with 128-byte stages (twice
  // the tiles, half the stages and barriers).  Measured on 32 x 14^2 x 256
  // -> 256, 3 x 3 (one call, 500 launches each): 98 tiles of 128 x 128 split
  // in two 29.7-31.2 us, 196 of 64 x 128 with 64-byte stages 27.9, with
  // 128-byte stages 22.9-24.7 (six stages in LDS 25.2, two 23.2, 256-byte
  // stages 23.0; 392 tiles of 64 x 64 23.7).
  const bool wide = c.CO % 128 == 0;
  const long long tiles128 = (M + 127) / 128 * ((c.CO + 127) / 128);
  const bool deep = wide && tiles128 * 2 <= cus && (c.C * es) % 128 == 0;
  const int bm = deep ? 64 : wide ? 128 : 256, bn = wide ? 128 : 64, kb = deep ? 128 : 64;
  a.cs = (int)((c.C * es + kb - 1) / kb);
  a.stages = (int)(c.KH * c.KW) * a.cs;
  a.ntiles = (int)((c.CO + bn - 1) / bn);
  const long long tiles = (M + bm - 1) / bm * a.ntiles;
  // K split when the tiles fill at most half the CUs (f16 / bf16: i8 sums stay
  // exact and whole): up to one workgroup a CU, at least 16 stages each.
  // Measured (batch 32, 3 x 3, 128 x 128 tiles): 7 x 7 x 512 -> 512 (52
  // tiles) 56.9 us whole, 27.7 split in 4; 14 x 14 x 256 -> 256 (98 tiles)
  // 31.3 / 27.9 in 2; 28 x 28 x 128 -> 128 (196 tiles) 19.8 whole, 33.0 in 2
  // (the zero fill and the atomic adds of the output cost more than the idle
  // CUs)
  // (XTILE_AMD_KSPLIT=0 keeps every tile whole.)  Ranges are spread evenly:
  // their lengths differ by at most one stage.
  long long ksplit = 1;
  const bool split_ok = !i8 && ksplit_allowed();
  if (split_ok && tiles * 2 <= cus) ksplit = std::max(1LL, std::min<long long>(cus / tiles, a.stages / 16));
  // up to one round of tiles with a long K: two halves of >= 64 stages
  // (14 x 14 x 512 -> 512, 196 tiles, 144 stages: 63.7 us whole, 56.9 split)
  else if (split_ok && tiles <= cus && a.stages >= 128) ksplit = 2;
  a.kstages = (int)(a.stages / ksplit);
  const long long nwg = tiles * ksplit;
  if (!grid_fits(nwg, 256) || M * c.CO % 4) return false;
  a.tiles = (int)tiles;
  a.ksplit = (int)ksplit;
  // the rotated walk keeps a whole filter and the XCD's input rows in its
  // 4 MB L2 at once (the walk in step reads one stage of them at a time):
  // deep whole-K tiles with a filter up to 2 MB
  a.rot = deep && ksplit == 1 && filt_bytes <= (2LL << 20) ? 1 : 0;
  a.nwg = (int)nwg;
  if (ksplit > 1) {
    const long long n4 = M * c.CO / 4;
    hipLaunchKernelGGL(ig_zero_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<float4v*>(out), n4);
  }
  a.d_ohw = div31((unsigned)(c.out_H * c.out_W));
  a.d_ow = div31((unsigned)c.out_W);
  const int el = i8 ? kIgI8 : c.elem == xt::Elem::BF16 ? kIgBF16 : kIgF16;
#define XT_IG(E)                                                                                       \
  do {                                                                                                 \
    if (deep) hipLaunchKernelGGL((conv_igemm_kernel<E, 64, 128, 32, 64, 128, 8>), dim3(a.nwg), dim3(768), 0, s, a); \
    else if (wide) hipLaunchKernelGGL((conv_igemm_kernel<E, 128, 128>), dim3(a.nwg), dim3(256), 0, s, a);      \
    else hipLaunchKernelGGL((conv_igemm_kernel<E, 256, 64>), dim3(a.nwg), dim3(256), 0, s, a);                 \
  } while (0)
  if (el == kIgI8) XT_IG(kIgI8);
  else if (el == kIgBF16) XT_IG(kIgBF16);
  else XT_IG(kIgF16);
#undef XT_IG
  e = hipGetLastError();
  return true;
}

}  // namespace xtk
