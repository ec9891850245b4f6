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
//     are contiguous) lives in LDS, zero-filled outside the image.  The next
//     unit's halo is loaded into registers while the current unit computes and
//     written to LDS between two barriers.
//   * v_mfma_f32_32x32x16_{f16,bf16}: waves take the unit's 32-pixel M tiles
//     in pairs (w, w+4) against every 32-channel N tile, so each fragment read
//     from LDS feeds two MFMAs.  The filter fragment is the A operand, so each
//     lane ends up holding runs of consecutive channels of one pixel.  Fragments of step s+1 are read while the
//     MFMAs of step s run.  LDS rows are padded by 16 bytes: the pitch is an
//     odd number of 16-byte chunks, so 16 consecutive pixels (or filter rows)
//     hit 16 distinct 4-bank groups.
//   * Outputs are written once and never re-read: non-temporal 16-byte buffer
//     stores; halo loads and output stores go through buffer descriptors whose
//     range check supplies the zero padding and drops the ragged edge.
//   * Waves 0-3 compute; waves 4-7 only fetch halos (see conv2d_kernel).
//
// Kernel choice (launch_conv2d): the band kernel below when the Blocks tile
// the whole output and filter + halo fit in LDS; else, for the same tiling
// with Cin * esize and Cout * esize multiples of 16, the implicit GEMM with
// DMA operands (conv_igemm.hip); for that tiling with Cin * esize not a
// multiple of 16 (the RGB stem), Cout * esize a multiple of 16 and column dilation 1, the
// LDS-patch kernel (conv_small.hip); else the persistent kernel above for f16 / bf16
// with Cin % 32 == 0, Cout % 16 == 0 (<= 128), one image per Block, every
// output channel and an f32 result; else the generic kernel
// (conv_general.hip), which takes every tile shape the planner accepts.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr int HV = 12;  // halo 16-byte vectors per thread per unit (at most)
constexpr int FB = 6;   // filter sub-blocks per thread per batch
constexpr int CT = 256; // compute threads (waves 0-3); they also stage the filter
constexpr int WG = 512; // threads: waves 0-3 compute, waves 4-7 load halos
constexpr int HT = 256; // halo loader threads
constexpr int kOutPitch = 144;  // LDS bytes per staged output pixel (32 floats + 16-byte pad)

typedef float float16v __attribute__((ext_vector_type(16)));



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
  int pitch;            // LDS bytes per halo pixel (2*Cin + 16)
  int kpitch;           // LDS bytes per filter row (2*K + 16)
  int halo_vecs;        // rf_h * rf_w * Cin / 8
  int halo_bytes;       // rf_h * rf_w * pitch
  int nmt;              // 32-pixel M tiles per unit
  int steps;            // K / 16 (even: Cin % 32 == 0)
  // Multiply-high reciprocals of the divisors used per thread (see udiv).
  Magic m_cv, m_rfw, m_tw, m_cg;  // Cin/8, rf_w, TW, Cout/8
  unsigned image_bytes;              // H*W*Cin*2: one batch entry of the source
  unsigned unit_out_bytes;           // UR*out_W*out_C*4: the output rows of one unit
};


template <bool BF16>
__device__ __forceinline__ float16v mfma32(short8 a, short8 b, float16v c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
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

// Loader thread `tid` owns the halo's 16-byte vectors tid + i*HT.  Their
// coordinates are recomputed per unit (a few multiply-highs) rather than kept
// in registers: every wave of the workgroup holds the same register budget.
struct HaloSlot {
  int r, c, src, dst;  // halo row / column, element offset from the halo origin, LDS byte offset
};

__device__ __forceinline__ HaloSlot halo_slot(const ConvArgs& p, int v) {
  const int cv = p.C / 8;
  const int pix = udiv(v, p.m_cv);
  const int c8 = v - pix * cv;
  HaloSlot h;
  h.r = udiv(pix, p.m_rfw);
  h.c = pix - h.r * p.rf_w;
  h.src = (h.r * p.W + h.c) * p.C + c8 * 8;
  h.dst = pix * p.pitch + c8 * 16;
  return h;
}

// Buffer descriptors (gfx9 raw buffers: stride 0, word3 0x00020000).  A
// buffer load whose offset lies past num_records returns zero and such a store
// is dropped, so halo padding and the unit's ragged edge need no branches.
constexpr unsigned kOutOfRange = 0x80000000u;  // every buffer here is < 2 GiB

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Halo of unit `t` -> registers, every load issued back to back (one round
// trip).  Vectors outside the image read as zero through the descriptor.
// dst[i] receives vector i's LDS offset (or -1 past the halo) for store_halo.
__device__ __forceinline__ void load_halo(const ConvArgs& p, const Unit& t, int tid, uint4v (&hv)[HV],
                                          int (&dst)[HV]) {
  const __amdgpu_buffer_rsrc_t img = buffer_of(t.S, p.image_bytes);
  const int org = (t.ih0 * p.W + t.iw0) * p.C;  // may be negative; only in-image sums are used
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int v = tid + i * HT;
    const HaloSlot h = halo_slot(p, v < p.halo_vecs ? v : 0);
    const int ih = t.ih0 + h.r, iw = t.iw0 + h.c;
    const bool inside = v < p.halo_vecs && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
    const unsigned off = inside ? unsigned(org + h.src) * 2u : kOutOfRange;
    hv[i] = __builtin_amdgcn_raw_buffer_load_b128(img, off, 0, 0);
    dst[i] = v < p.halo_vecs ? h.dst : -1;
  }
}

__device__ __forceinline__ void store_halo(unsigned char* Is, const uint4v (&hv)[HV], const int (&dst)[HV]) {
#pragma unroll
  for (int i = 0; i < HV; ++i)
    if (dst[i] >= 0) *reinterpret_cast<uint4v*>(Is + dst[i]) = hv[i];
}

// Filter -> LDS, transposed by 4(k) x 8(cout) register blocks; FB blocks per
// thread per batch, all of a batch's loads issued before the first use.
// Consecutive threads take consecutive 8-channel groups of the same K rows, so
// a wave's load covers whole 128-byte lines (every workgroup reads the same
// filter at the same moment; scattered 16-byte reads would multiply the L2
// requests by 8).  Rows Cout..rows-1 (the tail of the last 32-wide N tile)
// are zeroed.
__device__ __forceinline__ void stage_filter(const ConvArgs& p, const unsigned short* F,
                                             unsigned char* Fs, int rows, int tid) {
  const int K = p.KH * p.KW * p.C;
  const int kgroups = K / 4;
  const int cgroups = p.CO / 8;
  const int nsub = kgroups * cgroups;
  for (int base = tid; base < nsub; base += CT * FB) {
    uint4v r[FB][4];
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const int sb = base + b * CT;
      const int sbc = sb < nsub ? sb : 0;
      const int kg = udiv(sbc, p.m_cg), cg = sbc - kg * cgroups;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[b][i] = *reinterpret_cast<const uint4v*>(F + (long long)(kg * 4 + i) * p.CO + cg * 8);
    }
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const int sb = base + b * CT;
      if (sb >= nsub) continue;
      const int kg = udiv(sb, p.m_cg), cg = sb - kg * cgroups;
      const int k0 = kg * 4, c0 = cg * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint2v even, odd;
        even.x = (r[b][0][j] & 0xFFFFu) | (r[b][1][j] << 16);
        even.y = (r[b][2][j] & 0xFFFFu) | (r[b][3][j] << 16);
        odd.x = (r[b][0][j] >> 16) | (r[b][1][j] & 0xFFFF0000u);
        odd.y = (r[b][2][j] >> 16) | (r[b][3][j] & 0xFFFF0000u);
        *reinterpret_cast<uint2v*>(Fs + (c0 + 2 * j) * p.kpitch + k0 * 2) = even;
        *reinterpret_cast<uint2v*>(Fs + (c0 + 2 * j + 1) * p.kpitch + k0 * 2) = odd;
      }
    }
  }
  const int tail = (rows - p.CO) * (K / 8);  // 16-byte vectors of zero rows
  for (int v = tid; v < tail; v += CT) {
    const int row = p.CO + v / (K / 8), ch = v % (K / 8);
    *reinterpret_cast<uint4v*>(Fs + row * p.kpitch + ch * 16) = uint4v{0u, 0u, 0u, 0u};
  }
}

// M tiles mt0 and mt0+4 (MT == 2) or mt0 alone (MT == 1) of the unit against
// all NT N tiles.  Step s covers K [16s, 16s+16): tap (kh, kw) = s / (Cin/16),
// channels 16 * (s % (Cin/16)) ... + 16; lane l reads 8 of them (l/32 picks the
// half) for pixel / filter row l%32.
template <int MT, int NT, bool BF16>
__device__ __forceinline__ void conv_tiles(const ConvArgs& p, const Unit& t, const unsigned char* Fs,
                                           const unsigned char* Is, unsigned char* Os, int mt0, int lane) {
  const int lr = lane & 31, hi = lane >> 5;
  const int M = p.UR * p.TW;
  int abase[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int pix = min((mt0 + 4 * i) * 32 + lr, M - 1);
    const int ph = udiv(pix, p.m_tw), pw = pix - ph * p.TW;
    abase[i] = (ph * p.sh * p.rf_w + pw * p.sw) * p.pitch + hi * 16;
  }
  int bbase[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) bbase[j] = (j * 32 + lr) * p.kpitch + hi * 16;

  float16v acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Steps run tap by tap, two channel steps per inner iteration (Cin/16 is
  // even).  Per-lane LDS pointers advance by one uniform delta per iteration:
  // +64 bytes inside a tap, the tap-to-tap distance at its end, so the loop
  // carries a handful of scalar ops for its eight reads and MFMAs.
  //   A: pa = abase + kh*dh*rf_w*pitch + kw*dw*pitch + 32*c
  //   B: pb = bbase + 32*s (K is contiguous across taps)
  const int cs = p.C / 16;
  const int taps = p.KH * p.KW;
  const int acol = p.dw * p.pitch;
  const int arow = p.dh * p.rf_w * p.pitch - (p.KW - 1) * acol;  // last tap of a row -> next row
  int pa[MT], pb[NT];
#pragma unroll
  for (int i = 0; i < MT; ++i) pa[i] = abase[i];
#pragma unroll
  for (int j = 0; j < NT; ++j) pb[j] = bbase[j];
  short8 af[2][MT], bf[2][NT];
  auto rd = [&](int set, int imm) {
#pragma unroll
    for (int i = 0; i < MT; ++i) af[set][i] = *reinterpret_cast<const short8*>(Is + pa[i] + imm);
#pragma unroll
    for (int j = 0; j < NT; ++j) bf[set][j] = *reinterpret_cast<const short8*>(Fs + pb[j] + imm);
  };
  auto mma = [&](int set) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = mfma32<BF16>(bf[set][j], af[set][i], acc[i][j]);
  };
  rd(0, 0);
  int kw = 0;
  for (int tap = 0; tap < taps; ++tap) {
    const bool last = tap + 1 == taps;
    const bool row_end = ++kw == p.KW;
    kw = row_end ? 0 : kw;
    // bytes from this tap's first step to the next tap's; the last tap stays
    // on its final pair so the trailing reads are in bounds (and unused)
    const int to_next = last ? (cs - 2) * 32 : row_end ? arow : acol;
    for (int c = 0; c < cs; c += 2) {
      rd(1, 32);  // step c+1 of this tap
      mma(0);
      const bool in_tap = c + 2 < cs;
      const int da = in_tap ? 64 : to_next - c * 32;
      const int db = in_tap || !last ? 64 : 0;
#pragma unroll
      for (int i = 0; i < MT; ++i) pa[i] += da;
#pragma unroll
      for (int j = 0; j < NT; ++j) pb[j] += db;
      rd(0, 0);  // step c+2, or the next tap's first
      mma(1);
      // Issue order per half (one step of MFMAs): the other set's reads go in
      // front and between the first MFMAs, the last two MFMAs carry none, so
      // the reads have two MFMAs of time to land before the next half.
      constexpr int F = MT * NT, R = MT + NT;
      constexpr int lead = R - (F - 2) > 1 ? R - (F - 2) : 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        __builtin_amdgcn_sched_group_barrier(0x100, lead < R ? lead : R, 0);
#pragma unroll
        for (int g = 0; g < F; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (lead + g < R) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
    }
  }

  // The MFMAs compute D = F x P (A = filter fragment, B = pixel fragment), so
  // lane l holds pixel l%32 of the tile and register v holds output channel
  // 8*(v/4) + 4*(l/32) + v%4: four runs of four consecutive channels.  Each
  // 32x32 tile goes through the wave's own LDS staging rows (pixel-major,
  // 144-byte pitch) and leaves as four 16-byte stores per lane where eight
  // consecutive lanes cover one pixel's 128 channel bytes, so every store
  // instruction writes whole 128-byte lines.  Pixel q of the unit (row q / TW,
  // column q % TW) starts at q*out_C + (q / TW)*(out_W - TW)*out_C floats from
  // the unit origin; pixels past the unit and channels past Cout get an
  // out-of-range offset.
  const __amdgpu_buffer_rsrc_t ob = buffer_of(t.O, p.unit_out_bytes);
  const int rowgap = (p.out_W - p.TW) * p.out_C;
  const int sr = lane >> 3, sc = lane & 7;  // staging read: pixel 8k + sr, 16-byte chunk sc
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    unsigned pix[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = (mt0 + 4 * i) * 32 + 8 * k + sr;
      pix[k] = q < M ? unsigned(q * p.out_C + (int)udiv(q, p.m_tw) * rowgap) * 4u : kOutOfRange;
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4v val = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        *reinterpret_cast<float4v*>(Os + lr * kOutPitch + (8 * g + 4 * hi) * 4) = val;
      }
      const int co = j * 32 + 4 * sc;
      const bool cok = co < p.CO;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint4v val = *reinterpret_cast<const uint4v*>(Os + (8 * k + sr) * kOutPitch + sc * 16);
        __builtin_amdgcn_raw_buffer_store_b128(val, ob, cok && pix[k] != kOutOfRange ? pix[k] + co * 4u : kOutOfRange,
                                               0, 2);
      }
    }
  }
}

template <int NT, bool BF16>
__device__ __forceinline__ void compute_unit(const ConvArgs& p, const Unit& t, const unsigned char* Fs,
                                             const unsigned char* Is, unsigned char* Os, int tid) {
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Wave w owns M tiles w, w+4, w+8, ...  Up to CAP of them go through one
  // call, so the epilogue stores sit in no loop: a loop holding stores makes
  // the compiler wait for every outstanding load (the next unit's halo) before
  // entering it.  Larger units loop CAP tiles at a time (tiles past the end
  // are computed on clamped pixels and not stored).
  constexpr int CAP = NT >= 4 ? 1 : 2;  // accumulators: CAP * NT * 16 per lane
  const int cnt = (p.nmt - wave + 3) >> 2;
  if (cnt == 1) {
    conv_tiles<1, NT, BF16>(p, t, Fs, Is, Os + wave * 32 * kOutPitch, wave, lane);
  } else if (CAP >= 2 && cnt == 2) {
    conv_tiles<CAP, NT, BF16>(p, t, Fs, Is, Os + wave * 32 * kOutPitch, wave, lane);
  } else if (cnt > CAP) {
    for (int mt0 = wave; mt0 < p.nmt; mt0 += 4 * CAP) conv_tiles<CAP, NT, BF16>(p, t, Fs, Is, Os + wave * 32 * kOutPitch, mt0, lane);
  }
}

// Waves 0-3 compute (MFMAs and output stores only); waves 4-7 fetch the next
// unit's halo into registers and write it to LDS between the unit's two
// barriers.  Keeping the global loads out of the compute waves keeps their
// instruction stream free of waits on memory: each wave waits only on its own
// counters, and a compute wave has no load outstanding while it runs MFMAs.
template <int NT, bool BF16>
__global__ __launch_bounds__(WG, 1) void conv2d_kernel(ConvArgs p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  unsigned char* Fs = lds;
  unsigned char* Is = lds + NT * 32 * p.kpitch;
  unsigned char* Os = Is + p.halo_bytes;  // 4 compute waves x 32 pixel rows of output staging
  const int tid = threadIdx.x;
  const bool loader = __builtin_amdgcn_readfirstlane(tid >> 6) >= 4;
  const int ltid = tid - (WG - HT);

  uint4v hv[HV];
  int dst[HV];
  int u = blockIdx.x;  // the host launches at most total_units workgroups
  Unit cur = unit_of(p, u);
  if (loader) {
    load_halo(p, cur, ltid, hv, dst);
    store_halo(Is, hv, dst);
  } else {
    // Every Block uses the same filter (the launcher sends filters that move
    // with the Block to the generic kernel), so every unit of this
    // workgroup uses the first one's origin.
    // The compute waves stage it while the loaders fetch the first halo.
    int x, y, z;
    decode_block(u / p.units_per_block, p.gx, p.gy, x, y, z);
    stage_filter(p, p.filt + p.tf.at(x, y, z), Fs, NT * 32, tid);
  }
  __syncthreads();
  for (; u < p.total_units; u += gridDim.x) {
    const int un = u + gridDim.x;
    const bool more = un < p.total_units;  // uniform across the workgroup
    if (loader) {
      if (more) load_halo(p, unit_of(p, un), ltid, hv, dst);
    } else {
      compute_unit<NT, BF16>(p, cur, Fs, Is, Os, tid);
    }
    if (more) {
      __syncthreads();  // every compute wave is done with this halo
      if (loader) store_halo(Is, hv, dst);
      __syncthreads();
      cur = unit_of(p, un);
    }
  }
}

// ---------------------------------------------------------------------------
// Band kernel: one workgroup per band of R consecutive output rows of one
// image, used when the Blocks tile the whole output (TW = output width) and
// the band's receptive field fits in LDS beside the whole filter.  Blocks are
// independent (README.md:85-89) and every output pixel is computed with the
// same K order as in the per-Block kernel, so regrouping pixels into bands is
// a scheduling choice; R is picked so that the bands spread evenly over the
// CUs (C4: 32 images x 56 rows = 256 bands of 7 rows).  Workgroups reach
// the 8 XCDs round-robin; band ids are remapped so that each XCD takes a
// contiguous run of bands, whose shared halo rows then come from HBM into
// one L2 once (C4: 12.8-13.3 -> 12.2 us).
//   * The filter [KH*KW*Cin][Cout] (HWIO, Cout contiguous) and the band's halo
//     [rows][cols][Cin] go global -> LDS by buffer DMA (16 bytes per lane, one
//     1 KB run per wave instruction); halo pixels outside the image come from
//     out-of-range buffer offsets, which the DMA writes as zeros.
//   * MFMA view: D[pixel][cout] += P[pixel][k] F[k][cout] with
//     v_mfma_f32_32x32x16_{f16,bf16}.  Pixel fragments are ds_read_b128 of the
//     halo (channels contiguous); filter fragments come from ds_read_b64_tr_b16,
//     which returns K-contiguous lanes from the Cout-contiguous rows.
//   * Both LDS tiles are XOR-swizzled in 16-byte chunks (applied on the global
//     side of the DMA), so 16 consecutive pixels or the transposed 4x16 blocks
//     of four filter rows hit 16 distinct bank groups.
//   * Work: the band's 32-pixel M tiles x 32-channel N tiles, dealt
//     round-robin over the 8 waves (two waves per SIMD); a wave runs two of its
//     M tiles at a time against one N tile and stores them straight from the
//     accumulators (each store instruction writes two 128-byte pixel runs).
constexpr int BWG = 512;
#ifndef XT_BAND_MAX_MI
#define XT_BAND_MAX_MI 4  // M tiles per pass of a wave (1-4)
#endif

struct BandArgs {
  const unsigned char* src;
  const unsigned char* filt;
  float* out;
  int H, W, C;           // source image
  int KH, KW, CO;
  int OH, OW;            // output rows / columns per image
  int pad_t, pad_l, sh, sw, dh, dw;
  int R;                 // output rows per band
  int bands_per_image;
  int rf_w;              // halo columns
  int K, steps;          // K = KH*KW*C, steps = K / 16
  int rb_shift;          // log2(bytes per filter row)
  int fsw_unit, fsw_shift, fsw_mask;  // filter chunk swizzle: unit * ((k >> shift) & mask)
  int pitch;             // LDS bytes per halo pixel: 2*Cin (+16 to make the chunk count odd)
  int rpitch;            // LDS bytes per halo row: rf_w * pitch + a pad of whole chunks (see try_band)
  int nch;               // 16-byte data chunks per halo pixel: Cin * esize / 16
  int nchp;              // pitch / 16
  int ppi;               // halo pixels per DMA instruction: 64 / nchp
  int ipr;               // DMA instructions per halo row: ceil(rf_w / ppi)
  Magic m_nchp, m_ipr, m_ow;
  int filt_instr;        // 1 KB DMA runs of the filter
  unsigned filt_bytes;   // K*CO*esize (LDS offset of the halo)
  unsigned image_bytes;  // H*W*C*esize
};

enum { kBandF16 = 0, kBandBF16 = 1, kBandI8 = 2 };
typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int16v __attribute__((ext_vector_type(16)));

// f16 / bf16 accumulate in f32; i8 in i32 (exact), converted to f32 when stored.
template <int ELEM>
struct BandAcc {
  typedef float16v type;
};
template <>
struct BandAcc<kBandI8> {
  typedef int16v type;
};

// One K step of 32 bytes per pixel: 16 f16 / bf16 values or 32 i8 values.
template <int ELEM>
__device__ __forceinline__ typename BandAcc<ELEM>::type band_mfma(short8 a, short8 b,
                                                                 typename BandAcc<ELEM>::type c) {
  if constexpr (ELEM == kBandI8)
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(int4v, a), __builtin_bit_cast(int4v, b), c, 0,
                                                 0, 0);
  else
    return mfma32<ELEM == kBandBF16>(a, b, c);
}

typedef __attribute__((address_space(3))) unsigned char band_lds_t;

// MI M tiles of the band (first pixel q0, then every tstride pixels) against
// N tile j, all in one pass so that each filter fragment feeds MI MFMAs.  K
// runs tap by tap; a tap is CS steps of 32 bytes per pixel (16 f16 / bf16 or
// 32 i8 channels), CS = Cin * esize / 32.  Within a tap every fragment address
// is the tap's base plus a compile-time offset, so the per-step work is the
// reads and the MFMAs alone; the tap bookkeeping (a few scalar selects and
// MI + 2 vector adds) runs once per tap.  Fragments are read one step pair
// ahead of their MFMAs.  Pixels at or past qend are computed on clamped
// addresses and not stored.
template <int MI, int NT, int CS, int ELEM>
__device__ __forceinline__ void band_tiles(const BandArgs& p, const band_lds_t* Fs, const band_lds_t* Hs,
                                           __amdgpu_buffer_rsrc_t orc, int q0, int tstride, int qend, int j,
                                           int lane) {
  const int lr = lane & 31, hi = lane >> 5;
  const int g = lane >> 4, li = lane & 15;
  constexpr int ES = ELEM == kBandI8 ? 1 : 2;  // bytes per element
  constexpr int RS = 32 / ES;                  // K rows per step
  constexpr int RB = NT * 32 * ES;             // bytes per filter row (Cout = 32 NT)
  constexpr int BSTEP = RS * RB;               // filter bytes per K step
  // Filter fragment: two transposed reads per step.  16-bit: each 16-lane
  // group reads a 4 (K) x 16 (Cout) block, lane i at K row i/4 and columns
  // 4*(i%4)..+3 (ds_read_b64_tr_b16).  8-bit: an 8 x 16 block, lane i at K row
  // i/2 and columns 8*(i%2)..+7 (ds_read_b64_tr_b8).  A step moves RS rows,
  // which leaves the row swizzle unchanged, so each read is a per-lane
  // constant plus BSTEP * s.
  int pb[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int k, ncol;
    if constexpr (ELEM == kBandI8) {
      k = 16 * (g >> 1) + 8 * h + (li >> 1);
      ncol = 32 * j + 16 * (g & 1) + 8 * (li & 1);
    } else {
      k = 8 * (g >> 1) + 4 * h + (li >> 2);
      ncol = 32 * j + 16 * (g & 1) + 4 * (li & 3);
    }
    const int cb = ncol * ES;  // byte column
    pb[h] = k * RB + (((cb >> 4) ^ (p.fsw_unit * ((k >> p.fsw_shift) & p.fsw_mask))) << 4) + (cb & 15);
  }
  // Pixel fragment of tile t in the current tap, channel step c:
  // Hs + pa[t] + 32 c, pa[t] = (halo pixel of the tap) * pitch + 16 (l/32).
  int pa[MI];
#pragma unroll
  for (int t = 0; t < MI; ++t) {
    const int q = min(q0 + t * tstride + lr, qend - 1);
    const int r = (int)udiv((unsigned)q, p.m_ow), c = q - r * p.OW;
    pa[t] = r * p.sh * p.rpitch + c * p.sw * p.pitch + hi * 16;
  }
  typedef short8 __attribute__((address_space(3))) lds_s8;
  auto read = [&](const int (&ra)[MI], const int (&rb)[2], int c, short8 (&a)[MI], short8& b) {
#pragma unroll
    for (int t = 0; t < MI; ++t) a[t] = *reinterpret_cast<const lds_s8*>(Hs + ra[t] + c * 32);
    band_lds_t* f = const_cast<band_lds_t*>(Fs) + c * BSTEP;
    if constexpr (ELEM == kBandI8) {
      const int2v lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<int2v __attribute__((address_space(3)))*>(f + rb[0]));
      const int2v h4 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<int2v __attribute__((address_space(3)))*>(f + rb[1]));
      b = __builtin_bit_cast(short8, int4v{lo[0], lo[1], h4[0], h4[1]});
    } else {
      const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          reinterpret_cast<short4v __attribute__((address_space(3)))*>(f + rb[0]));
      const short4v h4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          reinterpret_cast<short4v __attribute__((address_space(3)))*>(f + rb[1]));
      b = short8{lo[0], lo[1], lo[2], lo[3], h4[0], h4[1], h4[2], h4[3]};
    }
  };
  typename BandAcc<ELEM>::type acc[MI];
#pragma unroll
  for (int t = 0; t < MI; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[t][v] = 0;
  auto mfmas = [&](const short8 (&a)[MI], const short8& b) {
#pragma unroll
    for (int t = 0; t < MI; ++t) acc[t] = band_mfma<ELEM>(a[t], b, acc[t]);
  };

  // Two register sets of one step pair each; the set in use alternates with
  // the pair index, so a tap of CS / 2 pairs starts on set PAR.
  short8 a00[MI], a01[MI], a10[MI], a11[MI], b00, b01, b10, b11;
  const int dcol = p.dw * p.pitch;                                // next tap in the filter row
  const int drow = p.dh * p.rpitch - (p.KW - 1) * p.dw * p.pitch;  // first tap of the next row
  const int taps = p.KH * p.KW;
  int tap = 0, kw = 0;
  read(pa, pb, 0, a00, b00);
  read(pa, pb, 1, a01, b01);
  auto tap_body = [&](auto par_c) {
    constexpr int PAR = decltype(par_c)::value;
    // the next tap's bases (the last tap's successor is itself: its reads are in bounds and unused)
    const bool last = tap + 1 >= taps;
    const bool row_end = kw + 1 == p.KW;
    const int da = last ? 0 : (row_end ? drow : dcol);
    const int db = last ? 0 : CS * BSTEP;
    int na[MI], nb[2];
#pragma unroll
    for (int t = 0; t < MI; ++t) na[t] = pa[t] + da;
    nb[0] = pb[0] + db;
    nb[1] = pb[1] + db;
#pragma unroll
    for (int k = 0; k < CS / 2; ++k) {
      const bool cur0 = ((PAR + k) & 1) == 0;
      const bool more = k + 1 < CS / 2;
      // read pair k + 1 of this tap, or pair 0 of the next, into the other set
      if (cur0) {
        if (more) { read(pa, pb, 2 * k + 2, a10, b10); read(pa, pb, 2 * k + 3, a11, b11); }
        else { read(na, nb, 0, a10, b10); read(na, nb, 1, a11, b11); }
      } else {
        if (more) { read(pa, pb, 2 * k + 2, a00, b00); read(pa, pb, 2 * k + 3, a01, b01); }
        else { read(na, nb, 0, a00, b00); read(na, nb, 1, a01, b01); }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (cur0) { mfmas(a00, b00); mfmas(a01, b01); }
      else { mfmas(a10, b10); mfmas(a11, b11); }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < MI; ++t) pa[t] = na[t];
    pb[0] = nb[0];
    pb[1] = nb[1];
    kw = row_end ? 0 : kw + 1;
    ++tap;
  };
  // Two taps per iteration keep the set parity static when CS / 2 is odd.
  // The loop body has no data-dependent branch (one makes the compiler wait
  // for every outstanding read at the block boundary).
  int t2 = 0;
  for (; t2 + 2 <= taps; t2 += 2) {
    tap_body(std::integral_constant<int, 0>{});
    tap_body(std::integral_constant<int, (CS / 2) & 1>{});
  }
  if (t2 < taps) tap_body(std::integral_constant<int, 0>{});

  // D = P x F: lane l holds channel 32j + l%32; register v holds pixel
  // 8*(v/4) + 4*(l/32) + v%4 of the tile.  Pixels at or past qend get an
  // out-of-range offset (the store is dropped).
#pragma unroll
  for (int t = 0; t < MI; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int q = q0 + t * tstride + 8 * (v >> 2) + 4 * hi + (v & 3);
      const unsigned off = q < qend ? (unsigned)((q * p.CO + 32 * j + lr) * 4) : kOutOfRange;
      // the element goes through a scalar: __builtin_bit_cast of an
      // ext_vector element lvalue reads element 0 whatever the index.  An
      // i8 sum is an exact i32; it is rounded to f32 once (nearest even).
      const float val = static_cast<float>(acc[t][v]);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), orc, off, 0, 2);
    }
}

// Tiles m0, m0 + mstep, ... (< nmt) of pixels [qbeg, qend) against N tile j,
// up to four per pass.
template <int NT, int CS, int ELEM>
__device__ __forceinline__ void band_wave(const BandArgs& p, const band_lds_t* Fs, const band_lds_t* Hs,
                                          __amdgpu_buffer_rsrc_t orc, int qbeg, int qend, int m0, int mstep,
                                          int j, int lane) {
  const int nmt = (qend - qbeg + 31) >> 5;
  int n = m0 < nmt ? (nmt - m0 + mstep - 1) / mstep : 0;
  int q0 = qbeg + m0 * 32;
  const int tstride = mstep * 32;
  while (n > 0) {
    const int c = min(n, XT_BAND_MAX_MI);
    switch (c) {
      case 1: band_tiles<1, NT, CS, ELEM>(p, Fs, Hs, orc, q0, tstride, qend, j, lane); break;
      case 2: band_tiles<2, NT, CS, ELEM>(p, Fs, Hs, orc, q0, tstride, qend, j, lane); break;
      case 3: band_tiles<3, NT, CS, ELEM>(p, Fs, Hs, orc, q0, tstride, qend, j, lane); break;
      default: band_tiles<4, NT, CS, ELEM>(p, Fs, Hs, orc, q0, tstride, qend, j, lane); break;
    }
    q0 += c * tstride;
    n -= c;
  }
}

template <int NT, int CS, int ELEM>
__global__ __launch_bounds__(BWG, 1) void conv2d_band_kernel(BandArgs p) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char blds[];
  typedef __attribute__((address_space(3))) unsigned char lds_t;
  lds_t* Fs = (lds_t*)blds;  // filter [K][Cout]
  lds_t* Hs = Fs + p.filt_bytes;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Consecutive bands share halo rows: each XCD takes a contiguous run of
  // them, so a shared row is fetched into one L2 rather than two.
  const int band = xcd_contiguous(blockIdx.x, gridDim.x);
  const int n = band / p.bands_per_image;
  const int r0 = (band - n * p.bands_per_image) * p.R;
  const int rows = min(p.R, p.OH - r0);
  const int hrows = (rows - 1) * p.sh + (p.KH - 1) * p.dh + 1;
  // -- DMA: filter, then halo --------------------------------------------
  {
    const __amdgpu_buffer_rsrc_t fr = buffer_of(p.filt, p.filt_bytes);
    for (int i = wave; i < p.filt_instr; i += BWG / 64) {
      const unsigned b = (unsigned)i * 1024u + lane * 16u;
      const int k = b >> p.rb_shift;
      const int pos = (b - (k << p.rb_shift)) >> 4;
      const int chunk = pos ^ (p.fsw_unit * ((k >> p.fsw_shift) & p.fsw_mask));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(fr, (void __attribute__((address_space(3)))*)(Fs + i * 1024),
                                               16, (unsigned)((k << p.rb_shift) + chunk * 16), 0, 0, 0);
    }
    // Halo pixels are `pitch` bytes apart in LDS (an odd number of 16-byte
    // chunks, so sixteen consecutive pixels fall in sixteen distinct bank
    // groups) and halo rows `rpitch` bytes apart (padded so that a group of
    // sixteen output pixels that crosses an output row still does).  One DMA
    // instruction writes ppi whole pixels of one halo row: lane l carries
    // chunk l % nchp of pixel l / nchp; the pad chunk reads zero, and lanes
    // past ppi * nchp or past the row are masked off (no LDS write).
    const __amdgpu_buffer_rsrc_t ir = buffer_of(p.src + (size_t)n * p.image_bytes, p.image_bytes);
    const int ih0 = r0 * p.sh - p.pad_t, iw0 = -p.pad_l;
    const int lp = (int)udiv((unsigned)lane, p.m_nchp);
    const int lc = lane - lp * p.nchp;
    const int nch = p.nch;
    const int hinstr = hrows * p.ipr;
    for (int i = wave; i < hinstr; i += BWG / 64) {
      const int hr = (int)udiv((unsigned)i, p.m_ipr), piece = i - hr * p.ipr;
      const int hc = piece * p.ppi + lp;
      const int ih = ih0 + hr, iw = iw0 + hc;
      const bool inside = lc < nch && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
      const unsigned off = inside ? (unsigned)((ih * p.W + iw) * nch + lc) * 16u : kOutOfRange;
      if (lp < p.ppi && hc < p.rf_w)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ir, (void __attribute__((address_space(3)))*)(Hs + hr * p.rpitch + piece * p.ppi * p.pitch), 16, off,
            0, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA has landed
  __syncthreads();                // and every other wave's

  // -- compute ------------------------------------------------------------
  const int M = rows * p.OW;
  const int j = wave % NT;              // this wave's N tile
  constexpr int MSTEP = (BWG / 64) / NT; // M-tile stride between a wave's tiles
  const __amdgpu_buffer_rsrc_t orc =
      buffer_of(p.out + ((size_t)n * p.OH + r0) * p.OW * p.CO, (unsigned)(M * p.CO * 4));

  band_wave<NT, CS, ELEM>(p, Fs, Hs, orc, 0, M, wave / NT, MSTEP, j, lane);
}

TileOff to_off(const xt::TileAddr& a) { return TileOff{a.c0, a.sx, a.sy, a.sz}; }

template <int NT, bool BF16>
hipError_t launch_conv_t(const ConvArgs& a, dim3 grid, size_t lds, hipStream_t s) {
  auto fn = conv2d_kernel<NT, BF16>;
  if (lds > size_t(kMaxLds)) return hipErrorInvalidValue;
  hipError_t e = allow_full_lds(reinterpret_cast<const void*>(fn));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(fn, grid, dim3(WG), lds, s, a);
  return hipGetLastError();
}

template <int NT, int CS, int ELEM>
hipError_t launch_band_t(const BandArgs& a, int bands, size_t lds, hipStream_t s) {
  auto fn = conv2d_band_kernel<NT, CS, ELEM>;
  if (lds > size_t(kMaxLds)) return hipErrorInvalidValue;
  hipError_t e = allow_full_lds(reinterpret_cast<const void*>(fn));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(fn, dim3(bands), dim3(BWG), lds, s, a);
  return hipGetLastError();
}

int ilog2(unsigned v) {
  int r = 0;
  while ((1u << (r + 1)) <= v) ++r;
  return r;
}

// The band kernel applies when the Blocks tile images [0, gB) x all output
// rows and columns exactly once, in the output's natural NHWC addressing, and
// every Block uses one filter.  Returns false (nothing launched) when
// it does not apply; `e` carries a launch error otherwise.
bool try_band(const xt::Plan& p, void* const* bufs, hipStream_t s, int max_lds, int cus, hipError_t& e) {
  const xt::ConvPlan& c = p.conv;
  if (c.cb.axis < 0 || c.ch.axis < 0 || c.cw.axis < 0 || c.cb.axis == c.ch.axis || c.cb.axis == c.cw.axis ||
      c.ch.axis == c.cw.axis)
    return false;
  const long long gB = p.grid[c.cb.axis], gH = p.grid[c.ch.axis], gW = p.grid[c.cw.axis];
  if (gH * c.TH != c.out_H || gW * c.TW != c.out_W || c.out_C != c.CO) return false;
  auto step = [&](const xt::TileAddr& t, int axis) { return axis == 0 ? t.sx : axis == 1 ? t.sy : t.sz; };
  const long long plane = c.out_H * c.out_W * c.out_C;
  if (c.out_addr.c0 != 0 || (gB > 1 && step(c.out_addr, c.cb.axis) != plane) ||
      (gH > 1 && step(c.out_addr, c.ch.axis) != c.TH * c.out_W * c.out_C) ||
      (gW > 1 && step(c.out_addr, c.cw.axis) != c.TW * c.out_C))
    return false;
  // one filter for every Block (its origin may be any offset into a stack of filters)
  if (c.filt_addr.sx || c.filt_addr.sy || c.filt_addr.sz) return false;
  if (c.TB != 1 || c.TC != c.CO || c.out_elem != xt::Elem::F32) return false;
  const bool i8 = c.elem == xt::Elem::I8;
  const long long es = i8 ? 1 : 2;
  // a K step is 32 bytes of a pixel; steps go in pairs within a tap
  // (and the unrolled taps take 2, 4, 6 or 8 steps: Cin * esize in {64, 128, 192, 256})
  if ((c.C * es) % 64 || c.C * es > 256 || c.CO % 32 || c.CO > 128 || c.CO == 96) return false;
  const long long K = c.KH * c.KW * c.C;
  const long long filt_bytes = K * c.CO * es;
  if (filt_bytes % 1024) return false;
  const long long PB = c.C * es;
  // LDS pitch of a halo pixel: an odd number of 16-byte chunks
  const long long pitch = (PB / 16) % 2 ? PB : PB + 16;
  const long long nchp = pitch / 16;
  if (nchp > 64) return false;
  const long long ppi = 64 / nchp;
  const long long rf_w = (c.out_W - 1) * c.stride_w + (c.KW - 1) * c.dil_w + 1;
  const long long image_bytes = c.H * c.W * PB;
  if (image_bytes >= (1LL << 31) || filt_bytes >= (1LL << 31)) return false;
  // Halo rows are rpitch bytes apart: rf_w pixels plus g pad chunks, g the
  // smallest in [0, 16) for which a step to the next output row moves the
  // pixel address by OW * sw pixels modulo 16 chunks (sh * rpitch = OW * sw *
  // pitch mod 256 bytes), as a step along a row does.  Then the sixteen
  // consecutive output pixels of a fragment read hit sixteen distinct 16-byte
  // bank groups even where they cross an output row (with an unpadded row the
  // address jumps by (rf_w - OW) pixels there: C4's 2-pixel jump cost about
  // one bank-conflict cycle per LDS instruction).  No such g: no pad.
  long long gpad = 0;
  for (long long g = 0; g < 16; ++g)
    if ((c.stride_h * (rf_w * nchp + g) - c.out_W * c.stride_w * nchp) % 16 == 0) {
      gpad = g;
      break;
    }
  const long long rpitch = rf_w * pitch + 16 * gpad;
  const long long ipr = (rf_w + ppi - 1) / ppi;
  // rows per band: spread gB * OH rows over the CUs, shrink until LDS fits
  const long long total_rows = gB * c.out_H;
  long long R = std::min<long long>(c.out_H, (total_rows + cus - 1) / std::max(cus, 1));
  size_t lds = 0;
  long long hrows_max = 0;
  for (; R >= 1; --R) {
    hrows_max = (R - 1) * c.stride_h + (c.KH - 1) * c.dil_h + 1;
    const long long halo = hrows_max * rpitch;
    if (filt_bytes + halo <= max_lds) {
      lds = static_cast<size_t>(filt_bytes + halo);
      break;
    }
  }
  if (R < 1) return false;
  // the kernel divides pixel indices below 2^16 by multiply-high reciprocals
  if (hrows_max * ipr >= 65536 || R * c.out_W >= 65536 || rf_w >= 65536 || c.out_W >= 65536) return false;
  if (R * c.out_W * c.CO * 4 >= (1LL << 31)) return false;
  BandArgs a;
  a.src = static_cast<const unsigned char*>(bufs[c.src_arg]);
  a.filt = static_cast<const unsigned char*>(bufs[c.filt_arg]) + c.filt_addr.c0 * es;
  a.out = static_cast<float*>(bufs[c.out_arg]);
  for (const void* ptr : {(const void*)a.src, (const void*)a.filt, (const void*)a.out})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) return false;
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
  a.dw = (int)c.dil_w;
  a.R = (int)R;
  a.bands_per_image = (int)((c.out_H + R - 1) / R);
  a.rf_w = (int)rf_w;
  a.K = (int)K;
  a.steps = (int)(K * es / 32);
  // Filter rows of RB = Cout * esize bytes.  The transposed reads of one
  // half-wave cover 64 bytes of four consecutive rows (16-bit) or 32 bytes of
  // eight rows (8-bit); XOR that block index with the row's position inside
  // a 256-byte bank window so the rows fall in distinct banks.
  const int RB = (int)(a.CO * es);
  const int blk = i8 ? 32 : 64;
  a.rb_shift = ilog2((unsigned)RB);
  a.fsw_unit = blk / 16;
  a.fsw_shift = ilog2(256 / RB);
  a.fsw_mask = RB / blk - 1;
  a.nch = (int)(PB / 16);
  a.pitch = (int)pitch;
  a.rpitch = (int)rpitch;
  a.nchp = (int)nchp;
  a.ppi = (int)ppi;
  a.ipr = (int)ipr;
  a.m_nchp = udiv_magic((unsigned)nchp);
  a.m_ipr = udiv_magic((unsigned)ipr);
  a.m_ow = udiv_magic((unsigned)c.out_W);
  a.filt_instr = (int)(filt_bytes / 1024);
  a.filt_bytes = (unsigned)filt_bytes;
  a.image_bytes = (unsigned)image_bytes;
  const long long bands = gB * a.bands_per_image;
  if (!grid_fits(bands, 512)) return false;
  const int el = i8 ? kBandI8 : c.elem == xt::Elem::BF16 ? kBandBF16 : kBandF16;
  const int nt = a.CO / 32;
  const int cs = (int)(PB / 32);  // K steps per tap: 2, 4, 6 or 8 (checked above)
#define XT_BAND_E(NTV, CSV)                                                                \
  do {                                                                                    \
    if (el == kBandI8) e = launch_band_t<NTV, CSV, kBandI8>(a, (int)bands, lds, s);        \
    else if (el == kBandBF16) e = launch_band_t<NTV, CSV, kBandBF16>(a, (int)bands, lds, s); \
    else e = launch_band_t<NTV, CSV, kBandF16>(a, (int)bands, lds, s);                     \
  } while (0)
#define XT_BAND(NTV)                      \
  do {                                    \
    if (cs == 2) XT_BAND_E(NTV, 2);       \
    else if (cs == 4) XT_BAND_E(NTV, 4);  \
    else if (cs == 6) XT_BAND_E(NTV, 6);  \
    else XT_BAND_E(NTV, 8);               \
  } while (0)
  switch (nt) {
    case 1: XT_BAND(1); break;
    case 2: XT_BAND(2); break;
    default: XT_BAND(4); break;
  }
#undef XT_BAND
#undef XT_BAND_E
  return true;
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
  a.pitch = 2 * a.C + 16;
  const int K = a.KH * a.KW * a.C;
  a.kpitch = 2 * K + 16;
  a.steps = K / 16;
  const int nt = (a.CO + 31) / 32;
  bool persistent_ok = c.elem != xt::Elem::I8 && c.out_elem == xt::Elem::F32 && c.TB == 1 && c.TC == c.CO &&
                       a.C % 32 == 0 && a.CO % 16 == 0 && a.CO <= 128 && a.out_C % 4 == 0 &&
                       a.tf.c0 % 8 == 0 && a.tf.sx == 0 && a.tf.sy == 0 && a.tf.sz == 0;
  for (const void* ptr : {(const void*)a.src, (const void*)a.filt, (const void*)a.out})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) persistent_ok = false;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int max_lds = 0, cus = 0;
  e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  // XTILE_AMD_CONV_IGEMM=1 puts the implicit-GEMM kernel first (tests run it
  // on shapes the band kernel takes)
  const char* igemm_env = std::getenv("XTILE_AMD_CONV_IGEMM");
  const bool igemm_first = igemm_env && igemm_env[0] == '1';
  if (igemm_first && launch_conv2d_igemm(p, bufs, s, e)) return e;
  if (try_band(p, bufs, s, max_lds, cus, e)) return e;
  // filters beyond the band kernel's LDS: each image resident in LDS when
  // its channels fit there, else the implicit GEMM with DMA operands
  if (launch_conv2d_image(p, bufs, s, e)) return e;
  if (launch_conv2d_igemm(p, bufs, s, e)) return e;
  // Cin below 8 (the RGB stem): input rows staged in LDS, K in runs of KW * Cin
  if (launch_conv2d_small(p, bufs, s, e)) return e;
  // the persistent kernel: f16 / bf16 in, f32 out, one image per Block, every
  // output channel, 16-byte channel runs; anything else takes the generic kernel
  if (!persistent_ok) return launch_conv2d_general(p, bufs, s, why);
  // Largest work unit (rows dividing TH) whose halo fits beside the filter.
  const int ntp = nt == 3 ? 4 : nt;  // N tiles compiled: 1, 2 or 4
  const size_t filt_bytes = size_t(ntp) * 32 * a.kpitch;
  size_t lds = 0;
  a.UR = 0;
  for (int ur = a.TH; ur >= 1; --ur) {
    if (a.TH % ur) continue;
    const int rf_h = (ur - 1) * a.sh + a.dh * (a.KH - 1) + 1;
    const int rf_w = (a.TW - 1) * a.sw + a.dw * (a.KW - 1) + 1;
    const long long halo_vecs = (long long)rf_h * rf_w * (a.C / 8);
    const size_t need = filt_bytes + size_t(rf_h) * rf_w * a.pitch + 4 * 32 * kOutPitch;
    if (halo_vecs <= HT * HV && need <= size_t(max_lds) && rf_w < 65536 && rf_h < 32767) {
      a.UR = ur;
      a.rf_h = rf_h;
      a.rf_w = rf_w;
      a.halo_vecs = static_cast<int>(halo_vecs);
      a.halo_bytes = rf_h * rf_w * a.pitch;
      lds = need;
      break;
    }
  }
  if (a.UR == 0) return launch_conv2d_general(p, bufs, s, why);  // halo + filter exceed LDS
  a.nmt = (a.UR * a.TW + 31) / 32;
  a.m_cv = udiv_magic(a.C / 8);
  a.m_rfw = udiv_magic(a.rf_w);
  a.m_tw = udiv_magic(a.TW);
  a.m_cg = udiv_magic(a.CO / 8);
  const long long image_bytes = (long long)a.H * a.W * a.C * 2;
  const long long unit_out_bytes = (long long)a.UR * a.out_W * a.out_C * 4;
  if (image_bytes >= (1LL << 31) || unit_out_bytes >= (1LL << 31)) return launch_conv2d_general(p, bufs, s, why);
  a.image_bytes = static_cast<unsigned>(image_bytes);
  a.unit_out_bytes = static_cast<unsigned>(unit_out_bytes);
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
  switch (ntp) {
    case 1: if (bf16) XT_CONV(1, true); else XT_CONV(1, false); break;
    case 2: if (bf16) XT_CONV(2, true); else XT_CONV(2, false); break;
    default: if (bf16) XT_CONV(4, true); else XT_CONV(4, false); break;
  }
#undef XT_CONV
  return e;
}

}  // namespace xtk
