// Tile matmul C = epilogue(A @ B) on the gfx950 matrix cores.
//
// Semantics: xt.matmul over one Block's tiles, the whole K extent of the tile
// (kernels/matmul.py:11-16,35; lib/xt/XTOps.cpp:218-253): f16 x f16 and
// bf16 x bf16 accumulate in f32 (the narrow-float extension); i8 x i8
// accumulates exactly in i32 and the result is f32.  The optional epilogue is
// the one of kernels/matmul.py:15-17: t * scale + bias with (1, TN) row tiles
// broadcast over the rows (two separately rounded f32 operations, never fused),
// then astype(int8) = xt.ftoi (round half to even, saturate to [-128, 127],
// NaN -> 0; the reference fixes no rule, this is the oracle's).
//
// Workgroup tiles are decoupled from xt Block tiles.  A Block's TM x TN output
// tile is split into (TM/BM) x (TN/BN) workgroup tiles when it is larger, and
// neighbouring Blocks are fused into one workgroup tile when it is smaller and
// the planner's affine addresses show them to be contiguous (the next Block
// along one grid axis continues the same A rows / B columns / C tile / scale
// and bias columns).  Blocks are independent (README.md:85-89), so both are
// pure scheduling choices.
//
// Programs whose Blocks map onto 256 x 256, 256 x 128, 128 x 256 or 128 x 128
// workgroup tiles run on gemm_dma_kernel (operands landed in LDS by DMA;
// described where it is defined), whatever the element type and result:
// 256 x 256 when its tiles fill the CUs (or are few enough to split K), else
// the first smaller tile whose tiles fill them, else the one with the most
// tiles (launch_gemm).  Blocks that map onto 64 x 64 tiles only run on
// gemm_kernel, a template for BM x BN tiles (instantiated at 64 x 64):
//   * 4 waves of (BM/2) x (BN/2), v_mfma_f32_32x32x16_{f16,bf16} or
//     v_mfma_i32_32x32x32_i8.  Every fragment is 16 bytes per lane, so one
//     K slice is 128 bytes of every row whatever the element type (64 f16/bf16
//     or 128 i8 values) and the staging below moves bytes.
//   * A rows (K-contiguous) go global -> VGPR -> LDS as 16-byte vectors.  B is
//     N-contiguous in memory but the matrix cores want K-contiguous lanes, so
//     each thread loads an 8(k) x 8(n) block of 16-bit values or a
//     16(k) x 8(n) block of bytes and transposes it in registers (16-bit
//     halves, or 4x4 byte transposes with v_perm_b32) into eight N rows.
//   * LDS tiles are unpadded [rows][128 B] arrays whose 16-byte chunks are
//     XOR-swizzled (chunk c of row r at c ^ swz(r)): fragment reads and the
//     transposed B stores both run at the bank-conflict-free rate.
//   * Two register staging sets keep two K slices in flight; sched_group_barrier
//     interleaves every MFMA with at most one fragment read, one global load,
//     one LDS store and two VALU ops.
//   * For an f32 result a half-wave stores one whole 128-byte line per
//     accumulator register.  For an i8 result the MFMAs compute
//     D = B^T-fragment x A-fragment instead, so each lane holds runs of four
//     consecutive output columns of one row and writes them as one 4-byte
//     store.
//   * Workgroups are dispatched round-robin over the 8 XCDs; the linear id is
//     remapped so that each XCD receives a contiguous run of tiles, and tiles
//     are ordered in groups of GROUP tile columns so that concurrently resident
//     workgroups share A and B panels in their XCD's L2.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr int SLICE = 128;  // bytes of K per LDS row and K slice
// K stages of gemm_dma_kernel in LDS: a stage's DMA has two stages of compute
// to land; three and five stages measured no faster on C3 (bench.py: four
// and five both 129.7 us before the DMA was spread over the MFMA slots)
constexpr int kDmaStages = 4;
constexpr int kTileGroup = 8;  // tile columns per group of the workgroup order

enum { kF16 = 0, kBF16 = 1, kI8 = 2 };

// Waves of gemm_dma_kernel: 4 (one per SIMD, 128 x 128 each) or 8 (two per
// SIMD, 128 x 64 each: half an LDS read more per MFMA, but a second wave to
// issue MFMAs while one waits).  Measured in one call (bench.py, 2000
// launches): C3 (f16) 122.6 us with 4 and 124.0 with 8, C5 (bf16) 319.9 and
// 317.2, C6 (i8) 72.6 and 71.2.
template <int ELEM>
constexpr int dma_waves() { return ELEM == kF16 ? 4 : 8; }

typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int16v __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const unsigned char* a;
  const unsigned char* b;
  void* c;
  const float* scale;
  const float* bias;
  TileOff ta, tb, tc, ts, tbias;  // element offsets
  long long lda, ldb, ldc;        // row pitches in elements
  int nk;                         // K slices
  int vgx, vgy;                   // virtual grid (fused axes divided by their factor)
  int mul[3];                     // block id = virtual id * mul (fused axes)
  int sub_m, sub_n;               // workgroup tiles per (fused) Block along M and N
  int nwg;
  int group;
  int has_scale, has_bias;
  // K split (DMA kernel, f32 results without an epilogue): nwg = tiles *
  // ksplit workgroups, K range r covering stages [r S / ksplit, (r + 1) S /
  // ksplit) of the S = 2 nk stages of 64 K bytes (ranges differ by at most
  // one stage; kstages = the shortest); ksplit = 1, tiles = nwg otherwise
  int tiles, ksplit, kstages;
};

template <int ELEM>
struct Acc {
  typedef float16v type;
};
template <>
struct Acc<kI8> {
  typedef int16v type;
};

template <int ELEM>
__device__ __forceinline__ typename Acc<ELEM>::type mfma(uint4v a, uint4v b, typename Acc<ELEM>::type c) {
  if constexpr (ELEM == kI8)
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(int4v, a), __builtin_bit_cast(int4v, b), c,
                                                 0, 0, 0);
  else if constexpr (ELEM == kBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c,
                                                  0, 0, 0);
}

// Workgroup -> tile origins.  Contiguous runs per XCD, then GROUP-wide column
// groups over the virtual grid.
struct TilePtrs {
  const unsigned char* A;
  const unsigned char* B;
  long long c_off;  // element offset of the C tile
  const float* S;
  const float* Bias;
};

// The workgroup's linear id with contiguous runs per XCD: the K range is
// gemm_lin / tiles, the tile gemm_lin % tiles.
__device__ __forceinline__ int gemm_lin(const GemmArgs& p) {
  int L = blockIdx.x;
  if ((p.nwg & 7) == 0) L = (L & 7) * (p.nwg >> 3) + (L >> 3);
  return L;
}

template <int ELEM, int BM, int BN, bool KS = false>
__device__ __forceinline__ TilePtrs gemm_tile_of(const GemmArgs& p) {
  constexpr int ES = ELEM == kI8 ? 1 : 2;
  int L = gemm_lin(p);
  if constexpr (KS) L -= (L / p.tiles) * p.tiles;
  const int subs = p.sub_m * p.sub_n;
  const int s = L % subs;
  int blk = L / subs;
  const int sm = s / p.sub_n;
  const int sn = s - sm * p.sub_n;
  const int per_plane = p.vgx * p.vgy;
  const int vz = blk / per_plane;
  blk -= vz * per_plane;
  const int per_group = p.group * p.vgy;
  const int gid = blk / per_group;
  const int first = gid * p.group;
  const int gsize = min(p.group, p.vgx - first);
  const int r = blk - gid * per_group;
  const int x = (first + r % gsize) * p.mul[0];
  const int y = (r / gsize) * p.mul[1];
  const int z = vz * p.mul[2];
  TilePtrs t;
  t.A = p.a + (p.ta.at(x, y, z) + (long long)sm * BM * p.lda) * ES;
  t.B = p.b + p.tb.at(x, y, z) * ES + (long long)sn * BN * ES;
  t.c_off = p.tc.at(x, y, z) + (long long)sm * BM * p.ldc + (long long)sn * BN;
  t.S = p.scale + p.ts.at(x, y, z) + sn * BN;
  t.Bias = p.bias + p.tbias.at(x, y, z) + sn * BN;
  return t;
}

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// 4x4 byte transpose: rows a..d (byte i = column i) -> o[i] = column i
// (byte j = row j).  v_perm_b32 takes bytes 0-3 from its second and 4-7 from
// its first source.
__device__ __forceinline__ void transpose4x4(unsigned a, unsigned b, unsigned c, unsigned d, unsigned (&o)[4]) {
  const unsigned ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const unsigned ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const unsigned cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);
  const unsigned cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);
  o[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);  // a0 b0 c0 d0
  o[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// Global -> VGPR staging of one K slice and the VGPR -> LDS stores.  B
// sub-blocks: nb = sb % (BN/8) selects 8 output columns, kb = sb / (BN/8) the
// 16-byte chunk of K (8 values of 16 bits or 16 bytes).
template <int ELEM, int BM, int BN>
struct Stager {
  static constexpr int AV = BM * 8 / 256;      // 16-byte A vectors per thread
  static constexpr int NB = BN / 8;            // B column blocks
  static constexpr int BSUB = 8 * NB;          // B sub-blocks per slice
  static constexpr int BROWS = ELEM == kI8 ? 16 : 8;
  static constexpr int KPS = ELEM == kI8 ? SLICE : SLICE / 2;  // K values per slice
  uint4v ra[AV];
  uint4v rb[ELEM == kI8 ? 1 : 8];  // 16-bit: 8 rows of 8 values
  uint2v rb8[ELEM == kI8 ? 16 : 1];  // bytes: 16 rows of 8 values

  // Buffer loads: the descriptors cover the workgroup's A and B panels, each
  // lane keeps one 32-bit offset, and the per-slice / per-row parts travel as
  // the uniform scalar offset, so the staging needs no per-row pointers.
  // lda, ldb in bytes.
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t A, __amdgpu_buffer_rsrc_t B, unsigned lda,
                                       unsigned ldb, int kt, int tid) {
    const unsigned va = (unsigned)(tid >> 3) * lda + (tid & 7) * 16;
#pragma unroll
    for (int i = 0; i < AV; ++i)
      ra[i] = __builtin_amdgcn_raw_buffer_load_b128(A, va, kt * SLICE + i * 32 * lda, 0);
    if (BSUB >= 256 || tid < BSUB) {
      const int nb = (unsigned)tid % NB, kb = (unsigned)tid / NB;
      if constexpr (ELEM == kI8) {
        const unsigned vb = (unsigned)(kb * 16) * ldb + nb * 8;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          rb8[i] = __builtin_bit_cast(uint2v, __builtin_amdgcn_raw_buffer_load_b64(B, vb, (kt * KPS + i) * ldb, 0));
      } else {
        const unsigned vb = (unsigned)(kb * 8) * ldb + nb * 16;
#pragma unroll
        for (int i = 0; i < 8; ++i) rb[i] = __builtin_amdgcn_raw_buffer_load_b128(B, vb, (kt * KPS + i) * ldb, 0);
      }
    }
  }

  __device__ __forceinline__ void store(unsigned char (*As)[SLICE], unsigned char (*Bs)[SLICE], int tid) const {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      *reinterpret_cast<uint4v*>(&As[row][(cv ^ swz(row)) * 16]) = ra[i];
    }
    if (BSUB >= 256 || tid < BSUB) {
      const int nb = (unsigned)tid % NB, kb = (unsigned)tid / NB;
      if constexpr (ELEM == kI8) {
        // rows k = 0..15 of columns n = 0..7 -> column n holds 16 K bytes
        uint4v col[8];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            unsigned o[4];
            transpose4x4(rb8[4 * q][h], rb8[4 * q + 1][h], rb8[4 * q + 2][h], rb8[4 * q + 3][h], o);
#pragma unroll
            for (int i = 0; i < 4; ++i) col[4 * h + i][q] = o[i];
          }
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const int r = nb * 8 + n;
          *reinterpret_cast<uint4v*>(&Bs[r][(kb ^ swz(r)) * 16]) = col[n];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // columns n = 2j (low halves) and 2j+1 (high halves) of the 8 loaded rows
          uint4v even, odd;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const unsigned lo = rb[2 * q][j], hi = rb[2 * q + 1][j];
            even[q] = (lo & 0xFFFFu) | (hi << 16);
            odd[q] = (lo >> 16) | (hi & 0xFFFF0000u);
          }
          const int r0 = nb * 8 + 2 * j, r1 = r0 + 1;
          *reinterpret_cast<uint4v*>(&Bs[r0][(kb ^ swz(r0)) * 16]) = even;
          *reinterpret_cast<uint4v*>(&Bs[r1][(kb ^ swz(r1)) * 16]) = odd;
        }
      }
    }
  }
};

// x * s + b as two separately rounded f32 operations.
__device__ __forceinline__ float scale_bias(float x, float s, float b, bool hs, bool hb) {
#pragma clang fp contract(off)
  float t = hs ? x * s : x;
  return hb ? t + b : t;
}

__device__ __forceinline__ int ftoi_i8(float v) {
  if (v != v) return 0;
  const float r = __builtin_rintf(v);  // round half to even
  return (int)fminf(fmaxf(r, -128.f), 127.f);
}

// The same conversion in three instructions: v_rndne_f32 (half to even),
// v_cvt_i32_f32 (saturates out-of-range values and infinities, converts NaN
// to 0; issued as assembly because a C++ cast of such values is undefined),
// v_med3_i32 (clamp to [-128, 127]).
__device__ __forceinline__ int ftoi_i8_fast(float v) {
  int i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(__builtin_rintf(v)));
  return min(max(i, -128), 127);
}

// Low bytes of four ints packed into one word (byte e from q[e]).
__device__ __forceinline__ unsigned pack_i8x4(const int (&q)[4]) {
  const unsigned lo = __builtin_amdgcn_perm((unsigned)q[1], (unsigned)q[0], 0x0c0c0400u);  // q0 q1 0 0
  const unsigned hi = __builtin_amdgcn_perm((unsigned)q[3], (unsigned)q[2], 0x04000c0cu);  // 0 0 q2 q3
  return lo | hi;
}

template <int ELEM, int BM, int BN, bool OUT_I8>
__global__ __launch_bounds__(256, BM * BN >= 65536 ? 1 : 2) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / 2, WN = BN / 2;  // 2 x 2 waves
  constexpr int MI = WM / 32, NI = WN / 32;
  constexpr int KS = SLICE / 32;  // MFMA K steps per slice (32 bytes each: 16 f16 or 32 i8)
  typedef typename Acc<ELEM>::type acc_t;
  __shared__ __attribute__((aligned(16))) unsigned char As[2][BM][SLICE];
  __shared__ __attribute__((aligned(16))) unsigned char Bs[2][BN][SLICE];

  const TilePtrs t = gemm_tile_of<ELEM, BM, BN>(p);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  Stager<ELEM, BM, BN> st0, st1;
  acc_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  const int nk = p.nk;  // >= 1
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(t.A), (short)0,
                                                                       (int)0xFFFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(t.B), (short)0,
                                                                       (int)0xFFFFFFFF, 0x00020000);
  const unsigned lda = (unsigned)(p.lda * (ELEM == kI8 ? 1 : 2)), ldb = (unsigned)(p.ldb * (ELEM == kI8 ? 1 : 2));
  st0.load(ra, rb, lda, ldb, 0, tid);
  st1.load(ra, rb, lda, ldb, min(1, nk - 1), tid);
  st0.store(As[0], Bs[0], tid);
  __syncthreads();
  const int lrow = lane & 31;
  uint4v af[2][MI], bfr[2][NI];
  // 16-byte chunk of this lane's K values in step ks: 2*ks + lane/32
  auto read_frags = [&](int buf, int ks, int set) {
    const int c = ks * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int r = wm * WM + i * 32 + lrow;
      af[set][i] = *reinterpret_cast<const uint4v*>(&As[buf][r][(c ^ swz(r)) * 16]);
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int r = wn * WN + j * 32 + lrow;
      bfr[set][j] = *reinterpret_cast<const uint4v*>(&Bs[buf][r][(c ^ swz(r)) * 16]);
    }
  };
  // One K slice: compute from LDS[cur], request slice kt+2 into `next2`, move
  // slice kt+1 from `next1` into LDS[cur^1].  Branch-free: slice indices are
  // clamped to the last slice, whose repeated copies land in the idle buffer.
  auto slice = [&](int kt, Stager<ELEM, BM, BN>& next2, const Stager<ELEM, BM, BN>& next1) {
    const int cur = kt & 1;
    read_frags(cur, 0, 0);
    next2.load(ra, rb, lda, ldb, min(kt + 2, nk - 1), tid);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_frags(cur, ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = OUT_I8 ? mfma<ELEM>(bfr[ks & 1][j], af[ks & 1][i], acc[i][j])
                             : mfma<ELEM>(af[ks & 1][i], bfr[ks & 1][j], acc[i][j]);
    }
    next1.store(As[cur ^ 1], Bs[cur ^ 1], tid);
    __builtin_amdgcn_sched_group_barrier(0x100, MI + NI, 0);
#pragma unroll
    for (int g = 0; g < MI * NI * KS; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
    __syncthreads();
  };
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    slice(kt, st0, st1);      // st1 holds slice kt+1; st0 now fetches kt+2
    slice(kt + 1, st1, st0);  // st0 holds slice kt+2; st1 now fetches kt+3
  }
  if (kt < nk) slice(kt, st0, st1);

  const bool hs = p.has_scale, hb = p.has_bias;
  if constexpr (OUT_I8) {
    // D = B^T x A per 32x32 tile: lane l holds output row m = l%32 of tile i
    // and register v output column 8*(v/4) + 4*(l/32) + v%4 of tile j, so four
    // consecutive columns pack into one 4-byte store.
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n0 = wn * WN + j * 32 + 8 * g + 4 * (lane >> 5);
        float4v sv = {1.f, 1.f, 1.f, 1.f}, bv = {0.f, 0.f, 0.f, 0.f};
        if (hs) sv = *reinterpret_cast<const float4v*>(t.S + n0);
        if (hb) bv = *reinterpret_cast<const float4v*>(t.Bias + n0);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const long long off = t.c_off + (long long)(wm * WM + i * 32 + lrow) * p.ldc + n0;
          unsigned packed = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float y = scale_bias((float)acc[i][j][4 * g + e], sv[e], bv[e], hs, hb);
            packed |= (unsigned)(ftoi_i8(y) & 0xff) << (8 * e);
          }
          *reinterpret_cast<unsigned*>(static_cast<signed char*>(p.c) + off) = packed;
        }
      }
  } else {
    // D = A x B per 32x32 tile: lane l holds output column l%32 of tile j and
    // register v row 8*(v/4) + 4*(l/32) + v%4 of tile i; a half-wave writes one
    // whole 128-byte line per register.
    const int orow = (lane >> 5) * 4;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int n = wn * WN + j * 32 + lrow;
      const float sv = hs ? t.S[n] : 1.f, bv = hb ? t.Bias[n] : 0.f;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const long long off = t.c_off + (long long)(wm * WM + i * 32 + (v >> 2) * 8 + orow + (v & 3)) * p.ldc + n;
          static_cast<float*>(p.c)[off] = scale_bias((float)acc[i][j][v], sv, bv, hs, hb);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// 256 x 256 GEMM whose operands reach LDS by DMA (buffer_load ... lds): no
// VGPR staging, no register transposes, no LDS stores.  f16 / bf16 or i8
// operands; an f32 result, or (OUT_I8) the i8 result of the epilogue.
//   * NW = 4 waves of 128 x 128 (4 x 4 tiles of v_mfma_f32_32x32x16_{f16,bf16}
//     or v_mfma_i32_32x32x32_i8), one per SIMD, or NW = 8 waves of 128 x 64
//     (4 x 2 tiles), two per SIMD.  A stage is 64 bytes of K
//     (32 f16 / bf16 or 64 i8 values): A [256 rows][64 B] and B [KR k][BR B]
//     (32 x 512 B, or 64 x 256 B for i8), 16 KB each, in one of NS LDS
//     buffers (each its own LDS variable, so that reading one while DMA into
//     others is in flight needs no wait).
//   * A DMA instruction fills 1 KB of LDS, lane L at byte 16 L.  The layouts
//     are swizzled by choosing which global chunk each lane fetches: A row r
//     keeps its 16-byte chunk c at position c ^ ((r >> 2) & 3), so a
//     16-lane phase of fragment reads (16 consecutive rows) hits 16 distinct
//     16-byte bank groups.  16-bit B row k keeps chunk c at c ^ 4 (k & 3), so
//     the four rows a half-wave reads with ds_read_b64_tr_b16 fall in four
//     different 64-byte bank groups; i8 B row k keeps it at c ^ 2 (k & 7), so
//     the eight rows a half-wave reads with ds_read_b64_tr_b8 fall in eight
//     different 32-byte bank groups.
//   * B fragments come straight from the [k][n] layout through the
//     transposing reads: lane l receives column l % 32 and the 16 bytes of K
//     16 (l / 32) .. + 15 (bytes), 8 from each of two reads, the operand
//     layout of the MFMA.  A 16-lane group of ds_read_b64_tr_b16 reads a
//     4 (k) x 16 (n) block, lane i at row i / 4 and columns 4 (i % 4) .. + 3;
//     of ds_read_b64_tr_b8 an 8 x 16 block, lane i at row i / 2 and columns
//     8 (i % 2) .. + 7.
//   * For an i8 result the MFMAs compute D = B^T-fragment x A-fragment, so
//     each lane holds runs of four consecutive output columns of one row and
//     writes them as one 4-byte store.
//   * Barrier B_s opens stage s.  Before it each wave waits for its own DMA
//     of stages s and s + 1 and for its LDS reads; so after it every wave's
//     DMA of both stages has landed and every wave is done with stage s - 1.
//     Then the DMA of stage s + NS - 1 goes into stage s - 1's buffer, the
//     stage's two K steps run (32 MFMAs a wave), and the first fragments of
//     stage s + 1 are read before B_{s+1}, so no barrier is followed by an
//     LDS round trip.  A stage's DMA has NS - 2 stages of compute to land.
//     The barrier is a bare s_barrier: __syncthreads' release fence would
//     also wait for the DMA that should stay in flight.
template <int ELEM, int NS, bool OUT_I8, bool EPI, int NW, bool KS = false, int BMT = 256, int BNT = 256>
__global__ __launch_bounds__(64 * NW, BMT * BNT <= 128 * 128 ? 2 : 1) void gemm_dma_kernel(GemmArgs p) {
  static_assert(!KS || (!EPI && !OUT_I8), "K split only without an epilogue");
  static_assert(NS >= 3 && NS <= 5, "stages");
  static_assert(NW == 4 || NW == 8, "waves");
  static_assert((BMT == 256 || BMT == 128) && (BNT == 256 || BNT == 128) && (NW == 4 || BMT * BNT == 65536),
                "tiles");
  // NW = 4: 2 x 2 waves of (BM / 2) x (BN / 2); NW = 8 (256 x 256 only): 2 x 4
  // waves of 128 x 64 (two waves per SIMD)
  constexpr int BM = BMT, BN = BNT, WM = BM / 2, WN = 2 * BN / NW, MI = WM / 32, NI = WN / 32;
  constexpr int ES = ELEM == kI8 ? 1 : 2;  // bytes per element
  constexpr int KB = 64;            // K bytes per A row and stage
  constexpr int AB = BM * KB;       // A bytes per stage
  constexpr int BR = BN * ES;       // B bytes per k row
  constexpr int KR = KB / ES;       // B k rows per stage
  constexpr int RPI = 1024 / BR;    // B k rows per DMA instruction
  constexpr int KSR = 32 / ES;      // B k rows per MFMA K step
  constexpr int STAGE = AB + KR * BR;
  constexpr int PA = BM / 16 / NW;  // A DMA instructions (16 rows each) per wave and stage
  constexpr int PB = KR * BR / 1024 / NW;  // B DMA instructions per wave and stage
  constexpr int PER = PA + PB;      // DMA instructions per wave and stage
  typedef typename Acc<ELEM>::type acc_t;
  typedef __attribute__((address_space(3))) unsigned char lds_t;
  __shared__ __attribute__((aligned(1024))) unsigned char S0[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char S1[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char S2[STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char S3[NS > 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char S4[NS > 4 ? STAGE : 16];
  unsigned char* const buf[5] = {S0, S1, S2, S3, S4};

  const TilePtrs t = gemm_tile_of<ELEM, BM, BN, KS>(p);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);
  static_assert(WM * 2 == BM && WN * (NW / 2) == BN, "wave layout");
  const i32x4 ra = raw_rsrc(t.A), rb = raw_rsrc(t.B);
  const unsigned lda = (unsigned)(p.lda * ES), ldb = (unsigned)(p.ldb * ES);
  // this workgroup's stages of 64 K bytes: [kbase, kbase + nk)
  const int krange = KS ? gemm_lin(p) / p.tiles : 0;
  const int kbase = KS ? (int)((long long)krange * (p.nk * 2) / p.ksplit) : 0;
  const int nk = KS ? (int)((long long)(krange + 1) * (p.nk * 2) / p.ksplit) - kbase : p.nk * 2;

  // B row k keeps its 16-byte chunk c at c ^ bsw(k) (rows of 128-byte i8:
  // (k / 2) % 4, so the eight rows a half-wave's tr_b8 read covers still
  // fall in distinct 16-byte bank groups)
  auto bsw = [](int k) { return ES == 2 ? 4 * (k & 3) : BR == 128 ? (k >> 1) & 3 : 2 * (k & 7); };
  // DMA lane offsets.  A instruction i (rows 16i .. 16i+15): lane L holds
  // row 16i + L/4 at position L%4, i.e. chunk (L%4) ^ ((L/16) & 3).  B
  // instruction i (k rows RPI i .. + RPI - 1, CPR chunks each): lane
  // (h, pc) = (L / CPR, L % CPR) holds chunk pc ^ bsw(RPI i + h), which
  // depends on i only through i & 1.
  constexpr int CPR = BR / 16;
  const unsigned va = (unsigned)(lane >> 2) * lda + (unsigned)(((lane & 3) ^ ((lane >> 4) & 3)) << 4);
  unsigned vb[2];
  {
    const int h = lane / CPR, pc = lane % CPR;
#pragma unroll
    for (int q = 0; q < 2; ++q) vb[q] = (unsigned)h * ldb + (unsigned)((pc ^ bsw(RPI * q + h)) << 4);
  }
  // this wave's share of stage kt: A instructions PA w .. + PA - 1 (q < PA),
  // B instructions PB w .. + PB - 1 (q >= PA)
  auto dma_one = [&](int kt, unsigned char* S, int q) {
    const int kg = kt + kbase;
    if (q < PA) {
      const int i = wave * PA + q;
      dma16(ra, lds_addr(S + i * 1024), va, (unsigned)(16 * i) * lda + (unsigned)kg * KB);
    } else {
      const int i = wave * PB + (q - PA);
      dma16(rb, lds_addr(S + AB + i * 1024), vb[i & 1], (unsigned)(kg * KR + RPI * i) * ldb);
    }
  };
  auto dma = [&](int kt, unsigned char* S) {
#pragma unroll
    for (int q = 0; q < PER; ++q) dma_one(kt, S, q);
  };

  // fragment offsets: A row r at r * 64, chunk c at c ^ ((r >> 2) & 3); B per
  // (tile j, read h) an offset in the stage's first K step, plus KSR rows for
  // the second
  const int lrow = lane & 31, hi = lane >> 5;
  int arow[MI], asw[MI], boff[NI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int r = wm * WM + i * 32 + lrow;
    arow[i] = r * KB;
    asw[i] = (r >> 2) & 3;
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
          cb = (wn * WN + j * 32 + 16 * (g & 1) + 4 * (li & 3)) * 2;
        } else {
          k = 16 * (g >> 1) + 8 * h + (li >> 1);
          cb = wn * WN + j * 32 + 16 * (g & 1) + 8 * (li & 1);
        }
        boff[j][h] = AB + k * BR + (((cb >> 4) ^ bsw(k)) << 4) + (cb & 15);
      }
  }
  acc_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
  uint4v af[2][MI], bfr[2][NI];
  auto read_a = [&](const unsigned char* S, int ks, int set, int i) {
    af[set][i] = *reinterpret_cast<const uint4v*>(S + arow[i] + (((ks * 2 + hi) ^ asw[i]) << 4));
  };
  auto read_b = [&](const unsigned char* S, int ks, int set, int j) {
    lds_t* const f = (lds_t*)(S + ks * KSR * BR);
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
    bfr[set][j] = uint4v{l2[0], l2[1], h2[0], h2[1]};
  };
  auto read_frags = [&](const unsigned char* S, int ks, int set) {
#pragma unroll
    for (int i = 0; i < MI; ++i) read_a(S, ks, set, i);
#pragma unroll
    for (int j = 0; j < NI; ++j) read_b(S, ks, set, j);
  };
  // D = A x B, or D^T = B^T x A^T for an i8 result
  auto mma = [&](int set, int i, int j) {
    if constexpr (OUT_I8) acc[i][j] = mfma<ELEM>(bfr[set][j], af[set][i], acc[i][j]);
    else acc[i][j] = mfma<ELEM>(af[set][i], bfr[set][j], acc[i][j]);
  };
  // MFMA n of a K step.  NW = 4: in shells of max(i, j) (shell k holds
  // n = k^2 .. k^2 + 2k: (0, k) .. (k-1, k), then (k, 0) .. (k, k)), the
  // fragments of A row i and B column j being read in slot max(i, j) of the
  // step before; NW = 8: (0,0) (1,0) (0,1) (1,1) (2,0) (3,0) (2,1) (3,1), the
  // step before reading A0, B0, A1 in its first slot and B1, A2, A3 in its
  // second.  Either way the first MFMAs of a step need only the earliest
  // reads.
  auto mma_n = [&](int set, int n) {
    if constexpr (NW == 4 && MI == 4 && NI == 4) {
      const int k = n < 1 ? 0 : n < 4 ? 1 : n < 9 ? 2 : 3, r = n - k * k;
      if (r < k) mma(set, r, k);
      else mma(set, k, r - k);
    } else if constexpr (NW == 4) {
      // the same shells over an MI x NI grid (MI, NI in {2, 4})
      int c = 0, mi = 0, mj = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int r = 0; r < k; ++r)
          if (r < MI && k < NI) {
            if (c == n) mi = r, mj = k;
            ++c;
          }
#pragma unroll
        for (int r = 0; r <= k; ++r)
          if (k < MI && r < NI) {
            if (c == n) mi = k, mj = r;
            ++c;
          }
      }
      mma(set, mi, mj);
    } else {
      mma(set, 2 * (n >> 2) + (n & 1), (n >> 1) & 1);
    }
  };
  // the fragment reads of slot g (of MI * NI / 4 slots) of a K step
  auto slot_reads = [&](const unsigned char* S, int ks, int set, int g) {
    if constexpr (NW == 4 && MI == 4 && NI == 4) {
      read_a(S, ks, set, g);
      read_b(S, ks, set, g);
    } else if constexpr (NW == 4) {
      // slot 0: A0 B0 A1 B1 (the first four MFMAs' shells); slot 1 of a
      // 4 x 2 or 2 x 4 grid: the rest (A2 A3 or B2 B3)
      if (g == 0) {
        read_a(S, ks, set, 0);
        read_b(S, ks, set, 0);
        read_a(S, ks, set, 1);
        read_b(S, ks, set, 1);
      } else if constexpr (MI == 4) {
        read_a(S, ks, set, 2);
        read_a(S, ks, set, 3);
      } else {
        read_b(S, ks, set, 2);
        read_b(S, ks, set, 3);
      }
    } else if (g == 0) {
      read_a(S, ks, set, 0);
      read_b(S, ks, set, 0);
      read_a(S, ks, set, 1);
    } else {
      read_b(S, ks, set, 1);
      read_a(S, ks, set, 2);
      read_a(S, ks, set, 3);
    }
  };

  // The LDS reads need no wait before a barrier: those of the stage whose
  // buffer the next DMA overwrites were consumed by its MFMAs, and the
  // prefetched reads target a buffer no DMA touches until later.
#define XT_WAIT_VM(n) XTK_WAIT_VM(n)
  // prologue: stages 0 .. NS-2 in flight; 0 and 1 landed before B_0
#pragma unroll
  for (int q = 0; q < NS - 1; ++q)
    if (q < nk) dma(q, buf[q]);
  if (nk >= NS - 1) XT_WAIT_VM(PER * (NS - 3));
  else XT_WAIT_VM(0);
  asm volatile("s_barrier" ::: "memory");
  read_frags(buf[0], 0, 0);

  // A stage is 2 MI NI / 4 slots of four MFMAs (8 with four waves, 4 with
  // eight).  Slot g issues, in this order (sched_barrier fences keep the
  // compiler from moving anything across): MFMA, this wave's DMA instruction
  // g of stage s + NS - 1, MFMA, the slot's first fragment read(s), MFMA, the
  // rest, MFMA.  The first half of the slots runs K step 0 on fragment set 0
  // and reads set 1; the second half runs step 1 and reads the next stage's
  // set 0.  Spread out this way the DMA never queues more than one
  // instruction per wave ahead of the MFMAs; issued as a burst after the
  // barrier, it held every wave's issue (C3: ~330 cycles a stage).
  constexpr int SLOTS = MI * NI / 2, HALF = SLOTS / 2;
  // one DMA instruction per slot, two in the first slots of a tile smaller
  // than 256 x 256 (6 for 4 slots, 4 for 2)
  static_assert(PER >= SLOTS && PER <= 2 * SLOTS, "DMA instructions per slot");
  // `more` (a stage NS - 1 ahead exists) is std::true_type in the steady
  // state, so the DMA of each slot is issued with no test in front of it
  // (a test per instruction cost C3 ~70 scalar instructions a stage), and
  // a bool in the last stages.
  auto stage = [&](auto more_c, int s, unsigned char* S, const unsigned char* Snext, unsigned char* Sfree) {
    const bool more = more_c;
#pragma unroll
    for (int g = 0; g < SLOTS; ++g) {
      const int set = g < HALF ? 0 : 1, n0 = 4 * (g % HALF);
      __builtin_amdgcn_sched_barrier(0);
      mma_n(set, n0);
      __builtin_amdgcn_sched_barrier(0);
      if (more) {
        dma_one(s + NS - 1, Sfree, g);
        if (g + SLOTS < PER) dma_one(s + NS - 1, Sfree, g + SLOTS);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma_n(set, n0 + 1);
      __builtin_amdgcn_sched_barrier(0);
      // the last stage's reads of Snext fetch a buffer it never uses: kept
      // unconditional so that the waits for this step's fragments do not
      // cover them
      if (g < HALF) slot_reads(S, 1, 1, g);
      else slot_reads(Snext, 0, 0, g - HALF);
      __builtin_amdgcn_sched_barrier(0);
      mma_n(set, n0 + 2);
      __builtin_amdgcn_sched_barrier(0);
      mma_n(set, n0 + 3);
    }
    __builtin_amdgcn_sched_barrier(0);
    // B_{s+1}: this wave's DMA of stage s + 2 landed (stages s+3 .. s+NS-1
    // may stay in flight), its reads done
    if (more) XT_WAIT_VM(PER * (NS - 3));
    else XT_WAIT_VM(0);
    asm volatile("s_barrier" ::: "memory");
  };
  int s0 = 0;
  // steady state: every stage of the group has a stage NS - 1 ahead
  for (; s0 + 2 * NS - 2 < nk; s0 += NS) {
#pragma unroll
    for (int q = 0; q < NS; ++q)
      stage(std::true_type{}, s0 + q, buf[q], buf[(q + 1) % NS], buf[(q + NS - 1) % NS]);
  }
  for (; s0 < nk; s0 += NS) {
#pragma unroll
    for (int q = 0; q < NS; ++q)
      if (s0 + q < nk)
        stage(s0 + q + NS - 1 < nk, s0 + q, buf[q], buf[(q + 1) % NS], buf[(q + NS - 1) % NS]);
  }
#undef XT_WAIT_VM

  const bool hs = p.has_scale, hb = p.has_bias;
  if constexpr (OUT_I8) {
    // D^T = B^T x A^T per 32x32 tile: lane l holds output row m = l%32 of
    // tile i and register v output column 8*(v/4) + 4*(l/32) + v%4 of tile j,
    // so four consecutive columns pack into one 4-byte store.  Without a
    // scale or bias the factors are 1 and 0: x * 1 = x exactly, and x + 0
    // differs from x only for -0, which ftoi maps to 0 like +0.
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n0 = wn * WN + j * 32 + 8 * g + 4 * hi;
        float4v sv = {1.f, 1.f, 1.f, 1.f}, bv = {0.f, 0.f, 0.f, 0.f};
        if (hs) sv = *reinterpret_cast<const float4v*>(t.S + n0);
        if (hb) bv = *reinterpret_cast<const float4v*>(t.Bias + n0);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const long long off = t.c_off + (long long)(wm * WM + i * 32 + lrow) * p.ldc + n0;
          int q[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) q[e] = ftoi_i8_fast(scale_bias((float)acc[i][j][4 * g + e], sv[e], bv[e], true, true));
          // a plain store: the L2 merges the 8-byte pieces of a row into
          // whole lines (non-temporal stores of them measured 120 us on C6
          // against 78 us for the same GEMM with f32 results)
          *reinterpret_cast<unsigned*>(static_cast<signed char*>(p.c) + off) = pack_i8x4(q);
        }
      }
  } else {
    // D = A x B per 32x32 tile: lane l holds output column l%32 of tile j and
    // register v row 8*(v/4) + 4*(l/32) + v%4 of tile i; a half-wave writes
    // one whole 128-byte line per register.  EPI = false: no scale or bias,
    // so no instructions are spent on them.
    const int orow = hi * 4;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int n = wn * WN + j * 32 + lrow;
      const float sv = EPI && hs ? t.S[n] : 1.f, bv = EPI && hb ? t.Bias[n] : 0.f;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const long long off = t.c_off + (long long)(wm * WM + i * 32 + (v >> 2) * 8 + orow + (v & 3)) * p.ldc + n;
          const float x = (float)acc[i][j][v];
          float* const o = static_cast<float*>(p.c) + off;
          // K split (never with an epilogue): the ranges' partial sums meet
          // in the zero-filled output, in an order that varies
          if constexpr (KS) __hip_atomic_fetch_add(o, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else __builtin_nontemporal_store(EPI ? scale_bias(x, sv, bv, hs, hb) : x, o);
        }
    }
  }
}

TileOff to_off(const xt::TileAddr& a) { return TileOff{a.c0, a.sx, a.sy, a.sz}; }

bool offs_multiple(const xt::TileAddr& a, long long m) {
  return a.c0 % m == 0 && a.sx % m == 0 && a.sy % m == 0 && a.sz % m == 0;
}

long long axis_step(const xt::TileAddr& a, int axis) {
  return axis == 0 ? a.sx : axis == 1 ? a.sy : a.sz;
}

// How one workgroup tile of `w` elements covers Blocks of `t` elements along
// M (is_m) or N: split (sub > 1), exact, or fused over `factor` neighbouring
// Blocks along a grid axis whose next Block continues the same rows/columns.
struct Cover {
  bool ok = false;
  int sub = 1;
  int axis = -1;
  int factor = 1;
};

Cover cover_dim(const xt::Plan& p, long long w, bool is_m) {
  Cover c;
  const long long t = is_m ? p.a.rows : p.b.cols;
  if (t % w == 0) {
    c.ok = true;
    c.sub = static_cast<int>(t / w);
    return c;
  }
  if (w % t) return c;
  const int f = static_cast<int>(w / t);
  for (int ax = 0; ax < 3; ++ax) {
    if (p.grid[ax] % f) continue;
    // the epilogue rows follow B's columns
    const bool rows_fixed = (!p.gemm_scale || axis_step(p.scale.addr, ax) == 0) &&
                            (!p.gemm_bias || axis_step(p.bias.addr, ax) == 0);
    const bool rows_follow = (!p.gemm_scale || axis_step(p.scale.addr, ax) == t) &&
                             (!p.gemm_bias || axis_step(p.bias.addr, ax) == t);
    bool contiguous;
    if (is_m)
      contiguous = axis_step(p.c.addr, ax) == t * p.c.ld && axis_step(p.a.addr, ax) == t * p.a.ld &&
                   axis_step(p.b.addr, ax) == 0 && rows_fixed;
    else
      contiguous = axis_step(p.c.addr, ax) == t && axis_step(p.b.addr, ax) == t &&
                   axis_step(p.a.addr, ax) == 0 && rows_follow;
    if (contiguous) {
      c.ok = true;
      c.axis = ax;
      c.factor = f;
      return c;
    }
  }
  return c;
}

// Zero-fills rows x (4 cols4) floats at pitch ld (a kernel, not
// hipMemsetAsync, so that a captured graph replays it correctly).
__global__ __launch_bounds__(256) void gemm_zero_kernel(float* __restrict__ c, long long ld, int rows, int cols4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long r = i / cols4;
  if (r >= rows) return;
  const long long q = i - r * cols4;
  __builtin_nontemporal_store(float4v{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<float4v*>(c + r * ld) + q);
}

// The C tiles of all Blocks form one [M][N] region at c0 with pitch ld:
// along one grid axis the Blocks step A and C by TM rows (B fixed), along
// the other B and C by TN columns (A fixed).
bool c_region(const xt::Plan& p, long long& M, long long& N) {
  if (p.grid[2] != 1) return false;
  const long long TM = p.a.rows, TN = p.b.cols;
  for (int am = 0; am < 2; ++am) {
    const int an = 1 - am;
    const bool m_ok = p.grid[am] == 1 || (axis_step(p.a.addr, am) == TM * p.a.ld &&
                                          axis_step(p.c.addr, am) == TM * p.c.ld && axis_step(p.b.addr, am) == 0);
    const bool n_ok = p.grid[an] == 1 || (axis_step(p.b.addr, an) == TN && axis_step(p.c.addr, an) == TN &&
                                          axis_step(p.a.addr, an) == 0);
    if (m_ok && n_ok) {
      M = TM * p.grid[am];
      N = TN * p.grid[an];
      return true;
    }
  }
  return false;
}

// The DMA kernel at a tile smaller than 256 x 256 (four waves).
template <int ELEM, bool OUT_I8, int BMT, int BNT>
void launch_small_t(const GemmArgs& a, hipStream_t s) {
  const dim3 grid(a.nwg), block(256);
  if constexpr (OUT_I8)
    hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, true, true, 4, false, BMT, BNT>), grid, block, 0, s, a);
  else if (a.has_scale || a.has_bias)
    hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, false, true, 4, false, BMT, BNT>), grid, block, 0, s, a);
  else if (BMT == 128 && BNT == 128 && a.ksplit > 1)
    hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, false, false, 4, true, 128, 128>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, false, false, 4, false, BMT, BNT>), grid, block, 0, s, a);
}

template <int ELEM, bool OUT_I8>
void launch_t(int bm, int bn, const GemmArgs& a, hipStream_t s) {
  const dim3 grid(a.nwg), block(256);
  if (bm == 256 && bn == 256) {
    constexpr int NW = dma_waves<ELEM>();
    const dim3 dblock(64 * NW);
    if constexpr (OUT_I8)
      hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, true, true, NW>), grid, dblock, 0, s, a);
    else if (a.has_scale || a.has_bias)
      hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, false, true, NW>), grid, dblock, 0, s, a);
    else if (a.ksplit > 1)
      hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, false, false, NW, true>), grid, dblock, 0, s, a);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<ELEM, kDmaStages, false, false, NW>), grid, dblock, 0, s, a);
  } else if (bm == 256) {
    launch_small_t<ELEM, OUT_I8, 256, 128>(a, s);
  } else if (bm == 128 && bn == 256) {
    launch_small_t<ELEM, OUT_I8, 128, 256>(a, s);
  } else if (bm == 128) {
    launch_small_t<ELEM, OUT_I8, 128, 128>(a, s);
  } else {
    hipLaunchKernelGGL((gemm_kernel<ELEM, 64, 64, OUT_I8>), grid, block, 0, s, a);
  }
}

}  // namespace

hipError_t launch_gemm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  const bool i8 = p.a.elem == xt::Elem::I8;
  const long long es = i8 ? 1 : 2;
  GemmArgs a;
  a.a = static_cast<const unsigned char*>(bufs[p.a.arg]);
  a.b = static_cast<const unsigned char*>(bufs[p.b.arg]);
  a.c = bufs[p.c.arg];
  a.scale = p.gemm_scale ? static_cast<const float*>(bufs[p.scale.arg]) : nullptr;
  a.bias = p.gemm_bias ? static_cast<const float*>(bufs[p.bias.arg]) : nullptr;
  a.has_scale = p.gemm_scale;
  a.has_bias = p.gemm_bias;
  a.ta = to_off(p.a.addr);
  a.tb = to_off(p.b.addr);
  a.tc = to_off(p.c.addr);
  a.ts = p.gemm_scale ? to_off(p.scale.addr) : TileOff{0, 0, 0, 0};
  a.tbias = p.gemm_bias ? to_off(p.bias.addr) : TileOff{0, 0, 0, 0};
  a.lda = p.a.ld;
  a.ldb = p.b.ld;
  a.ldc = p.c.ld;
  const long long kbytes = p.gemm_k * es;
  const long long TM = p.a.rows, TN = p.b.cols;
  if (kbytes % SLICE || TM % 64 || TN % 64) {
    why = i8 ? "i8 matmul tile must have M, N multiples of 64 and K a multiple of 128"
             : "matmul tile must have M, N, K multiples of 64";
    return hipErrorInvalidValue;
  }
  a.nk = static_cast<int>(kbytes / SLICE);
  for (const void* ptr : {bufs[p.a.arg], bufs[p.b.arg], bufs[p.c.arg]})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) {
      why = "matmul buffers must be 16-byte aligned";
      return hipErrorInvalidValue;
    }
  if ((a.lda * es) % 16 || (a.ldb * es) % 16 || !offs_multiple(p.a.addr, 16 / es) ||
      !offs_multiple(p.b.addr, 16 / es)) {
    why = "matmul input tiles must start on 16-byte boundaries";
    return hipErrorInvalidValue;
  }
  // the staging addresses each workgroup's A and B panels with 32-bit offsets
  if (TM * a.lda * es >= (1LL << 32) || p.gemm_k * a.ldb * es >= (1LL << 32)) {
    why = "matmul A and B tile panels must each span less than 4 GiB";
    return hipErrorInvalidValue;
  }
  if (p.c.ld % 4 || !offs_multiple(p.c.addr, 4)) {
    why = "matmul output tiles must start on 4-element boundaries";
    return hipErrorInvalidValue;
  }
  for (int e = 0; e < 2; ++e) {
    const bool on = e == 0 ? p.gemm_scale : p.gemm_bias;
    const xt::Access2D& v = e == 0 ? p.scale : p.bias;
    if (on && (reinterpret_cast<uintptr_t>(bufs[v.arg]) % 16 || !offs_multiple(v.addr, 4))) {
      why = "matmul scale / bias tiles must start on 16-byte boundaries";
      return hipErrorInvalidValue;
    }
  }
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  const bool out_i8 = p.c.elem == xt::Elem::I8;
  long long M = 0, N = 0;
  float* const cbase = static_cast<float*>(bufs[p.c.arg]) + p.c.addr.c0;
  const bool can_split = ksplit_allowed() && !i8 && !out_i8 && !p.gemm_scale && !p.gemm_bias && c_region(p, M, N) && N % 4 == 0 &&
                         p.c.ld % 4 == 0 && reinterpret_cast<uintptr_t>(cbase) % 16 == 0 && M < (1LL << 31);
  // Workgroup tile, all on the DMA kernel: 256 x 256 when the Blocks map onto
  // it and its tiles fill the CUs, or are few enough for the K split below;
  // else the first of 256 x 128, 128 x 256, 128 x 128 whose tiles fill the
  // CUs, else the one with the most tiles (a 2048^3 f16 GEMM: 64 tiles of
  // 256 x 256, 256 of 128 x 128); 64 x 64 (register-staged) when none maps.
  struct Cand {
    int bm = 0, bn = 0;
    Cover cm, cn;
    long long tiles = 0;
  };
  auto try_tile = [&](int bmv, int bnv, Cand& c) {
    c.bm = bmv;
    c.bn = bnv;
    c.cm = cover_dim(p, bmv, true);
    c.cn = cover_dim(p, bnv, false);
    if (!c.cm.ok || !c.cn.ok || (c.cm.axis >= 0 && c.cm.axis == c.cn.axis)) return false;
    long long g[3] = {p.grid[0], p.grid[1], p.grid[2]};
    if (c.cm.axis >= 0) g[c.cm.axis] /= c.cm.factor;
    if (c.cn.axis >= 0) g[c.cn.axis] /= c.cn.factor;
    c.tiles = g[0] * g[1] * g[2] * c.cm.sub * c.cn.sub;
    return true;
  };
  Cand pick, c256, c128;
  const bool has256 = try_tile(256, 256, c256);
  // A GEMM of at most CUs / 8 tiles of 256 x 256 that can split K takes 128
  // x 128 tiles with the split (1024 x 1024 x 4096 f16: 42.3 us on 16 tiles
  // of 256 x 256 in 8 K ranges, 28.2 on 64 of 128 x 128 in 4; hipBLASLt 25.1)
  const bool tiny = can_split && has256 && c256.tiles * 8 <= cus;
  if (tiny && try_tile(128, 128, c128)) {
    pick = c128;
  } else if (has256 && (c256.tiles >= cus || tiny)) {
    pick = c256;
  } else {
    Cand most = has256 ? c256 : Cand{};
    bool found = false;
    const int shapes[3][2] = {{256, 128}, {128, 256}, {128, 128}};
    for (const auto& sh : shapes) {
      Cand c;
      if (!try_tile(sh[0], sh[1], c)) continue;
      if (c.tiles >= cus) {
        pick = c;
        found = true;
        break;
      }
      if (c.tiles > most.tiles) most = c;
    }
    if (!found) pick = most;
    if (pick.bm == 0 && try_tile(64, 64, pick) == false) {
      why = "matmul Blocks cannot be mapped onto 64x64 workgroup tiles";
      return hipErrorInvalidValue;
    }
  }
  const int bm = pick.bm, bn = pick.bn;
  const Cover cm = pick.cm, cn = pick.cn;
  a.mul[0] = a.mul[1] = a.mul[2] = 1;
  int vg[3] = {p.grid[0], p.grid[1], p.grid[2]};
  if (cm.axis >= 0) {
    a.mul[cm.axis] = cm.factor;
    vg[cm.axis] /= cm.factor;
  }
  if (cn.axis >= 0) {
    a.mul[cn.axis] = cn.factor;
    vg[cn.axis] /= cn.factor;
  }
  a.vgx = vg[0];
  a.vgy = vg[1];
  a.sub_m = cm.sub;
  a.sub_n = cn.sub;
  long long nwg = (long long)vg[0] * vg[1] * vg[2] * a.sub_m * a.sub_n;
  if (!grid_fits(nwg, 256)) {
    why = "matmul grid of " + std::to_string(nwg) + " workgroup tiles exceeds one launch";
    return hipErrorInvalidValue;
  }
  a.nwg = static_cast<int>(nwg);
  a.group = kTileGroup;
  a.tiles = a.nwg;
  a.ksplit = 1;
  a.kstages = a.nk * 2;
  // K split: when the 256 x 256 tiles fill at most an eighth of the CUs, f32
  // results of f16 / bf16 products without an epilogue split K into ranges
  // of at least 16 stages (spread evenly: lengths differ by at most one),
  // one workgroup each, adding their partial sums atomically into the
  // zero-filled output (the f32 addition order, and so the last bits, vary
  // between runs; i8 sums stay exact and whole).  XTILE_AMD_KSPLIT=0 turns
  // the split off (run-to-run reproducible results).
  // Measured (f16, 30 launches): 1024 x 1024 x 4096 (16 tiles) 79.2 us whole,
  // 42.8 in 8 ranges; 2048^3 (64 tiles) 47.3 whole, 71.4 in 4; 1024 x 8192 x
  // 8192 (128 tiles) 155.9 whole, 164.4 in 2.
  if (can_split && ((bm == 256 && bn == 256 && nwg * 8 <= cus) || (tiny && bm == 128 && bn == 128 && nwg * 2 <= cus))) {
    const long long nk2 = a.nk * 2LL;
    const long long ks = std::min<long long>(cus / nwg, nk2 / 16);
    if (ks > 1) {
      a.kstages = (int)(nk2 / ks);
      a.ksplit = (int)ks;
      a.nwg = (int)(nwg * ks);
      const long long n4 = M * (N / 4);
      hipLaunchKernelGGL(gemm_zero_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, cbase, p.c.ld,
                         (int)M, (int)(N / 4));
    }
  }
  switch (p.a.elem) {
    case xt::Elem::I8: out_i8 ? launch_t<kI8, true>(bm, bn, a, s) : launch_t<kI8, false>(bm, bn, a, s); break;
    case xt::Elem::BF16:
      out_i8 ? launch_t<kBF16, true>(bm, bn, a, s) : launch_t<kBF16, false>(bm, bn, a, s);
      break;
    default: out_i8 ? launch_t<kF16, true>(bm, bn, a, s) : launch_t<kF16, false>(bm, bn, a, s); break;
  }
  return hipGetLastError();
}

}  // namespace xtk
