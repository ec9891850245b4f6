// Tile matmul C = A @ B with f16 or bf16 inputs and f32 accumulation on the
// gfx950 matrix cores.
//
// Semantics: xt.matmul over one Block's tiles, the whole K extent of the
// tile (kernels/matmul.py:11-16,35; lib/xt/XTOps.cpp:218-253 with the
// narrow-float extension).
//
// Workgroup tiles are decoupled from xt Block tiles.  A Block's TM x TN output
// tile is split into (TM/BM) x (TN/BN) workgroup tiles when it is larger, and
// neighbouring Blocks are fused into one workgroup tile when it is smaller and
// the planner's affine addresses show them to be contiguous (the next Block
// along one grid axis continues the same A rows / B columns / C tile).  Blocks
// are independent (README.md:85-89), so both are pure scheduling choices.
//
// Two kernel families:
//   gemm256_kernel  BM x BN x BK = 256 x 256 x 64, 4 waves of 128 x 128 using
//                   v_mfma_f32_32x32x16_{f16,bf16}; one workgroup per CU
//                   (128 KB of LDS), 256 accumulators per lane in AGPRs.
//                   Per 16-wide K step a wave reads 8 LDS fragments for 16
//                   MFMAs, half the LDS bytes per FLOP of a 64 x 64 wave tile.
//   gemm_kernel     BM, BN in {64, 128} x BK = 64, 4 waves of (BM/2) x (BN/2)
//                   using v_mfma_f32_16x16x32; for tiles the 256 family cannot
//                   cover.
// Common data path:
//   * A slices (K-contiguous rows) go global -> VGPR -> LDS with 16-byte
//     accesses.
//   * B slices are N-contiguous in memory but MFMA wants K-contiguous lanes, so
//     each thread loads a 4(k) x 8(n) sub-block, transposes it in registers and
//     writes eight 8-byte K-runs into an N-major LDS tile.
//   * Both LDS tiles are double buffered: the next slice's global loads are in
//     flight while the current slice feeds the MFMAs; one barrier per slice.
//   * LDS rows are padded by 8 elements (16 bytes): every ds_read_b128 of a
//     fragment and every LDS store above runs at the bank-conflict-free rate.
//   * Workgroups are dispatched round-robin over the 8 XCDs; the linear id is
//     remapped so that each XCD receives a contiguous run of tiles, and tiles
//     are ordered in groups of GROUP tile columns so that concurrently resident
//     workgroups share A and B panels in their XCD's L2.
#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr int BK = 64;
constexpr int PAD = 8;
constexpr int LDK = BK + PAD;  // LDS row pitch in 16-bit elements

typedef float float16v __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const unsigned short* a;
  const unsigned short* b;
  float* c;
  TileOff ta, tb, tc;
  long long lda, ldb, ldc;
  int K;
  int vgx, vgy;       // virtual grid (fused axes divided by their factor)
  int mul[3];         // block id = virtual id * mul (fused axes)
  int sub_m, sub_n;   // workgroup tiles per (fused) Block along M and N
  int nwg;
  int group;
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

template <bool BF16>
__device__ __forceinline__ float16v mfma32(short8 a, short8 b, float16v c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Workgroup -> (tile origin pointers).  Contiguous runs per XCD, then
// GROUP-wide column groups over the virtual grid.
struct TilePtrs {
  const unsigned short* A;
  const unsigned short* B;
  float* C;
};

template <int BM, int BN>
__device__ __forceinline__ TilePtrs gemm_tile_of(const GemmArgs& p) {
  int L = blockIdx.x;
  if ((p.nwg & 7) == 0) L = (L & 7) * (p.nwg >> 3) + (L >> 3);
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
  t.A = p.a + p.ta.at(x, y, z) + (long long)sm * BM * p.lda;
  t.B = p.b + p.tb.at(x, y, z) + (long long)sn * BN;
  t.C = p.c + p.tc.at(x, y, z) + (long long)sm * BM * p.ldc + (long long)sn * BN;
  return t;
}

// Global -> VGPR staging of one BK slice (A rows, B 4x8 sub-blocks) and the
// VGPR -> LDS stores with the B transpose.
template <int BM, int BN>
struct Stager {
  static constexpr int A_VECS = BM * BK / 8 / 256;  // 16-byte vectors per thread
  static constexpr int B_SUBS = (BK / 4) * (BN / 8);
  static constexpr int B_ITERS = (B_SUBS + 255) / 256;
  uint4v ra[A_VECS];
  uint4v rb[B_ITERS][4];

  __device__ __forceinline__ void load(const unsigned short* A, const unsigned short* B,
                                       long long lda, long long ldb, int kt, int tid) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      ra[i] = *reinterpret_cast<const uint4v*>(A + (long long)row * lda + kt * BK + cv * 8);
    }
#pragma unroll
    for (int it = 0; it < B_ITERS; ++it) {
      const int sb = tid + it * 256;
      if (B_SUBS % 256 == 0 || sb < B_SUBS) {
        const int kb = sb & 15, nb = sb >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          rb[it][i] = *reinterpret_cast<const uint4v*>(B + (long long)(kt * BK + kb * 4 + i) * ldb + nb * 8);
      }
    }
  }

  __device__ __forceinline__ void store(unsigned short (*As)[LDK], unsigned short (*Bs)[LDK],
                                        int tid) const {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      *reinterpret_cast<uint4v*>(&As[row][cv * 8]) = ra[i];
    }
#pragma unroll
    for (int it = 0; it < B_ITERS; ++it) {
      const int sb = tid + it * 256;
      if (B_SUBS % 256 == 0 || sb < B_SUBS) {
        const int kb = sb & 15, nb = sb >> 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // columns n = 2j and 2j+1 of the 4 loaded rows
          const unsigned int d0 = rb[it][0][j], d1 = rb[it][1][j];
          const unsigned int d2 = rb[it][2][j], d3 = rb[it][3][j];
          uint2v even, odd;
          even.x = (d0 & 0xFFFFu) | (d1 << 16);
          even.y = (d2 & 0xFFFFu) | (d3 << 16);
          odd.x = (d0 >> 16) | (d1 & 0xFFFF0000u);
          odd.y = (d2 >> 16) | (d3 & 0xFFFF0000u);
          *reinterpret_cast<uint2v*>(&Bs[nb * 8 + 2 * j][kb * 4]) = even;
          *reinterpret_cast<uint2v*>(&Bs[nb * 8 + 2 * j + 1][kb * 4]) = odd;
        }
      }
    }
  }
};

// Stager of the 256 family.  LDS tiles are unpadded [rows][64] arrays whose
// 16-byte chunks are XOR-swizzled: chunk c of row r lives at c ^ swz(r) with
// swz(r) = (r ^ r >> 3) & 7.  Eight consecutive rows then spread one chunk
// index over all eight chunk positions (fragment reads), and rows 8 apart get
// different positions too (transposed B stores): every access below runs at
// the bank-conflict-free rate.  B is staged as 8(k) x 8(n) sub-blocks: a
// half-wave reads 512 contiguous bytes of one B row per instruction.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

struct Stager256 {
  static constexpr int BM = 256, BN = 256;
  uint4v ra[BM * BK / 8 / 256];  // 8 row chunks of A
  uint4v rb[8];                  // one 8(k) x 8(n) sub-block of B

  __device__ __forceinline__ void load(const unsigned short* A, const unsigned short* B,
                                       long long lda, long long ldb, int kt, int tid) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      ra[i] = *reinterpret_cast<const uint4v*>(A + (long long)row * lda + kt * BK + cv * 8);
    }
    const int nb = tid & 31, kb = tid >> 5;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      rb[i] = *reinterpret_cast<const uint4v*>(B + (long long)(kt * BK + kb * 8 + i) * ldb + nb * 8);
  }

  __device__ __forceinline__ void store(unsigned short (*As)[BK], unsigned short (*Bs)[BK],
                                        int tid) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      *reinterpret_cast<uint4v*>(&As[row][(cv ^ swz(row)) * 8]) = ra[i];
    }
    const int nb = tid & 31, kb = tid >> 5;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // columns n = 2j (low halves) and 2j+1 (high halves) of the 8 loaded rows
      uint4v even, odd;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned int lo = rb[2 * q][j], hi = rb[2 * q + 1][j];
        even[q] = (lo & 0xFFFFu) | (hi << 16);
        odd[q] = (lo >> 16) | (hi & 0xFFFF0000u);
      }
      const int r0 = nb * 8 + 2 * j, r1 = r0 + 1;
      *reinterpret_cast<uint4v*>(&Bs[r0][(kb ^ swz(r0)) * 8]) = even;
      *reinterpret_cast<uint4v*>(&Bs[r1][(kb ^ swz(r1)) * 8]) = odd;
    }
  }
};

// --- 256 x 256 family ---------------------------------------------------------

template <bool BF16>
__global__ __launch_bounds__(256, 1) void gemm256_kernel(GemmArgs p) {
  constexpr int BM = 256, BN = 256;
  constexpr int WM = 128, WN = 128;  // 2 x 2 waves
  constexpr int MI = WM / 32, NI = WN / 32;
  __shared__ __attribute__((aligned(16))) unsigned short As[2][BM][BK];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[2][BN][BK];

  const TilePtrs t = gemm_tile_of<BM, BN>(p);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Two register staging sets keep two K slices in flight: slice kt+2 is
  // requested while slice kt feeds the MFMAs and slice kt+1 (requested one
  // iteration earlier) is moved to LDS.
  Stager256 st0, st1;
  float16v acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = p.K / BK;  // >= 1
  st0.load(t.A, t.B, p.lda, p.ldb, 0, tid);
  st1.load(t.A, t.B, p.lda, p.ldb, min(1, nk - 1), tid);
  st0.store(As[0], Bs[0], tid);
  __syncthreads();
  const int lrow = lane & 31;
  // Fragments of K step ks+1 are read from LDS while the 16 MFMAs of step ks
  // run (two register sets), so only the first read of each slice is exposed.
  short8 af[2][MI], bfr[2][NI];
  // chunk index of this lane's 8 K values in step ks: 2*ks + lane/32
  auto read_frags = [&](int buf, int ks, int set) {
    const int c = ks * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int r = wm * WM + i * 32 + lrow;
      af[set][i] = *reinterpret_cast<const short8*>(&As[buf][r][(c ^ swz(r)) * 8]);
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int r = wn * WN + j * 32 + lrow;
      bfr[set][j] = *reinterpret_cast<const short8*>(&Bs[buf][r][(c ^ swz(r)) * 8]);
    }
  };
  // One K slice: compute from LDS[cur], request slice kt+2 into `next2`, move
  // slice kt+1 from `next1` into LDS[cur^1].  Branch-free: slice indices are
  // clamped to the last slice, whose repeated copies land in the idle buffer.
  auto slice = [&](int kt, Stager256& next2, const Stager256& next1) {
    const int cur = kt & 1;
    read_frags(cur, 0, 0);
    next2.load(t.A, t.B, p.lda, p.ldb, min(kt + 2, nk - 1), tid);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      if (ks + 1 < BK / 16) read_frags(cur, ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = mfma32<BF16>(af[ks & 1][i], bfr[ks & 1][j], acc[i][j]);
    }
    next1.store(As[cur ^ 1], Bs[cur ^ 1], tid);
    // Issue order for the slice: the first 8 fragment reads, then every MFMA
    // followed by at most one fragment read, one global load, one LDS store
    // and two VALU ops, so the global loads, the B transposes and the LDS
    // stores of the next slices issue while the MFMA pipe stays busy.
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int g = 0; g < MI * NI * (BK / 16); ++g) {
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

  // D layout of a 32x32 f32 MFMA tile: lane l, register v holds
  // row 8*(v/4) + 4*(l/32) + v%4, column l%32.
  const int orow = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        t.C[(long long)(wm * WM + i * 32 + (v >> 2) * 8 + orow + (v & 3)) * p.ldc + wn * WN + j * 32 +
            lrow] = acc[i][j][v];
}

// --- 64/128 family --------------------------------------------------------------

template <int BM, int BN, bool BF16>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / 2, WN = BN / 2;   // 2 x 2 waves
  constexpr int MI = WM / 16, NI = WN / 16; // 16x16 MFMA tiles per wave
  __shared__ __attribute__((aligned(16))) unsigned short As[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[2][BN][LDK];

  const TilePtrs t = gemm_tile_of<BM, BN>(p);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  Stager<BM, BN> st;
  float4v acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / BK;
  st.load(t.A, t.B, p.lda, p.ldb, 0, tid);
  st.store(As[0], Bs[0], tid);
  __syncthreads();
  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) st.load(t.A, t.B, p.lda, p.ldb, kt + 1, tid);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      short8 af[MI], bfr[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        af[i] = *reinterpret_cast<const short8*>(&As[cur][wm * WM + i * 16 + lrow][ks * 32 + lk]);
#pragma unroll
      for (int j = 0; j < NI; ++j)
        bfr[j] = *reinterpret_cast<const short8*>(&Bs[cur][wn * WN + j * 16 + lrow][ks * 32 + lk]);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = mfma16<BF16>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) st.store(As[cur ^ 1], Bs[cur ^ 1], tid);
    __syncthreads();
  }

  // D layout of a 16x16 f32 MFMA tile: lane l holds rows 4*(l/16)+v, column l%16.
  const int orow = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        t.C[(long long)(wm * WM + i * 16 + orow + v) * p.ldc + wn * WN + j * 16 + lrow] = acc[i][j][v];
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
    bool contiguous;
    if (is_m)
      contiguous = axis_step(p.c.addr, ax) == t * p.c.ld && axis_step(p.a.addr, ax) == t * p.a.ld &&
                   axis_step(p.b.addr, ax) == 0;
    else
      contiguous = axis_step(p.c.addr, ax) == t && axis_step(p.b.addr, ax) == t &&
                   axis_step(p.a.addr, ax) == 0;
    if (contiguous) {
      c.ok = true;
      c.axis = ax;
      c.factor = f;
      return c;
    }
  }
  return c;
}

}  // namespace

hipError_t launch_gemm(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  GemmArgs a;
  a.a = static_cast<const unsigned short*>(bufs[p.a.arg]);
  a.b = static_cast<const unsigned short*>(bufs[p.b.arg]);
  a.c = static_cast<float*>(bufs[p.c.arg]);
  a.ta = to_off(p.a.addr);
  a.tb = to_off(p.b.addr);
  a.tc = to_off(p.c.addr);
  a.lda = p.a.ld;
  a.ldb = p.b.ld;
  a.ldc = p.c.ld;
  a.K = static_cast<int>(p.gemm_k);
  const long long TM = p.a.rows, TN = p.b.cols;
  if (a.K % BK || TM % 64 || TN % 64) {
    why = "matmul tile must have M, N, K multiples of 64";
    return hipErrorInvalidValue;
  }
  for (const void* ptr : {bufs[p.a.arg], bufs[p.b.arg], bufs[p.c.arg]})
    if (reinterpret_cast<uintptr_t>(ptr) % 16) {
      why = "matmul buffers must be 16-byte aligned";
      return hipErrorInvalidValue;
    }
  if (a.lda % 8 || a.ldb % 8 || !offs_multiple(p.a.addr, 8) || !offs_multiple(p.b.addr, 8)) {
    why = "matmul input tiles must start on 16-byte boundaries";
    return hipErrorInvalidValue;
  }
  // Prefer 256 x 256 workgroup tiles when the Blocks can be split or fused into them.
  int bm = 256, bn = 256;
  Cover cm = cover_dim(p, 256, true), cn = cover_dim(p, 256, false);
  if (!cm.ok || !cn.ok || (cm.axis >= 0 && cm.axis == cn.axis)) {
    bm = TM % 128 == 0 ? 128 : 64;
    bn = TN % 128 == 0 ? 128 : 64;
    cm = cover_dim(p, bm, true);
    cn = cover_dim(p, bn, false);
  }
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
  if (nwg > 0x7fffffff) {
    why = "matmul grid too large";
    return hipErrorInvalidValue;
  }
  a.nwg = static_cast<int>(nwg);
  a.group = 8;
  const bool bf16 = p.a.elem == xt::Elem::BF16;
  dim3 grid(a.nwg), block(256);
#define XT_GEMM(BMV, BNV, BFV) hipLaunchKernelGGL((gemm_kernel<BMV, BNV, BFV>), grid, block, 0, s, a)
  if (bm == 256) {
    if (bf16) hipLaunchKernelGGL((gemm256_kernel<true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gemm256_kernel<false>), grid, block, 0, s, a);
  } else if (bm == 128 && bn == 128) {
    if (bf16) XT_GEMM(128, 128, true); else XT_GEMM(128, 128, false);
  } else if (bm == 128) {
    if (bf16) XT_GEMM(128, 64, true); else XT_GEMM(128, 64, false);
  } else if (bn == 128) {
    if (bf16) XT_GEMM(64, 128, true); else XT_GEMM(64, 128, false);
  } else {
    if (bf16) XT_GEMM(64, 64, true); else XT_GEMM(64, 64, false);
  }
#undef XT_GEMM
  return hipGetLastError();
}

}  // namespace xtk
