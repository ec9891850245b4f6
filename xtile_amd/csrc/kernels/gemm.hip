// Tile matmul C = A @ B with f16 or bf16 inputs and f32 accumulation on the
// gfx950 matrix cores (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Semantics: xt.matmul over one Block's tiles, the whole K extent of the
// tile (kernels/matmul.py:11-16,35; lib/xt/XTOps.cpp:218-253 with the
// narrow-float extension).  Each xt Block's TM x TN output tile is covered by
// (TM/BM) x (TN/BN) workgroups; every workgroup streams K in BK-wide slices.
//
// Data path per workgroup (BM x BN x BK = 128 x 128 x 64, 256 threads):
//   * A slices (K-contiguous rows) go global -> VGPR -> LDS with 16-byte
//     accesses.
//   * B slices are N-contiguous in memory but MFMA wants K-contiguous lanes, so
//     each thread loads a 4(k) x 8(n) sub-block, transposes it in registers and
//     writes eight 8-byte K-runs into an N-major LDS tile.
//   * Both LDS tiles are double buffered: the next slice's global loads are in
//     flight while the current slice feeds the MFMAs; one barrier per slice.
//   * Rows are padded by 8 elements (16 bytes) so the 16-lane groups of a
//     ds_read_b128 fall on distinct banks.
//   * Workgroups are dispatched round-robin over the 8 XCDs; the linear id is
//     remapped so that each XCD receives a contiguous run of tiles, and tiles
//     are ordered in groups of GROUP block columns so that concurrently
//     resident workgroups share A and B panels in their XCD's L2.
#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

constexpr int BK = 64;
constexpr int PAD = 8;
constexpr int LDK = BK + PAD;  // LDS row pitch in 16-bit elements

struct GemmArgs {
  const unsigned short* a;
  const unsigned short* b;
  float* c;
  TileOff ta, tb, tc;
  long long lda, ldb, ldc;
  int K;
  int gx, gy;
  int sub_m, sub_n;  // workgroup tiles per xt Block along M and N
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

// Block order: contiguous runs per XCD, then GROUP-wide column groups.
__device__ __forceinline__ void gemm_tile_of(const GemmArgs& p, int& x, int& y, int& z, int& sm,
                                             int& sn) {
  int L = blockIdx.x;
  if ((p.nwg & 7) == 0) L = (L & 7) * (p.nwg >> 3) + (L >> 3);
  const int subs = p.sub_m * p.sub_n;
  const int s = L % subs;
  int blk = L / subs;
  sm = s / p.sub_n;
  sn = s - sm * p.sub_n;
  const int per_plane = p.gx * p.gy;
  z = blk / per_plane;
  blk -= z * per_plane;
  const int per_group = p.group * p.gy;
  const int gid = blk / per_group;
  const int first = gid * p.group;
  const int gsize = min(p.group, p.gx - first);
  const int r = blk - gid * per_group;
  x = first + r % gsize;
  y = r / gsize;
}

template <int BM, int BN, bool BF16>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / 2, WN = BN / 2;   // 2 x 2 waves
  constexpr int MI = WM / 16, NI = WN / 16; // 16x16 MFMA tiles per wave
  constexpr int A_VECS = BM * BK / 8 / 256; // 16-byte vectors per thread
  constexpr int B_SUBS = (BK / 4) * (BN / 8);
  constexpr int B_ITERS = (B_SUBS + 255) / 256;
  __shared__ __attribute__((aligned(16))) unsigned short As[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[2][BN][LDK];

  int x, y, z, sm, sn;
  gemm_tile_of(p, x, y, z, sm, sn);
  const unsigned short* A = p.a + p.ta.at(x, y, z) + (long long)sm * BM * p.lda;
  const unsigned short* B = p.b + p.tb.at(x, y, z) + (long long)sn * BN;
  float* C = p.c + p.tc.at(x, y, z) + (long long)sm * BM * p.ldc + (long long)sn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  uint4v ra[A_VECS];
  uint4v rb[B_ITERS][4];

  auto load_slice = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      ra[i] = *reinterpret_cast<const uint4v*>(A + (long long)row * p.lda + kt * BK + cv * 8);
    }
#pragma unroll
    for (int it = 0; it < B_ITERS; ++it) {
      const int sb = tid + it * 256;
      if (sb < B_SUBS) {
        const int kb = sb & 15, nb = sb >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          rb[it][i] = *reinterpret_cast<const uint4v*>(
              B + (long long)(kt * BK + kb * 4 + i) * p.ldb + nb * 8);
      }
    }
  };
  auto store_slice = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      const int v = tid + i * 256;
      const int row = v >> 3, cv = v & 7;
      *reinterpret_cast<uint4v*>(&As[buf][row][cv * 8]) = ra[i];
    }
#pragma unroll
    for (int it = 0; it < B_ITERS; ++it) {
      const int sb = tid + it * 256;
      if (sb < B_SUBS) {
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
          *reinterpret_cast<uint2v*>(&Bs[buf][nb * 8 + 2 * j][kb * 4]) = even;
          *reinterpret_cast<uint2v*>(&Bs[buf][nb * 8 + 2 * j + 1][kb * 4]) = odd;
        }
      }
    }
  };

  float4v acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / BK;
  load_slice(0);
  store_slice(0);
  __syncthreads();
  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_slice(kt + 1);
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
    if (kt + 1 < nk) store_slice(cur ^ 1);
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
        C[(long long)(wm * WM + i * 16 + orow + v) * p.ldc + wn * WN + j * 16 + lrow] = acc[i][j][v];
}

TileOff to_off(const xt::TileAddr& a) { return TileOff{a.c0, a.sx, a.sy, a.sz}; }

bool offs_multiple(const xt::TileAddr& a, long long m) {
  return a.c0 % m == 0 && a.sx % m == 0 && a.sy % m == 0 && a.sz % m == 0;
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
  a.gx = p.grid[0];
  a.gy = p.grid[1];
  const long long TM = p.a.rows, TN = p.b.cols;
  int bm = TM % 128 == 0 ? 128 : 64;
  int bn = TN % 128 == 0 ? 128 : 64;
  if (TM % bm || TN % bn || a.K % BK) {
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
  a.sub_m = static_cast<int>(TM / bm);
  a.sub_n = static_cast<int>(TN / bn);
  long long nwg = (long long)p.grid[0] * p.grid[1] * p.grid[2] * a.sub_m * a.sub_n;
  if (nwg > 0x7fffffff) {
    why = "matmul grid too large";
    return hipErrorInvalidValue;
  }
  a.nwg = static_cast<int>(nwg);
  a.group = 8;
  const bool bf16 = p.a.elem == xt::Elem::BF16;
  dim3 grid(a.nwg), block(256);
#define XT_GEMM(BMV, BNV, BFV) hipLaunchKernelGGL((gemm_kernel<BMV, BNV, BFV>), grid, block, 0, s, a)
  if (bm == 128 && bn == 128) {
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
