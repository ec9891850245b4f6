// Bandwidth-bound tile programs: elementwise binary ops and row softmax.
//
// One xt Block is one workgroup of 256 threads (4 wave64s).  Tiles are read
// and written with 128-bit global accesses whenever every row start is
// 16-byte aligned; consecutive lanes touch consecutive 16-byte chunks so each
// wave instruction covers whole 64-byte segments.
//
// Semantics follow the reference DSL: add/sub/mul are plain IEEE f32 ops
// (xtile/dsl.py:321-325,351-352); softmax is x - max(x), exp, sum, then
// multiply by reciprocal(sum) exactly as `x / r` is traced
// (xtile/dsl.py:354-357, kernels/softmax.py:13-18).  exp is exp_fast
// (common.h: relative error below 5.3e-6 for normal results, against the
// 1e-5 relative bar of the f32 softmax), and full-wave reductions use DPP
// (wave_reduce); together they took C2 from 43.0 to 41.9 us a launch.
#include "common.h"
#include "launch.h"

namespace xtk {
namespace {

struct EwArgs {
  const float* a;
  const float* b;
  float* c;
  TileOff ta, tb, tc;
  long long lda, ldb, ldc;
  int rows, cols;
  BlockDecode grid;  // y fastest when that makes neighbouring workgroups neighbours in memory
  int cv_shift;      // log2(cols / VW) when that is a power of two, else -1
};

template <int OP>
__device__ __forceinline__ float ew_apply(float x, float y) {
  if constexpr (OP == 0) return x + y;
  else if constexpr (OP == 1) return x - y;
  else return x * y;
}

// Streaming accesses: tiles are read and written exactly once per launch, so
// loads and stores are non-temporal (they do not displace reusable lines).
template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void st_nt(T v, T* p) { __builtin_nontemporal_store(v, p); }

// Each thread handles U vectors per step; U is the smallest of 1, 2, 4 that
// covers the tile in one step (4 when it takes several).  All U loads are
// issued before any is consumed; indices past the end of the tile (only in a
// tile's last step) are clamped to element 0 and their results discarded, so a
// step costs one memory round trip, not U.  POW2: the row length in vectors is
// a power of two and row/column come from a shift and a mask.
template <int OP, int VW, int U, bool POW2>
__global__ __launch_bounds__(256) void ew_binary_kernel(EwArgs p) {
  int x, y, z;
  p.grid(blockIdx.x, x, y, z);
  const float* A = p.a + p.ta.at(x, y, z);
  const float* B = p.b + p.tb.at(x, y, z);
  float* C = p.c + p.tc.at(x, y, z);
  const int cv = p.cols / VW;
  const int n = p.rows * cv;
  for (int base = threadIdx.x; base < n; base += 256 * U) {
    long long offa[U], offb[U], offc[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * 256;
      ok[u] = i < n;
      const int ic = ok[u] ? i : 0;
      const int r = POW2 ? (ic >> p.cv_shift) : ic / cv;
      const int col = (POW2 ? (ic & (cv - 1)) : ic - r * cv) * VW;
      offa[u] = r * p.lda + col;
      offb[u] = r * p.ldb + col;
      offc[u] = r * p.ldc + col;
    }
    if constexpr (VW == 4) {
      float4v va[U], vb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        va[u] = ld_nt(reinterpret_cast<const float4v*>(A + offa[u]));
        vb[u] = ld_nt(reinterpret_cast<const float4v*>(B + offb[u]));
      }
      issue_fence();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float4v vc;
        vc.x = ew_apply<OP>(va[u].x, vb[u].x);
        vc.y = ew_apply<OP>(va[u].y, vb[u].y);
        vc.z = ew_apply<OP>(va[u].z, vb[u].z);
        vc.w = ew_apply<OP>(va[u].w, vb[u].w);
        if (ok[u]) st_nt(vc, reinterpret_cast<float4v*>(C + offc[u]));
      }
    } else {
      float va[U], vb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        va[u] = ld_nt(A + offa[u]);
        vb[u] = ld_nt(B + offb[u]);
      }
      issue_fence();
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (ok[u]) st_nt(ew_apply<OP>(va[u], vb[u]), C + offc[u]);
    }
  }
}

// The flat form of a program whose Blocks' tiles cover one contiguous run in
// every operand at the same relative positions: c[i] = a[i] op b[i] over the
// run, 512 float4 per workgroup (two per thread, all four loads issued before
// the first use).  One Block's work is then spread over several workgroups and
// one workgroup covers parts of several Blocks; both are pure scheduling,
// since Blocks are independent.  For C1 (1024 x 1024, 32 x 64 tiles) this
// measured 3.43-3.45 us per launch against 4.05 us for the tiled kernel with
// its Block decode and 32 separate rows per workgroup.
template <int OP>
__global__ __launch_bounds__(256) void ew_flat_kernel(const float4v* __restrict__ a, const float4v* __restrict__ b,
                                                      float4v* __restrict__ c, long long nv) {
  const long long base = (long long)blockIdx.x * 512 + threadIdx.x;
  float4v va[2], vb[2];
  bool ok[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const long long i = base + u * 256;
    ok[u] = i < nv;
    va[u] = ld_nt(a + (ok[u] ? i : 0));
    vb[u] = ld_nt(b + (ok[u] ? i : 0));
  }
  issue_fence();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float4v vc;
    vc.x = ew_apply<OP>(va[u].x, vb[u].x);
    vc.y = ew_apply<OP>(va[u].y, vb[u].y);
    vc.z = ew_apply<OP>(va[u].z, vb[u].z);
    vc.w = ew_apply<OP>(va[u].w, vb[u].w);
    if (ok[u]) st_nt(vc, c + base + u * 256);
  }
}

struct SoftmaxArgs {
  const float* x;
  float* y;
  TileOff tx, ty;
  long long ldx, ldy;
  int rows, cols;
  BlockDecode grid;
  int tpr;  // threads per row (power of two, <= 256)
};

// Row reduction across the `tpr` threads that share a row.  For tpr <= 64 the
// group lies inside one wave and a butterfly suffices; wider rows combine the
// per-wave partials through LDS with a single barrier.  Max and sum use
// separate LDS slots, so the barrier of each reduction also orders the
// previous reduction's reads before the next writes of the same slot.
template <bool IS_MAX, int TPR>
__device__ __forceinline__ float row_reduce(float v, float* lds) {
  if constexpr (TPR >= 64) {
    v = wave_reduce<IS_MAX>(v);
  } else {
#pragma unroll
    for (int o = TPR >> 1; o > 0; o >>= 1) {
      const float t = __shfl_xor(v, o, 64);
      v = IS_MAX ? fmaxf(v, t) : v + t;
    }
  }
  if constexpr (TPR <= 64) {
    return v;
  } else {
    constexpr int PER_ROW = TPR / 64;
    float* slot = lds + (IS_MAX ? 0 : 4);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) slot[wave] = v;
    __syncthreads();
    const int first = (wave / PER_ROW) * PER_ROW;
    float r = slot[first];
#pragma unroll
    for (int k = 1; k < PER_ROW; ++k) r = IS_MAX ? fmaxf(r, slot[first + k]) : r + slot[first + k];
    return r;
  }
}

// All NV row loads of a pass are unconditional (out-of-range columns and rows
// read element 0 of the tile and are masked out afterwards) so they are in
// flight together; only the stores are predicated.
// EXACT: the row is exactly NV*VW*TPR elements and the tile has a multiple of
// 256/TPR rows, so no lane or row needs masking.
template <int NV, int VW, int TPR, bool EXACT>
__global__ __launch_bounds__(256) void row_softmax_kernel(SoftmaxArgs p) {
  __shared__ float lds[8];
  int x, y, z;
  p.grid(blockIdx.x, x, y, z);
  const float* X = p.x + p.tx.at(x, y, z);
  float* Y = p.y + p.ty.at(x, y, z);
  constexpr int tpr = TPR;
  constexpr int rpp = 256 / TPR;
  const int lane = threadIdx.x & (TPR - 1);
  const int row_in_pass = threadIdx.x / TPR;
  const int passes = (p.rows + rpp - 1) / rpp;
  for (int pass = 0; pass < passes; ++pass) {
    const int r = pass * rpp + row_in_pass;
    const bool live = EXACT || r < p.rows;
    const float* xr = X + (long long)(live ? r : 0) * p.ldx;
    float* yr = Y + (long long)r * p.ldy;
    float v[NV][VW];
    bool ok[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int col = (lane + j * tpr) * VW;
      ok[j] = EXACT || (live && col < p.cols);
      const int cc = ok[j] ? col : 0;
      if constexpr (VW == 4) {
        float4v t = ld_nt(reinterpret_cast<const float4v*>(xr + cc));
        v[j][0] = t.x;
        v[j][1] = t.y;
        v[j][2] = t.z;
        v[j][3] = t.w;
      } else {
        v[j][0] = ld_nt(xr + cc);
      }
    }
    issue_fence();
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int k = 0; k < VW; ++k) m = ok[j] ? fmaxf(m, v[j][k]) : m;
    m = row_reduce<true, TPR>(m, lds);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        v[j][k] = ok[j] ? exp_fast(v[j][k] - m) : 0.0f;
        s += v[j][k];
      }
    s = row_reduce<false, TPR>(s, lds);
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (!ok[j]) continue;
      const int col = (lane + j * tpr) * VW;
      if constexpr (VW == 4) {
        float4v t;
        t.x = v[j][0] * inv;
        t.y = v[j][1] * inv;
        t.z = v[j][2] * inv;
        t.w = v[j][3] * inv;
        st_nt(t, reinterpret_cast<float4v*>(yr + col));
      } else {
        st_nt(v[j][0] * inv, yr + col);
      }
    }
  }
}

// Full-row softmax: a TPB-thread workgroup owns one row of the tile at a time,
// each thread NV float4 of it (cols == TPB * NV * 4 exactly, row starts
// 16-byte aligned).  The row's loads are one instruction per float4 with
// compile-time offsets, max/sum are trees within the thread, then a wave
// butterfly, then one LDS exchange across the TPB/64 waves.  On gfx950 a
// 512-thread group with two float4 per thread keeps the HBM read/write
// stream at the rate of a plain device copy for 4096-wide rows.
template <int TPB, int NV>
__global__ __launch_bounds__(TPB) void row_softmax_wide_kernel(SoftmaxArgs p) {
  constexpr int NW = TPB / 64;
  __shared__ float lds[2][NW];
  int x, y, z;
  p.grid(blockIdx.x, x, y, z);
  const float* X = p.x + p.tx.at(x, y, z);
  float* Y = p.y + p.ty.at(x, y, z);
  const int w = threadIdx.x >> 6;
  for (int r = 0; r < p.rows; ++r) {
    const float4v* xr = reinterpret_cast<const float4v*>(X + r * p.ldx) + threadIdx.x;
    float4v* yr = reinterpret_cast<float4v*>(Y + r * p.ldy) + threadIdx.x;
    float4v v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = ld_nt(xr + j * TPB);
    issue_fence();
    float m = fmaxf(fmaxf(v[0].x, v[0].y), fmaxf(v[0].z, v[0].w));
#pragma unroll
    for (int j = 1; j < NV; ++j) m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
    m = wave_reduce<true>(m);
    if ((threadIdx.x & 63) == 0) lds[0][w] = m;
    __syncthreads();
    m = lds[0][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) m = fmaxf(m, lds[0][k]);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      v[j].x = exp_fast(v[j].x - m);
      v[j].y = exp_fast(v[j].y - m);
      v[j].z = exp_fast(v[j].z - m);
      v[j].w = exp_fast(v[j].w - m);
      s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    }
    s = wave_reduce<false>(s);
    // the max slot and the sum slot are distinct, so this barrier also orders
    // every read of lds[0] above before the next row's writes to it
    if ((threadIdx.x & 63) == 0) lds[1][w] = s;
    __syncthreads();
    s = lds[1][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) s += lds[1][k];
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < NV; ++j) st_nt(v[j] * inv, yr + j * TPB);
  }
}

// The same full-row softmax for the common case of one row per Block on a
// 1-D grid: Block x's row starts x * step float4 vectors past the row of
// Block 0, so the prologue is one multiply-add (no Block decode, no row loop,
// a four-argument kernarg segment).
template <int TPB, int NV>
__global__ __launch_bounds__(TPB) void row_softmax_1d_kernel(const float4v* __restrict__ x, float4v* __restrict__ y,
                                                             long long xstep, long long ystep) {
  constexpr int NW = TPB / 64;
  __shared__ float lds[2][NW];
  const int w = threadIdx.x >> 6;
  const float4v* xr = x + blockIdx.x * xstep + threadIdx.x;
  float4v* yr = y + blockIdx.x * ystep + threadIdx.x;
  float4v v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = ld_nt(xr + j * TPB);
  issue_fence();
  float m = fmaxf(fmaxf(v[0].x, v[0].y), fmaxf(v[0].z, v[0].w));
#pragma unroll
  for (int j = 1; j < NV; ++j) m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
  m = wave_reduce<true>(m);
  if ((threadIdx.x & 63) == 0) lds[0][w] = m;
  __syncthreads();
  m = lds[0][0];
#pragma unroll
  for (int k = 1; k < NW; ++k) m = fmaxf(m, lds[0][k]);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    v[j].x = exp_fast(v[j].x - m);
    v[j].y = exp_fast(v[j].y - m);
    v[j].z = exp_fast(v[j].z - m);
    v[j].w = exp_fast(v[j].w - m);
    s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  s = wave_reduce<false>(s);
  if ((threadIdx.x & 63) == 0) lds[1][w] = s;
  __syncthreads();
  s = lds[1][0];
#pragma unroll
  for (int k = 1; k < NW; ++k) s += lds[1][k];
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < NV; ++j) st_nt(v[j] * inv, yr + j * TPB);
}

TileOff to_off(const xt::TileAddr& a) { return TileOff{a.c0, a.sx, a.sy, a.sz}; }

bool aligned4(const xt::Access2D& a, const void* base) {
  return (reinterpret_cast<uintptr_t>(base) % 16) == 0 && a.ld % 4 == 0 && a.cols % 4 == 0 &&
         a.addr.c0 % 4 == 0 && a.addr.sx % 4 == 0 && a.addr.sy % 4 == 0 && a.addr.sz % 4 == 0;
}

}  // namespace

hipError_t launch_ew_binary(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  EwArgs a;
  a.a = static_cast<const float*>(bufs[p.a.arg]);
  a.b = static_cast<const float*>(bufs[p.b.arg]);
  a.c = static_cast<float*>(bufs[p.c.arg]);
  a.ta = to_off(p.a.addr);
  a.tb = to_off(p.b.addr);
  a.tc = to_off(p.c.addr);
  a.lda = p.a.ld;
  a.ldb = p.b.ld;
  a.ldc = p.c.ld;
  a.rows = static_cast<int>(p.c.rows);
  a.cols = static_cast<int>(p.c.cols);
  if (p.a.rows != p.c.rows || p.b.rows != p.c.rows || p.a.cols != p.c.cols ||
      p.b.cols != p.c.cols) {
    why = "elementwise operand tiles differ in shape";
    return hipErrorInvalidValue;
  }
  const bool vec = aligned4(p.a, a.a) && aligned4(p.b, a.b) && aligned4(p.c, a.c);
  if (p.ew_flat > 0 && p.ew_flat % 4 == 0 && vec) {
    // aligned4 checked every operand's origin and pitch: the run starts on a
    // 16-byte boundary in each
    const long long nv = p.ew_flat / 4;
    const long long wgs = (nv + 511) / 512;
    if (!grid_fits(wgs, 256)) {
      why = "elementwise run of " + std::to_string(p.ew_flat) + " elements exceeds one launch";
      return hipErrorInvalidValue;
    }
    const float4v* fa = reinterpret_cast<const float4v*>(a.a + p.a.addr.c0);
    const float4v* fb = reinterpret_cast<const float4v*>(a.b + p.b.addr.c0);
    float4v* fc = reinterpret_cast<float4v*>(a.c + p.c.addr.c0);
    const dim3 grid(static_cast<unsigned>(wgs)), block(256);
    switch (p.ew_op) {
      case xt::EwOp::Add: hipLaunchKernelGGL(ew_flat_kernel<0>, grid, block, 0, s, fa, fb, fc, nv); break;
      case xt::EwOp::Sub: hipLaunchKernelGGL(ew_flat_kernel<1>, grid, block, 0, s, fa, fb, fc, nv); break;
      default: hipLaunchKernelGGL(ew_flat_kernel<2>, grid, block, 0, s, fa, fb, fc, nv); break;
    }
    return hipGetLastError();
  }
  const int vw = vec ? 4 : 1;
  const long long cv = a.cols / vw;
  const long long nvec = static_cast<long long>(a.rows) * cv;
  if (nvec >= (1LL << 30)) {
    why = "elementwise tile too large";
    return hipErrorInvalidValue;
  }
  a.cv_shift = -1;
  if (cv > 0 && (cv & (cv - 1)) == 0) a.cv_shift = __builtin_ctzll(static_cast<unsigned long long>(cv));
  const int u = nvec <= 256 ? 1 : nvec <= 512 ? 2 : 4;
  const long long sx = p.c.addr.sx < 0 ? -p.c.addr.sx : p.c.addr.sx;
  const long long sy = p.c.addr.sy < 0 ? -p.c.addr.sy : p.c.addr.sy;
  a.grid = block_decode(p.grid[0], p.grid[1], p.grid[1] > 1 && (sx == 0 || (sy != 0 && sy < sx)));
  const long long blocks = grid_blocks(p);
  if (!grid_fits(blocks, 256)) {
    why = "elementwise grid of " + std::to_string(blocks) + " Blocks exceeds one launch (2^24 workgroups of 256)";
    return hipErrorInvalidValue;
  }
  dim3 grid(static_cast<unsigned>(blocks)), block(256);
  const int op = static_cast<int>(p.ew_op);
  const bool pow2 = a.cv_shift >= 0;
  // kernel variant index: op (3) x vector width (2) x U (3) x pow2 (2)
#define XT_EW(OPV, VWV, UV, P2) \
  hipLaunchKernelGGL((ew_binary_kernel<OPV, VWV, UV, P2>), grid, block, 0, s, a)
#define XT_EW_P2(OPV, VWV, UV) \
  do { if (pow2) XT_EW(OPV, VWV, UV, true); else XT_EW(OPV, VWV, UV, false); } while (0)
#define XT_EW_U(OPV, VWV)                \
  do {                                   \
    if (u == 1) XT_EW_P2(OPV, VWV, 1);   \
    else if (u == 2) XT_EW_P2(OPV, VWV, 2); \
    else XT_EW_P2(OPV, VWV, 4);          \
  } while (0)
#define XT_EW_OP(VWV)                  \
  do {                                 \
    if (op == 0) XT_EW_U(0, VWV);      \
    else if (op == 1) XT_EW_U(1, VWV); \
    else XT_EW_U(2, VWV);              \
  } while (0)
  if (vw == 4) XT_EW_OP(4);
  else XT_EW_OP(1);
#undef XT_EW_OP
#undef XT_EW_U
#undef XT_EW_P2
#undef XT_EW
  return hipGetLastError();
}

hipError_t launch_row_softmax(const xt::Plan& p, void* const* bufs, hipStream_t s,
                              std::string& why) {
  SoftmaxArgs a;
  a.x = static_cast<const float*>(bufs[p.a.arg]);
  a.y = static_cast<float*>(bufs[p.c.arg]);
  a.tx = to_off(p.a.addr);
  a.ty = to_off(p.c.addr);
  a.ldx = p.a.ld;
  a.ldy = p.c.ld;
  a.rows = static_cast<int>(p.a.rows);
  a.cols = static_cast<int>(p.a.cols);
  a.grid = block_decode(p.grid[0], p.grid[1], false);
  if (p.c.rows != p.a.rows || p.c.cols != p.a.cols) {
    why = "softmax input and output tiles differ in shape";
    return hipErrorInvalidValue;
  }
  const int vw = (aligned4(p.a, a.x) && aligned4(p.c, a.y)) ? 4 : 1;
  const long long blocks = grid_blocks(p);
  const bool wide = vw == 4 && a.cols % 2048 == 0 && a.cols <= 8 * 2048;
  if (!grid_fits(blocks, wide ? 512 : 256)) {
    why = "softmax grid of " + std::to_string(blocks) + " Blocks exceeds one launch";
    return hipErrorInvalidValue;
  }
  dim3 grid(static_cast<unsigned>(blocks));
  if (wide && a.rows == 1 && p.grid[1] == 1 && p.grid[2] == 1) {
    // one row per Block on a 1-D grid (aligned4 makes every offset a float4 multiple)
    const float4v* x4 = reinterpret_cast<const float4v*>(a.x + p.a.addr.c0);
    float4v* y4 = reinterpret_cast<float4v*>(a.y + p.c.addr.c0);
    const long long xs = p.a.addr.sx / 4, ys = p.c.addr.sx / 4;
    switch (a.cols / 2048) {
#define XT_SM1(NVV) \
  case NVV: hipLaunchKernelGGL((row_softmax_1d_kernel<512, NVV>), grid, dim3(512), 0, s, x4, y4, xs, ys); break
      XT_SM1(1); XT_SM1(2); XT_SM1(3); XT_SM1(4); XT_SM1(5); XT_SM1(6); XT_SM1(7); XT_SM1(8);
#undef XT_SM1
    }
    return hipGetLastError();
  }
  if (wide) {
    a.tpr = 512;
    switch (a.cols / 2048) {
#define XT_SMW(NVV) \
  case NVV: hipLaunchKernelGGL((row_softmax_wide_kernel<512, NVV>), grid, dim3(512), 0, s, a); break
      XT_SMW(1); XT_SMW(2); XT_SMW(3); XT_SMW(4); XT_SMW(5); XT_SMW(6); XT_SMW(7); XT_SMW(8);
#undef XT_SMW
    }
    return hipGetLastError();
  }
  // smallest NV in {1,2,4,8} with NV * VW * 256 >= cols, then the narrowest
  // power-of-two thread group that covers the row
  int nv = 1;
  while (nv < 8 && nv * vw * 256 < a.cols) nv *= 2;
  if (nv * vw * 256 < a.cols) {
    // rows above 2048 floats are planned here only as float4 vectors; a buffer
    // that is not 16-byte aligned runs on the tile interpreter instead
    if (p.vm_fallback) return launch_tilevm(p, bufs, s, why);
    why = "softmax rows of " + std::to_string(a.cols) +
          " floats need 16-byte aligned buffers, and the tile interpreter cannot run this program: " +
          p.vm_fallback_why;
    return hipErrorInvalidValue;
  }
  int need = (a.cols + nv * vw - 1) / (nv * vw);
  int tpr = 1;
  while (tpr < need) tpr *= 2;
  a.tpr = tpr;
  const bool exact = a.cols == nv * vw * tpr && a.rows % (256 / tpr) == 0;
  dim3 block(256);
#define XT_SM(NVV, VWV, TPRV)                                                               \
  do {                                                                                      \
    if (VWV == 4 && TPRV >= 64 && exact)                                                    \
      hipLaunchKernelGGL((row_softmax_kernel<NVV, VWV, TPRV, (VWV == 4 && TPRV >= 64)>),    \
                         grid, block, 0, s, a);                                             \
    else                                                                                    \
      hipLaunchKernelGGL((row_softmax_kernel<NVV, VWV, TPRV, false>), grid, block, 0, s, a); \
  } while (0)
#define XT_SM_TPR(NVV, VWV)                          \
  switch (tpr) {                                     \
    case 1: XT_SM(NVV, VWV, 1); break;               \
    case 2: XT_SM(NVV, VWV, 2); break;               \
    case 4: XT_SM(NVV, VWV, 4); break;               \
    case 8: XT_SM(NVV, VWV, 8); break;               \
    case 16: XT_SM(NVV, VWV, 16); break;             \
    case 32: XT_SM(NVV, VWV, 32); break;             \
    case 64: XT_SM(NVV, VWV, 64); break;             \
    case 128: XT_SM(NVV, VWV, 128); break;           \
    default: XT_SM(NVV, VWV, 256); break;            \
  }
  if (vw == 4) {
    switch (nv) {
      case 1: XT_SM_TPR(1, 4); break;
      case 2: XT_SM_TPR(2, 4); break;
      case 4: XT_SM_TPR(4, 4); break;
      default: XT_SM_TPR(8, 4); break;
    }
  } else {
    switch (nv) {
      case 1: XT_SM_TPR(1, 1); break;
      case 2: XT_SM_TPR(2, 1); break;
      case 4: XT_SM_TPR(4, 1); break;
      default: XT_SM_TPR(8, 1); break;
    }
  }
#undef XT_SM_TPR
#undef XT_SM
  return hipGetLastError();
}

}  // namespace xtk
