/*
 * TEST INFRASTRUCTURE - the parity oracle.  Not part of the product: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * A loop-lowered CPU executor of an xt program: every Block of the grid runs
 * the program's ops one loop nest at a time, exactly as the reference's
 * serialized form would (lib/xt/XTSerialize.cpp:68-104: z outer, then y, then
 * x).  Blocks are independent (README.md:85-89), so with nthreads > 1 they
 * are distributed over OpenMP threads.
 *
 * Semantics restated (file:line into the reference):
 *   load        tile at element offset coord*S (lib/xt/XTToNova.cpp:82-101)
 *   shared = k  the first block of the sharing group provides the value, i.e.
 *               coordinates read block-id axes < k as 0 (XTSerialize.cpp:86-101)
 *   load_conv2d halo slice + zero pad, out = sum in*f (XTToNova.cpp:110-142,
 *               353-437); source rows/cols outside the array read as 0
 *   add/sub/mul right-aligned broadcast (lib/xt/XTOps.cpp:104-120)
 *   reduce_*    keeps the reduced dim (lib/xt/XTOps.cpp:274-299), sequential order
 *   matmul/mma  C = sum_k A*B (+acc); accumulated in double, rounded once
 *   truediv     traced as mul(x, reciprocal(y)) (xtile/dsl.py:354-357)
 *   reshape     row-major reinterpretation; transpose swaps dims 1,2 (rank 3);
 *               permute reorders dims (lib/xt/XTOps.cpp:309-397)
 *   itof/ftoi   ftoi rounds half to even and saturates to the i8 range
 *               (the reference fixes no rounding rule: parity unpinned)
 * Values are held as f32 inside a block; f16/bf16/i8 loads convert exactly,
 * stores round to nearest even (f16/bf16).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum {
  XO_F32 = 0,
  XO_F16 = 1,
  XO_BF16 = 2,
  XO_I8 = 3,
};

enum {
  XO_LOAD = 1,
  XO_LOAD_CONV = 2,
  XO_STORE = 3,
  XO_ADD = 10,
  XO_SUB = 11,
  XO_MUL = 12,
  XO_EXP = 20,
  XO_COS = 21,
  XO_SIN = 22,
  XO_RECIP = 23,
  XO_RSQRT = 24,
  XO_SIGMOID = 25,
  XO_TANH = 26,
  XO_SILU = 27,
  XO_ITOF = 28,
  XO_FTOI = 29,
  XO_RSUM = 30,
  XO_RMAX = 31,
  XO_MATMUL = 40,
  XO_MMA = 41,
  XO_RESHAPE = 50,
  XO_TRANSPOSE = 51,
  XO_PERMUTE = 52,
};

#define XO_MAXR 4

typedef struct {
  int code;
  int dst, a, b, c;          /* value slots (-1 unused) */
  int arg;                   /* memref argument index */
  int rank;                  /* rank of dst (or of the stored tile) */
  long long shape[XO_MAXR];  /* dst shape (or stored tile shape) */
  int coord_axis[XO_MAXR];   /* -1: constant */
  long long coord_val[XO_MAXR];
  int shared;
  int axis;
  long long pad[4], stride[2], dil[2];
  int perm[XO_MAXR];
} xo_op;

typedef struct {
  int nargs;
  int arg_elem[16];
  int arg_rank[16];
  long long arg_shape[16][XO_MAXR];
  int nvals;
  int val_rank[64];
  long long val_shape[64][XO_MAXR];
  int nops;
  const xo_op* ops;
  int grid[3];
} xo_prog;

/* ---- element conversion ---------------------------------------------- */

static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  int exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float v = (float)man * (1.0f / 16777216.0f);
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static uint16_t f32_to_f16(float f) { /* round to nearest even */
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0));
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (absx < 0x38800000u) {                                    /* subnormal or zero */
    float a;
    memcpy(&a, &absx, 4);
    float scaled = a * 16777216.0f; /* in units of 2^-24 */
    float r = nearbyintf(scaled);   /* default rounding mode: half to even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t e = ((absx >> 23) - 127 + 15);
  uint32_t m = absx & 0x7fffffu;
  uint32_t out = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) out += 1;
  return (uint16_t)(sign | out);
}

static float bf16_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return (uint16_t)(x >> 16);
}

static float ftoi_i8(float v) {
  if (v != v) return 0.0f;
  float r = nearbyintf(v);
  if (r > 127.0f) r = 127.0f;
  if (r < -128.0f) r = -128.0f;
  return r;
}

static float read_elem(const void* base, int elem, long long i) {
  switch (elem) {
    case XO_F32: return ((const float*)base)[i];
    case XO_F16: return f16_to_f32(((const uint16_t*)base)[i]);
    case XO_BF16: return bf16_to_f32(((const uint16_t*)base)[i]);
    default: return (float)((const int8_t*)base)[i];
  }
}

static void write_elem(void* base, int elem, long long i, float v) {
  switch (elem) {
    case XO_F32: ((float*)base)[i] = v; break;
    case XO_F16: ((uint16_t*)base)[i] = f32_to_f16(v); break;
    case XO_BF16: ((uint16_t*)base)[i] = f32_to_bf16(v); break;
    default: ((int8_t*)base)[i] = (int8_t)ftoi_i8(v); break;
  }
}

/* ---- helpers ------------------------------------------------------------ */

static long long numel(int rank, const long long* s) {
  long long n = 1;
  for (int d = 0; d < rank; ++d) n *= s[d];
  return n;
}

/* element offset of tile element `idx` (row-major within the tile) */
static long long tile_elem_offset(const xo_prog* p, const xo_op* o, const int bid[3],
                                  long long idx) {
  const long long* mem = p->arg_shape[o->arg];
  int rank = o->rank;
  long long t[XO_MAXR];
  for (int d = rank - 1; d >= 0; --d) {
    t[d] = idx % o->shape[d];
    idx /= o->shape[d];
  }
  long long off = 0;
  for (int d = 0; d < rank; ++d) {
    long long coord;
    if (o->coord_axis[d] < 0) coord = o->coord_val[d];
    else coord = o->coord_axis[d] < o->shared ? 0 : bid[o->coord_axis[d]];
    off = off * mem[d] + coord * o->shape[d] + t[d];
  }
  return off;
}

static float unary(int code, float x) {
  switch (code) {
    case XO_EXP: return expf(x);
    case XO_COS: return cosf(x);
    case XO_SIN: return sinf(x);
    case XO_RECIP: return 1.0f / x;
    case XO_RSQRT: return 1.0f / sqrtf(x);
    case XO_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case XO_TANH: return tanhf(x);
    case XO_SILU: return x * (1.0f / (1.0f + expf(-x)));
    case XO_ITOF: return x;
    case XO_FTOI: return ftoi_i8(x);
  }
  return x;
}

/* ---- one block ------------------------------------------------------------- */

static void run_block(const xo_prog* p, void** bufs, const int bid[3], float** vals) {
  for (int k = 0; k < p->nops; ++k) {
    const xo_op* o = &p->ops[k];
    float* dst = o->dst >= 0 ? vals[o->dst] : NULL;
    switch (o->code) {
      case XO_LOAD: {
        /* row by row: the innermost tile dim is contiguous in the memref */
        long long n = numel(o->rank, o->shape), w = o->shape[o->rank - 1];
        int elem = p->arg_elem[o->arg];
        for (long long i = 0; i < n; i += w) {
          long long base = tile_elem_offset(p, o, bid, i);
          for (long long j = 0; j < w; ++j) dst[i + j] = read_elem(bufs[o->arg], elem, base + j);
        }
        break;
      }
      case XO_STORE: {
        const float* src = vals[o->a];
        long long n = numel(o->rank, o->shape), w = o->shape[o->rank - 1];
        int elem = p->arg_elem[o->arg];
        for (long long i = 0; i < n; i += w) {
          long long base = tile_elem_offset(p, o, bid, i);
          for (long long j = 0; j < w; ++j) write_elem(bufs[o->arg], elem, base + j, src[i + j]);
        }
        break;
      }
      case XO_LOAD_CONV: {
        /* source [N,H,W,C], filter value [KH,KW,C,CO], result [TB,TH,TW,TC] */
        const long long* src = p->arg_shape[o->arg];
        const float* filt = vals[o->b];
        const long long* fs = p->val_shape[o->b];
        long long KH = fs[0], KW = fs[1], C = fs[2], CO = fs[3];
        long long TB = o->shape[0], TH = o->shape[1], TW = o->shape[2], TC = o->shape[3];
        long long ci[4];
        for (int d = 0; d < 4; ++d)
          ci[d] = o->coord_axis[d] < 0 ? o->coord_val[d] : bid[o->coord_axis[d]];
        long long b0 = ci[0] * TB, oh0 = ci[1] * TH, ow0 = ci[2] * TW, c0 = ci[3] * C;
        int elem = p->arg_elem[o->arg];
        double* acc = (double*)malloc(sizeof(double) * (size_t)TC);
        for (long long b = 0; b < TB; ++b)
          for (long long i = 0; i < TH; ++i)
            for (long long j = 0; j < TW; ++j) {
              for (long long co = 0; co < TC; ++co) acc[co] = 0.0;
              for (long long kh = 0; kh < KH; ++kh) {
                long long ih = (oh0 + i) * o->stride[0] - o->pad[0] + kh * o->dil[0];
                if (ih < 0 || ih >= src[1]) continue; /* zero padding */
                for (long long kw = 0; kw < KW; ++kw) {
                  long long iw = (ow0 + j) * o->stride[1] - o->pad[1] + kw * o->dil[1];
                  if (iw < 0 || iw >= src[2]) continue;
                  long long base = (((b0 + b) * src[1] + ih) * src[2] + iw) * src[3] + c0;
                  for (long long c = 0; c < C; ++c) {
                    double x = (double)read_elem(bufs[o->arg], elem, base + c);
                    const float* fr = filt + ((kh * KW + kw) * C + c) * CO;
                    for (long long co = 0; co < TC; ++co) acc[co] += x * (double)fr[co];
                  }
                }
              }
              float* out = dst + ((b * TH + i) * TW + j) * TC;
              for (long long co = 0; co < TC; ++co) out[co] = (float)acc[co];
            }
        free(acc);
        break;
      }
      case XO_ADD:
      case XO_SUB:
      case XO_MUL: {
        const float* A = vals[o->a];
        const float* B = vals[o->b];
        const long long* sa = p->val_shape[o->a];
        const long long* sb = p->val_shape[o->b];
        int ra = p->val_rank[o->a], rb = p->val_rank[o->b], r = o->rank;
        long long n = numel(r, o->shape);
        for (long long i = 0; i < n; ++i) {
          long long rem = i, ia = 0, ib = 0, mula = 1, mulb = 1;
          for (int d = r - 1; d >= 0; --d) {
            long long t = rem % o->shape[d];
            rem /= o->shape[d];
            int da = d - (r - ra), db = d - (r - rb);
            if (da >= 0) {
              ia += (sa[da] == 1 ? 0 : t) * mula;
              mula *= sa[da];
            }
            if (db >= 0) {
              ib += (sb[db] == 1 ? 0 : t) * mulb;
              mulb *= sb[db];
            }
          }
          float x = A[ia], y = B[ib];
          dst[i] = o->code == XO_ADD ? x + y : o->code == XO_SUB ? x - y : x * y;
        }
        break;
      }
      case XO_EXP: case XO_COS: case XO_SIN: case XO_RECIP: case XO_RSQRT:
      case XO_SIGMOID: case XO_TANH: case XO_SILU: case XO_ITOF: case XO_FTOI: {
        const float* A = vals[o->a];
        long long n = numel(o->rank, o->shape);
        for (long long i = 0; i < n; ++i) dst[i] = unary(o->code, A[i]);
        break;
      }
      case XO_RSUM:
      case XO_RMAX: {
        const float* A = vals[o->a];
        const long long* s = p->val_shape[o->a];
        long long R = s[0], C = s[1];
        if (o->axis == 1) {
          for (long long i = 0; i < R; ++i) {
            float acc = o->code == XO_RSUM ? 0.0f : -INFINITY;
            for (long long j = 0; j < C; ++j)
              acc = o->code == XO_RSUM ? acc + A[i * C + j] : fmaxf(acc, A[i * C + j]);
            dst[i] = acc;
          }
        } else {
          for (long long j = 0; j < C; ++j) {
            float acc = o->code == XO_RSUM ? 0.0f : -INFINITY;
            for (long long i = 0; i < R; ++i)
              acc = o->code == XO_RSUM ? acc + A[i * C + j] : fmaxf(acc, A[i * C + j]);
            dst[j] = acc;
          }
        }
        break;
      }
      case XO_MATMUL:
      case XO_MMA: {
        const float* A = vals[o->a];
        const float* B = vals[o->b];
        long long M = p->val_shape[o->a][0], K = p->val_shape[o->a][1];
        long long N = p->val_shape[o->b][1];
        double* row = (double*)malloc(sizeof(double) * (size_t)N);
        for (long long i = 0; i < M; ++i) {
          for (long long j = 0; j < N; ++j) row[j] = 0.0;
          for (long long k = 0; k < K; ++k) {
            double a = A[i * K + k];
            const float* br = B + k * N;
            for (long long j = 0; j < N; ++j) row[j] += a * (double)br[j];
          }
          for (long long j = 0; j < N; ++j) {
            double v = row[j];
            if (o->code == XO_MMA) v += (double)vals[o->c][i * N + j];
            dst[i * N + j] = (float)v;
          }
        }
        free(row);
        break;
      }
      case XO_RESHAPE: {
        memcpy(dst, vals[o->a], sizeof(float) * (size_t)numel(o->rank, o->shape));
        break;
      }
      case XO_TRANSPOSE: {
        const float* A = vals[o->a];
        const long long* s = p->val_shape[o->a];
        for (long long b = 0; b < s[0]; ++b)
          for (long long i = 0; i < s[1]; ++i)
            for (long long j = 0; j < s[2]; ++j)
              dst[(b * s[2] + j) * s[1] + i] = A[(b * s[1] + i) * s[2] + j];
        break;
      }
      case XO_PERMUTE: {
        const float* A = vals[o->a];
        const long long* s = p->val_shape[o->a];
        int r = p->val_rank[o->a];
        long long n = numel(r, s);
        long long in_stride[XO_MAXR];
        in_stride[r - 1] = 1;
        for (int d = r - 2; d >= 0; --d) in_stride[d] = in_stride[d + 1] * s[d + 1];
        for (long long i = 0; i < n; ++i) {
          long long rem = i, src = 0;
          for (int d = r - 1; d >= 0; --d) {
            long long t = rem % o->shape[d];
            rem /= o->shape[d];
            src += t * in_stride[o->perm[d]];
          }
          dst[i] = A[src];
        }
        break;
      }
      default:
        break;
    }
  }
}

/* Runs every block of the grid.  Returns 0 on success, -1 on allocation
 * failure.  nthreads <= 1 runs blocks sequentially in z -> y -> x order. */
int xo_run(const xo_prog* p, void** bufs, int nthreads) {
  long long nblocks = (long long)p->grid[0] * p->grid[1] * p->grid[2];
  int failed = 0;
#ifdef _OPENMP
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads)
#endif
  {
    float* vals[64];
    int ok = 1;
    for (int v = 0; v < p->nvals; ++v) {
      vals[v] = (float*)malloc(sizeof(float) * (size_t)numel(p->val_rank[v], p->val_shape[v]));
      if (!vals[v]) ok = 0;
    }
    if (!ok) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
      failed = 1;
    } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
      for (long long blk = 0; blk < nblocks; ++blk) {
        int bid[3];
        bid[0] = (int)(blk % p->grid[0]);
        bid[1] = (int)((blk / p->grid[0]) % p->grid[1]);
        bid[2] = (int)(blk / ((long long)p->grid[0] * p->grid[1]));
        run_block(p, bufs, bid, vals);
      }
    }
    for (int v = 0; v < p->nvals; ++v) free(vals[v]);
  }
  return failed ? -1 : 0;
}

/* Exposed conversions so tests can pin them against numpy. */
float xo_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t xo_f32_to_f16(float f) { return f32_to_f16(f); }
float xo_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
uint16_t xo_f32_to_bf16(float f) { return f32_to_bf16(f); }
int xo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
