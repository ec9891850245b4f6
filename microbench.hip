// Microbenchmarks of the gfx950 CU resources the tile kernels are bound by:
// LDS read bandwidth for the fragment patterns the conv and GEMM kernels use,
// the transposing filter read, the matrix-core issue rate of a dependent
// chain (alone and fed from LDS, with or without other waves of the CU
// streaming memory traffic), and the L2 -> CU throughput of LDS DMA and of
// plain 16-byte loads.  Measurement tooling beside bench.py; the library
// never uses it.
//
//   hipcc -std=c++17 -O3 --offload-arch=gfx950 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops microbench.hip -o microbench && ./microbench
//
// Every kernel runs 256 workgroups (one per CU) and times itself per wave
// with s_memtime (the shader clock) and s_memrealtime (100 MHz), so each line
// gives cycles and the clock the chip ran at.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef short short8 __attribute__((ext_vector_type(8)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_t;

constexpr int kBlocks = 256;
constexpr int kLds = 64 * 1024;  // dynamic LDS of every kernel below

__device__ __forceinline__ unsigned lds_u(const void* p) {
  return (unsigned)reinterpret_cast<uintptr_t>((const lds_t*)p);
}
__device__ __forceinline__ i32x4 rsrc(const void* base, unsigned bytes) {
  const unsigned long long b = reinterpret_cast<unsigned long long>(base);
  return i32x4{(int)(unsigned)b, (int)(unsigned)(b >> 32) & 0xFFFF, (int)bytes, 0x00020000};
}
__device__ __forceinline__ void stamp(unsigned long long* out, unsigned long long c0, unsigned long long r0) {
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    out[(blockIdx.x * 16 + w) * 2] = c1 - c0;
    out[(blockIdx.x * 16 + w) * 2 + 1] = r1 - r0;
  }
}
__device__ __forceinline__ void fill_lds(unsigned char* lds) {
  for (int i = threadIdx.x; i < kLds / 4; i += blockDim.x)
    ((unsigned*)lds)[i] = ((unsigned)i * 2654435761u) & 0xBBFFBBFFu;  // finite f16 pairs
  __syncthreads();
}

// ds_read_b128, eight in flight per wave.  Pattern 0: 16-lane groups of 16
// consecutive 16-byte chunks.  Pattern 1: the MFMA A fragment of 32 output
// pixels starting at pixel 40 of a row of 56 (so the group crosses a row),
// pixel pitch `pitch`, row pitch `rpitch` (56 * pitch: rows laid out
// contiguously; 58 * pitch: an unpadded halo row, two pixels longer).
__global__ void k_lds(int iters, int pattern, int pitch, int rpitch, unsigned long long* out) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  fill_lds(lds);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  unsigned base = lds_u(lds) + (w & 3) * 64;
  if (pattern == 0) {
    base += (lane & 15) * 16 + (lane >> 4) * 256 + (w & 7) * 4096;
  } else {
    const int q = 40 + (lane & 31);
    base += (q / 56) * rpitch + (q % 56) * pitch + (lane >> 5) * 16;
  }
  u4 v0, v1, v2, v3, v4, v5, v6, v7;
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:32\n\tds_read_b128 %2, %8 offset:64\n\t"
        "ds_read_b128 %3, %8 offset:96\n\tds_read_b128 %4, %8 offset:16\n\tds_read_b128 %5, %8 offset:48\n\t"
        "ds_read_b128 %6, %8 offset:80\n\tds_read_b128 %7, %8 offset:112\n\ts_waitcnt lgkmcnt(0)"
        : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
        : "v"(base)
        : "memory");
  }
  asm volatile("" ::"v"(v0), "v"(v1), "v"(v2), "v"(v3), "v"(v4), "v"(v5), "v"(v6), "v"(v7));
  stamp(out, c0, r0);
}

// ds_read_b64_tr_b16 on a [K][64] f16 filter with the conv band kernel's
// chunk swizzle (16 x 32-channel fragments of two reads each), eight reads in
// flight.
__global__ void k_tr(int iters, unsigned long long* out) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  fill_lds(lds);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, li = lane & 15, j = w & 1;
  int pb[2];
  for (int h = 0; h < 2; ++h) {
    const int k = 8 * (g >> 1) + 4 * h + (li >> 2);
    const int cb = (32 * j + 16 * (g & 1) + 4 * (li & 3)) * 2;
    pb[h] = k * 128 + (((cb >> 4) ^ (4 * ((k >> 1) & 1))) << 4) + (cb & 15);
  }
  const lds_t* L = (const lds_t*)lds;
  short4v a[8];
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      a[i] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((short4v __attribute__((address_space(3)))*)(L + pb[i & 1] + 2048 * (i >> 1)));
    asm volatile("s_waitcnt lgkmcnt(0)" ::"v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]),
                 "v"(a[7])
                 : "memory");
  }
  stamp(out, c0, r0);
}

// v_mfma_f32_32x32x16_f16 dependent chain (one accumulator), in waves 0-3.
// FEED: the A operand comes from ds_read_b128 two steps ahead, in the band
// kernel's pixel pattern (32 pixels of 56-pixel rows, 144-byte pixels,
// 8576-byte rows, 36 steps over 9 taps).  HELP (waves 4-7, when launched
// with 512 threads): 0 idle, 1 non-temporal 1 KB stores to a 64 MB buffer,
// 2 LDS DMA of 1 KB from it.
template <bool FEED, int HELP>
__global__ void k_mfma(int iters, unsigned char* buf, unsigned long long* out, float* sink) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  fill_lds(lds);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w >= 4) {
    const unsigned win = 64u << 20;
    const i32x4 r = rsrc(buf, win);
    unsigned off = ((blockIdx.x * 4 + (w - 4)) * 65536u) % win;
    // LDS DMA targets [48 KB, 64 KB): 8 instructions of 1 KB per helper wave
    const unsigned ldsb = lds_u(lds) + 49152 + (w - 4) * 4096;
    for (int it = 0; HELP && it < iters * 4; ++it) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned o = (off + i * 1024 + lane * 16) % win;
        if (HELP == 1) {
          const u4 v = {o, o, o, o};
          asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen nt" ::"v"(v), "v"(o), "s"(r) : "memory");
        } else {
          unsigned saved;
          asm volatile(
              "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
              : "=&s"(saved)
              : "s"(ldsb + i * 1024), "v"(o), "s"(r)
              : "memory");
        }
      }
      off = (off + 4096) % win;
      asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  typedef short8 __attribute__((address_space(3))) lds_s8;
  const lds_t* L = (const lds_t*)lds;
  const int q = 32 * w + (lane & 31);  // pixels 0-127: rows 0-2 of the band
  // largest offset: row 2 + kh 2 -> 4 * 8576 + 55 * 144 + 2 * 144 + 112 + 16 = 42640 < 48 KB
  const int base = (q / 56) * 8576 + (q % 56) * 144 + (lane >> 5) * 16;
  half8 b;
  for (int i = 0; i < 8; ++i) b[i] = (_Float16)(i * 0.01f + lane * 0.001f);
  float16v acc;
  for (int i = 0; i < 16; ++i) acc[i] = 0;
  short8 ring[3];
  auto rd = [&](int s) {
    const int t = s >> 2, c = s & 3;
    return *(const lds_s8*)(L + base + (t / 3) * 8576 + (t % 3) * 144 + 32 * c);
  };
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    if (FEED) {
      ring[0] = rd(0);
      ring[1] = rd(1);
    }
#pragma unroll
    for (int s = 0; s < 36; ++s) {
      short8 a = __builtin_bit_cast(short8, b);
      if (FEED) {
        if (s + 2 < 36) ring[(s + 2) % 3] = rd(s + 2);
        a = ring[s % 3];
        asm volatile("s_waitcnt lgkmcnt(1)" ::: "memory");
      }
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    }
  }
  float s = 0;
  for (int i = 0; i < 16; ++i) s += acc[i];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  stamp(out, c0, r0);
}

// L2 -> CU throughput: every wave streams 8 x 1 KB a round from a 2 MB
// (L2-resident) buffer, by LDS DMA (DMA) or into registers.
template <bool DMA>
__global__ void k_l2(const unsigned char* src, int iters, unsigned long long* out, float* sink) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned win = 2u << 20;
  const i32x4 r = rsrc(src, win);
  // DMA targets: 8 KB per wave, 16 waves at most -> [0, 128 KB) of a 128 KB allocation
  const unsigned lbase = lds_u(lds) + w * 8192;
  unsigned off = ((blockIdx.x * 16 + w) * 8192u) % win;
  u4 acc = {0, 0, 0, 0};
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const unsigned o = (off + i * 1024 + lane * 16) % win;
      if (DMA) {
        unsigned saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "s"(lbase + i * 1024), "v"(o), "s"(r)
                     : "memory");
      } else {
        u4 v;
        asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(o), "s"(r));
        acc ^= v;
      }
    }
    off = (off + 8192u * 16 * 256) % win;
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  sink[blockIdx.x * blockDim.x + threadIdx.x] = (float)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
  stamp(out, c0, r0);
}

struct Timing {
  double cycles, ghz;
};

int main() {
  unsigned char* buf;
  unsigned long long* d;
  float* sink;
  if (hipMalloc(&buf, 64u << 20) != hipSuccess || hipMalloc(&d, kBlocks * 16 * 2 * 8) != hipSuccess ||
      hipMalloc(&sink, kBlocks * 1024 * 4) != hipSuccess || hipMemset(buf, 1, 64u << 20) != hipSuccess) {
    fprintf(stderr, "allocation failed\n");
    return 1;
  }
  std::vector<unsigned long long> h(kBlocks * 16 * 2);
  // median over the timed waves of the second of two launches
  auto timed = [&](auto launch, int waves) {
    launch();
    launch();
    if (hipDeviceSynchronize() != hipSuccess) { fprintf(stderr, "kernel failed\n"); exit(1); }
    if (hipMemcpy(h.data(), d, h.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) exit(1);
    std::vector<double> c, g;
    for (int b = 0; b < kBlocks; ++b)
      for (int w = 0; w < waves; ++w) {
        const double cy = (double)h[(b * 16 + w) * 2], rt = (double)h[(b * 16 + w) * 2 + 1];
        c.push_back(cy);
        g.push_back(cy / (rt * 10.0));
      }
    std::sort(c.begin(), c.end());
    std::sort(g.begin(), g.end());
    return Timing{c[c.size() / 2], g[g.size() / 2]};
  };
  const int IT = 2000;
  printf("# LDS reads (B/clk/CU)\n");
  for (int waves : {4, 8}) {
    Timing t = timed([&] { hipLaunchKernelGGL(k_lds, dim3(kBlocks), dim3(64 * waves), kLds, 0, IT, 0, 16, 0, d); }, waves);
    printf("lds  ds_read_b128 contiguous 16-lane groups       waves/CU %d: %6.1f B/clk  (%.2f GHz)\n", waves,
           (double)IT * 8 * 1024 * waves / t.cycles, t.ghz);
    for (int pitch : {128, 144, 160, 176, 192})
      for (int jump : {0, 2}) {
        Timing u = timed(
            [&] { hipLaunchKernelGGL(k_lds, dim3(kBlocks), dim3(64 * waves), kLds, 0, IT, 1, pitch, (56 + jump) * pitch, d); },
            waves);
        printf("lds  A fragment, pixel pitch %3d, row %s waves/CU %d: %6.1f B/clk\n", pitch,
               jump ? "+2 pixels (unpadded halo)" : "contiguous               ", waves,
               (double)IT * 8 * 1024 * waves / u.cycles);
      }
    Timing v = timed([&] { hipLaunchKernelGGL(k_tr, dim3(kBlocks), dim3(64 * waves), kLds, 0, IT, d); }, waves);
    printf("lds  ds_read_b64_tr_b16 filter fragments          waves/CU %d: %6.1f B/clk\n", waves,
           (double)IT * 8 * 512 * waves / v.cycles);
  }
  printf("# matrix cores: v_mfma_f32_32x32x16_f16 dependent chain in 4 waves (one per SIMD)\n");
  const int MI = 200;
  auto mline = [&](const char* name, Timing t) {
    const double cpm = t.cycles / (MI * 36.0);
    printf("mfma %-52s: %5.1f cycles per MFMA at %.2f GHz (%.1f ns)\n", name, cpm, t.ghz, cpm / t.ghz);
  };
  mline("operands in registers", timed([&] { hipLaunchKernelGGL((k_mfma<false, 0>), dim3(kBlocks), dim3(256), kLds, 0, MI, buf, d, sink); }, 4));
  mline("A from LDS two steps ahead (band pixel pattern)", timed([&] { hipLaunchKernelGGL((k_mfma<true, 0>), dim3(kBlocks), dim3(256), kLds, 0, MI, buf, d, sink); }, 4));
  mline("  + 4 idle waves", timed([&] { hipLaunchKernelGGL((k_mfma<true, 0>), dim3(kBlocks), dim3(512), kLds, 0, MI, buf, d, sink); }, 4));
  mline("  + 4 waves streaming 1 KB stores to HBM", timed([&] { hipLaunchKernelGGL((k_mfma<true, 1>), dim3(kBlocks), dim3(512), kLds, 0, MI, buf, d, sink); }, 4));
  mline("  + 4 waves streaming LDS DMA from HBM", timed([&] { hipLaunchKernelGGL((k_mfma<true, 2>), dim3(kBlocks), dim3(512), kLds, 0, MI, buf, d, sink); }, 4));
  printf("# L2 -> CU throughput from a 2 MB buffer (B/clk/CU)\n");
  if (hipFuncSetAttribute((const void*)k_l2<true>, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024) != hipSuccess) return 1;
  for (int dma : {1, 0})
    for (int waves : {4, 8, 16}) {
      Timing t = timed(
          [&] {
            if (dma) hipLaunchKernelGGL(k_l2<true>, dim3(kBlocks), dim3(64 * waves), 128 * 1024, 0, buf, 200, d, sink);
            else hipLaunchKernelGGL(k_l2<false>, dim3(kBlocks), dim3(64 * waves), 0, 0, buf, 200, d, sink);
          },
          waves);
      printf("l2   %s waves/CU %2d: %6.1f B/clk  (%.2f GHz)\n", dma ? "LDS DMA (buffer_load_dwordx4 lds)" : "buffer_load_dwordx4 to VGPRs     ",
             waves, 200.0 * 8 * 1024 * waves / t.cycles, t.ghz);
    }
  return 0;
}
