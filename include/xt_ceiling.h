/*
 * Measurement kernels behind bench.py's "attainable" ceilings
 * (libxt_ceiling.so, built beside libxtile_amd.so).  No reference
 * counterpart: the reference publishes no performance figures, so the
 * ceilings that the benchmark's roofline fractions are read against are
 * measured on the box by these kernels, in the same HIP-graph protocol as the
 * tile programs.  Plain C; every function returns 0 on success or a
 * hipError_t value, and enqueues on `stream` (a hipStream_t, NULL: the null
 * stream) without synchronising.
 */
#ifndef XT_CEILING_H
#define XT_CEILING_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming copy of `bytes` (a multiple of 16, both pointers 16-byte
 * aligned): one pass of a grid of 256-thread workgroups, each thread issuing
 * its 16-byte non-temporal loads (two up to 32 MiB, eight beyond) before its
 * first store; arrays of 32 GiB or more by 512 workgroups walking the array.
 * Moves 2 * bytes through HBM. */
int xt_ceiling_copy(const void* src, void* dst, size_t bytes, void* stream);

/* A kernel of `workgroups` 256-thread workgroups that does nothing: the
 * per-launch floor of a graph replay at a given grid size. */
int xt_ceiling_noop(int workgroups, void* stream);

/* One wave that occupies `stream` for `microseconds` (1 to 10^6) of the
 * device's constant-rate wall clock and does nothing else.  Enqueued ahead
 * of a timed run, it lets the host finish enqueuing the run (tens to
 * hundreds of microseconds for a graph of launches) before the first timed
 * kernel starts, so that a short run's events time the kernels and not the
 * host's submission. */
int xt_ceiling_hold(unsigned microseconds, void* stream);

/* Back-to-back MFMAs: `workgroups` workgroups of 4 waves, each wave running
 * `iters` rounds of 8 independent 32x32 MFMAs on fragments it reads once from
 * `operands` (16 bytes per lane per fragment; at least
 * workgroups * 256 * 16 * 16 bytes), then writing one float per lane to
 * `out` (workgroups * 256 floats).  kind 0: v_mfma_f32_32x32x16_f16,
 * 1: v_mfma_f32_32x32x16_bf16, 2: v_mfma_i32_32x32x32_i8.  Work: workgroups
 * * 4 * iters * 8 * 32768 FLOP (65536 OP for i8). */
int xt_ceiling_mfma(const void* operands, float* out, int workgroups, int iters, int kind, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XT_CEILING_H */
