/*
 * xtile_amd C ABI: the boundary between the xtile Python layer and the
 * MI355X runtime (libxtile_amd.so).  Plain C: opaque handles, pointers and
 * sizes; no MLIR, Python or torch types.
 *
 * It replaces the reference's nanobind module `_xtile`
 * (python/XTModule.cpp:210-231), which the Python facade calls from
 * xtile/__init__.py:71,113-157.  Each entry point below names the reference
 * function it stands in for.
 *
 * Ownership: every module owns its own IR (the reference gives every parsed
 * module its own MLIRContext, python/XTModule.cpp:82-126).  Strings returned
 * through `char**` are allocated by the library and released with xt_free().
 * Device buffers are owned by the caller.
 *
 * Errors: every function returning int returns an xt_status; on failure
 * `*err` (when err is non-NULL) receives a newline-joined diagnostic text
 * that the caller must xt_free().
 *
 * Threading: distinct modules are independent and may be used from different
 * threads.  Calls on one module are serialised by a per-module lock.
 */
#ifndef XTILE_AMD_H
#define XTILE_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct xt_module xt_module;

typedef enum xt_status {
  XT_OK = 0,
  XT_ERR_PARSE = 1,       /* text is not a valid xt module (Python: ValueError) */
  XT_ERR_TYPE = 2,        /* wrong object / null handle       (Python: TypeError) */
  XT_ERR_PASS = 3,        /* a pass or verification failed    (Python: RuntimeError) */
  XT_ERR_UNSUPPORTED = 4, /* program has no HIP kernel        (Python: NotImplementedError) */
  XT_ERR_ARGUMENT = 5,    /* buffers do not match the function (Python: ValueError) */
  XT_ERR_DEVICE = 6       /* HIP runtime error                (Python: RuntimeError) */
} xt_status;

/* Release a string returned by this library. */
void xt_free(void* p);

/* Library version string (static, do not free). */
const char* xt_version(void);

/* Parse and verify `len` bytes of xt text into a new module.
 * Replaces `parse` / `_parse_module` (python/XTModule.cpp:112-126), which
 * raised ValueError("failed to parse test module") on failure. */
int xt_module_parse(const char* text, size_t len, xt_module** out, char** err);

/* Destroy a module (the reference's capsule destructor,
 * python/XTModule.cpp:87-110). NULL is ignored. */
void xt_module_free(xt_module* m);

/* Print the module as MLIR-style text.
 * Replaces `_module_asm` (python/XTModule.cpp:228-230). */
int xt_module_print(xt_module* m, char** out_text, char** err);

/* Run one pass in place: "xt-serialize" or "canonicalize".
 * Replaces `xt_serialize` (python/XTModule.cpp:161-167, runPass :128-151);
 * "canonicalize" is the pattern set of lib/xt/XTOps.cpp:399-449. */
int xt_pass_run(xt_module* m, const char* pass, char** err);

/* Number of functions in the module and the name of function `index`
 * (static for the module's lifetime until the next pass; do not free). */
int xt_module_num_funcs(xt_module* m);
const char* xt_module_func_name(xt_module* m, int index);

/* Signature of function `func` (NULL or "" = the only function) as JSON:
 * {"name": ..., "grid": [x,y,z], "args": [{"dtype": "f32", "shape": [..]}, ..]}.
 * No reference counterpart: the reference has no execution, so callers
 * never needed buffer metadata. */
int xt_func_signature(xt_module* m, const char* func, char** out_json, char** err);

/* Plan the HIP launch of `func` without running it: the kernel chosen
 * ("gemm f16->f32 tile=128x128 k=4096 grid=(32,32,1)"), and the algorithmic
 * bytes and FLOPs of one launch.  Stands in for the reference's lowering
 * pipeline `compile` (xtile/__init__.py:160-168), whose x1 command stream the
 * GPU backend replaces with a kernel launch.  A program planned as a fused
 * kernel is compiled here (hiprtc, no GPU needed; cached per process and on
 * disk), so a first call may take a fraction of a second. */
int xt_plan(xt_module* m, const char* func, char** out_desc, double* algo_bytes,
            double* algo_flops, char** err);

/* Launch `func` on the current HIP device.  `bufs[i]` is the device pointer
 * of memref argument i (function argument order, xtile/dsl.py:491-495) and
 * `buf_bytes[i]` its size in bytes; every buffer must hold at least the
 * memref's dense row-major extent.  `stream` is a hipStream_t (NULL: the
 * null stream).  Asynchronous: returns once the kernel is enqueued.
 * No reference counterpart (the reference stops at NPU command text). */
int xt_gpu_run(xt_module* m, const char* func, void* const* bufs, const size_t* buf_bytes,
               int nbufs, void* stream, char** err);

#ifdef __cplusplus
}
#endif

#endif /* XTILE_AMD_H */
