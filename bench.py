"""Benchmark of the xtile_amd HIP path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|c1|..|c10]

One step = one launch of the tile program over one batch of synthetic input
(numpy PCG64, seed = config index, shapes of BASELINE.json's configs).  The
headline line is C2 (row softmax fp32 8192x4096);
the six BASELINE.json configurations (C1-C6), C7 (a row layernorm run as a
fused tile program) and C10 (an attention Block, matmul -> row softmax ->
matmul, run as a staged tile program) are measured and reported under
"per_config".

Order of work: every input is generated on the host first; then the GPU
legs run back to back - the ceiling kernels of include/xt_ceiling.h (an MFMA
loop, a streaming copy, an empty kernel), then each configuration, then the
vendor GEMM - and only then the CPU legs (the oracle), so the GPU is never
left idle between timed regions.

Timing of a configuration: one eager launch whose output is kept as the
reference; for runs of more than 64 launches, K launches captured in a HIP
graph, instantiated and uploaded to the device; ~100 ms of pre-conditioning
work (a ceiling kernel, never the configuration's own); W untimed warm-up
launches; device synchronisation; a hold kernel (one wave waiting a few
hundred microseconds of wall clock) that keeps the stream busy while the host
enqueues the timed launches; then the K launches (the graph's one replay, or
K eager launches for K <= 64) between two HIP events on the launch stream,
and device synchronisation; per-step time = elapsed / K, the events
bracketing exactly the K launches.  Every step reads a different input set
(buffer rotation over >= 1 GiB) so inputs are not left resident in the
256 MB Infinity Cache between steps.  Inputs are in HBM before the timed
region starts; no host transfer is timed.

Checks: the output of input set 0 is cleared after the warm-up, just before
the timed launches; afterwards it must equal the eager reference bit for bit
("replay_equals_eager"), and the reference must match the oracle (the CPU
leg's own output on the same inputs) to the configuration's bar.  A failed
check fails the run: no JSON line is printed and the exit status is 1.

roofline.achieved = algorithmic bytes (or FLOPs) of one launch / per-step
time; roofline.traffic = measured HBM bytes per launch from the rocprofv3
FETCH_SIZE / WRITE_SIZE summaries under profiles/ (null when absent);
roofline.ceiling = what this GPU attains for the same bound in the same run
(the ceiling kernels: C1 against a copy of its own 12.6 MB, the other
bandwidth-bound configurations against a 256 MiB streaming copy, matrix-bound
ones against the MFMA loop of their element type) and roofline.frac_of_ceiling
= achieved / ceiling.

Output: one JSON line on stdout, short enough to survive a tail of a few KB
(per_config holds numbers only); one human-readable line per configuration on
stderr before it; --detail PATH writes every configuration's full record
(timing protocol, CPU sample, ceiling notes).

cpu_baseline = the oracle (oracle/xt_oracle.c, the loop-lowered C executor of
the same xt program) timed on this host's cores over whole repetitions of the
same workload for about --cpu-seconds.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "GB/s (add, softmax) & TFLOP/s (matmul, conv2d) on 1 MI355X, % of roofline"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0, "i8": 5000.0, "f32": 157.3}  # dense; i8 in TOP/s
ROTATE_BYTES = 1 << 30
ALL = ["c1", "c2", "c3", "c4", "c5", "c6", "c7", "c10"]


def _f32(a):
    return np.asarray(a, dtype=np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def make_config(name: str):
    """(module, host inputs, dtypes, out index, meta) for one configuration."""
    from xtile_amd import kernels as K

    if name == "c1":
        rng = np.random.default_rng(1)
        a = _f32(rng.uniform(-1, 1, (1024, 1024)))
        b = _f32(rng.uniform(-1, 1, (1024, 1024)))
        return K.CONFIGS["c1_add"](), [a, b, np.zeros_like(a)], ["f32"] * 3, 2, {
            "workload": "c1_add: C = A + B fp32 1024x1024, 32x64 tiles, grid (32,16,1)",
            "unit": "GB/s", "bound": "hbm", "dtype": "f32", "check": ("exact", 0.0),
            "data": "synthetic: numpy PCG64 seed=1, uniform[-1,1]",
        }
    if name == "c2":
        rng = np.random.default_rng(2)
        x = _f32(rng.normal(0.0, 2.0, (8192, 4096)))
        return K.CONFIGS["c2_softmax"](), [x, np.zeros_like(x)], ["f32"] * 2, 1, {
            "workload": "c2_softmax: row softmax fp32 8192x4096, one 1x4096 row per Block, grid (8192,1,1)",
            "unit": "GB/s", "bound": "hbm", "dtype": "f32", "check": ("max_rel", 1e-5),
            "data": "synthetic: numpy PCG64 seed=2, normal(0,2)",
        }
    if name == "c7":
        rng = np.random.default_rng(7)
        x = _f32(rng.normal(0.0, 1.5, (8192, 4096)))
        g = _f32(rng.normal(1.0, 0.2, (1, 4096)))
        b = _f32(rng.normal(0.0, 0.2, (1, 4096)))
        n = np.full((1, 1), 1.0 / 4096, np.float32)
        e = np.full((1, 1), 1e-5, np.float32)
        return K.layernorm(8192, 4096, 1), [x, g, b, n, e, np.zeros_like(x)], ["f32"] * 6, 5, {
            "workload": "c7_layernorm: row layernorm fp32 8192x4096 (a program outside the four benchmark "
                        "families, run as a fused tile program), one 1x4096 row per Block, grid (8192,1,1)",
            "unit": "GB/s", "bound": "hbm", "dtype": "f32", "check": ("max_abs", 5e-5),
            "data": "synthetic: numpy PCG64 seed=7, x normal(0,1.5), gamma normal(1,0.2), beta normal(0,0.2)",
        }
    if name == "c3":
        rng = np.random.default_rng(3)
        a = rng.uniform(-1, 1, (4096, 4096)).astype(np.float16)
        b = rng.uniform(-1, 1, (4096, 4096)).astype(np.float16)
        return K.CONFIGS["c3_matmul_f16"](), [a, b, np.zeros((4096, 4096), np.float32)], [
            "f16", "f16", "f32"], 2, {
            "workload": "c3_matmul_f16: C = A @ B, M=N=K=4096, f16 in, f32 acc/out, 128x128 Block tiles, "
                        "B shared=1, grid (32,32,1)",
            "unit": "TFLOP/s", "bound": "mfma", "dtype": "f16", "check": ("frob", 1e-3),
            "data": "synthetic: numpy PCG64 seed=3, uniform[-1,1] -> f16",
        }
    if name == "c4":
        rng = np.random.default_rng(4)
        x = rng.normal(0, 0.1, (32, 56, 56, 64)).astype(np.float16)
        f = rng.normal(0, 0.1, (3, 3, 64, 64)).astype(np.float16)
        return K.CONFIGS["c4_conv2d_f16"](), [x, f, np.zeros((32, 56, 56, 64), np.float32)], [
            "f16", "f16", "f32"], 2, {
            "workload": "c4_conv2d_f16: NHWC 32x56x56x64 * 3x3x64x64, stride 1, pad 1, f16 in, f32 out, "
                        "1x4x56x64 Block tiles, filter shared=2, grid (32,14,1)",
            "unit": "TFLOP/s", "bound": "hbm", "dtype": "f16", "check": ("frob", 1e-3),
            "data": "synthetic: numpy PCG64 seed=4, normal(0,0.1) -> f16",
        }
    if name == "c8":
        rng = np.random.default_rng(8)
        x = rng.normal(0, 0.5, (32, 224, 224, 3)).astype(np.float16)
        f = rng.normal(0, 0.1, (7, 7, 3, 64)).astype(np.float16)
        return K.conv2d(32, 224, 224, 3, 64, 7, 7, 4, 112, pad=(3, 3, 3, 3), stride=(2, 2)), [
            x, f, np.zeros((32, 112, 112, 64), np.float32)], ["f16", "f16", "f32"], 2, {
            "workload": "c8_conv2d_stem_f16 (outside the five reference configurations: a 3-channel stem): NHWC "
                        "32x224x224x3 * 7x7x3x64, stride 2, pad 3, f16 in, f32 out, 1x4x112x64 Block tiles, filter "
                        "shared=2, grid (32,28,1)",
            "unit": "TFLOP/s", "bound": "hbm", "dtype": "f16", "check": ("frob", 1e-3),
            "data": "synthetic: numpy PCG64 seed=8, input normal(0,0.5), filter normal(0,0.1) -> f16",
        }
    if name == "c9":
        rng = np.random.default_rng(9)
        x = rng.normal(0, 0.1, (32, 14, 14, 256)).astype(np.float16)
        f = rng.normal(0, 0.1, (3, 3, 256, 256)).astype(np.float16)
        return K.conv2d(32, 14, 14, 256, 256, 3, 3, 2, 14), [
            x, f, np.zeros((32, 14, 14, 256), np.float32)], ["f16", "f16", "f32"], 2, {
            "workload": "c9_conv2d_deep_f16 (outside the five reference configurations: a deep layer whose filter "
                        "exceeds the band kernel's LDS): NHWC 32x14x14x256 * 3x3x256x256, stride 1, pad 1, f16 in, "
                        "f32 out, 1x2x14x256 Block tiles, filter shared=2, grid (32,7,1)",
            "unit": "TFLOP/s", "bound": "mfma", "dtype": "f16", "check": ("frob", 1e-3),
            "data": "synthetic: numpy PCG64 seed=9, normal(0,0.1) -> f16",
        }
    if name == "c10":
        rng = np.random.default_rng(10)
        heads, nq, nk, d, tq = 1024, 64, 64, 64, 64
        q = rng.normal(0, 0.5, (heads, nq, d)).astype(np.float16)
        k = rng.normal(0, 0.5, (heads, nk, d)).astype(np.float16)
        v = _f32(rng.normal(0, 1.0, (heads, nk, d)))
        return K.attention(heads, nq, nk, d, tq), [q, k, v, np.zeros((heads, nq, d), np.float32)], [
            "f16", "f16", "f32", "f32"], 3, {
            "workload": "c10_attention (outside the five reference configurations: a program with matmul, "
                        "transpose and row softmax in one Block, on the staged kernel): softmax(Q K^T) V, 1024 "
                        "heads x 64 queries x 64 keys, d=64, Q/K f16, V and result f32, one 64-query tile per "
                        "head, K/V shared=1, grid (1,1024,1)",
            "unit": "TFLOP/s", "bound": "mixed", "dtype": "f16+f32", "check": ("frob", 1e-5),
            "data": "synthetic: numpy PCG64 seed=10, Q,K normal(0,0.5) -> f16, V normal(0,1)",
            # the f16 product Q K^T and the f32 product P V, in FLOPs per launch
            "flops_by_type": {"f16": 2.0 * heads * nq * nk * d, "f32": 2.0 * heads * nq * nk * d},
        }
    if name == "c5":
        rng = np.random.default_rng(5)
        a = bf16_bits(_f32(rng.normal(0, 0.02, (4096, 4096))))
        b = bf16_bits(_f32(rng.normal(0, 0.02, (4096, 11008))))
        return K.CONFIGS["c5_matmul_bf16"](), [a, b, np.zeros((4096, 11008), np.float32)], [
            "bf16", "bf16", "f32"], 2, {
            "workload": "c5_matmul_bf16: C = A @ B, M=4096 N=11008 K=4096, bf16 in (RNE), f32 out, "
                        "256x128 Block tiles, A shared=1, grid (86,16,1)",
            "unit": "TFLOP/s", "bound": "mfma", "dtype": "bf16", "check": ("frob", 1e-3),
            "data": "synthetic: numpy PCG64 seed=5, normal(0,0.02) -> bf16 (RNE)",
        }
    if name == "c6":
        rng = np.random.default_rng(6)
        m = n = k = 4096
        a = rng.integers(-128, 128, (m, k), dtype=np.int8)
        b = rng.integers(-128, 128, (k, n), dtype=np.int8)
        s = _f32(rng.uniform(0.5, 2.0, (1, n)) / (np.sqrt(k) * 64))
        bias = _f32(rng.uniform(-20, 20, (1, n)))
        return K.CONFIGS["c6_matmul_i8"](), [a, b, np.zeros((m, n), np.int8), s, bias], [
            "i8", "i8", "i8", "f32", "f32"], 2, {
            "workload": "c6_matmul_i8: kernels/matmul.py, C = int8(A @ B * scale + bias), M=N=K=4096, "
                        "i8 in, i32 acc, f32 epilogue, i8 out, 64x64 Block tiles, B/scale/bias shared=1, grid (64,64,1)",
            "unit": "TOP/s", "bound": "mfma", "dtype": "i8", "check": ("exact", 0.0),
            "data": "synthetic: numpy PCG64 seed=6, A,B uniform int8, scale ~U[0.5,2]/(64 sqrt(K)), bias ~U[-20,20]",
        }
    raise ValueError(f"unknown config {name}")


def _traffic(name: str):
    """HBM bytes per launch from the profiles/<config>_*.txt summary (fetch + write)."""
    paths = sorted((ROOT / "profiles").glob(f"{name}_*.txt"))
    if not paths:
        return None
    vals = {}
    for line in paths[0].read_text().splitlines():
        m = re.match(r"\s*(fetch_bytes|write_bytes)\s*[:=]\s*([0-9.eE+]+)", line)
        if m:
            vals[m.group(1)] = float(m.group(2))
    if "fetch_bytes" in vals and "write_bytes" in vals:
        return vals["fetch_bytes"] + vals["write_bytes"]
    return None


# -- device helpers ------------------------------------------------------------------


def to_device(arr: np.ndarray, dtype: str, device):
    import torch

    if dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16).to(device)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


def to_host(t, dtype: str) -> np.ndarray:
    import torch

    t = t.detach().cpu()
    if dtype == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def torch_uint8():
    import torch

    return torch.uint8


_HIP = None


def _hip():
    """The HIP runtime torch loaded (one runtime per process)."""
    global _HIP
    if _HIP is None:
        import torch

        _HIP = ctypes.CDLL(str(Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"))
        vp, pp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        for name, args in {"hipStreamBeginCapture": [vp, ctypes.c_int], "hipStreamEndCapture": [vp, pp],
                           "hipGraphInstantiate": [pp, vp, vp, vp, ctypes.c_size_t],
                           "hipGraphUpload": [vp, vp], "hipGraphLaunch": [vp, vp],
                           "hipGraphExecDestroy": [vp], "hipGraphDestroy": [vp]}.items():
            getattr(_HIP, name).argtypes = args
            getattr(_HIP, name).restype = ctypes.c_int
    return _HIP


class HipGraph:
    """`steps` launches captured from `stream` into a HIP graph, instantiated
    and uploaded to the device before anything is timed.  A graph that is not
    uploaded pays a one-time setup on its first launch (20-60 us per 20-launch
    graph on MI355X), which would otherwise land in a short timed region."""

    def __init__(self, launch, n_sets: int, steps: int, stream):
        hip = _hip()
        self.stream = ctypes.c_void_p(stream.cuda_stream)
        self.graph, self.exe = ctypes.c_void_p(), ctypes.c_void_p()
        self._ok(hip.hipStreamBeginCapture(self.stream, 2), "hipStreamBeginCapture")  # relaxed mode
        try:
            for i in range(steps):
                launch(i % n_sets)
        finally:
            rc = hip.hipStreamEndCapture(self.stream, ctypes.byref(self.graph))
        self._ok(rc, "hipStreamEndCapture")
        self._ok(hip.hipGraphInstantiate(ctypes.byref(self.exe), self.graph, None, None, 0), "hipGraphInstantiate")
        self._ok(hip.hipGraphUpload(self.exe, self.stream), "hipGraphUpload")

    @staticmethod
    def _ok(rc, what):
        if rc:
            raise RuntimeError(f"{what} failed (hipError {rc})")

    def replay(self):
        self._ok(_hip().hipGraphLaunch(self.exe, self.stream), "hipGraphLaunch")

    def __del__(self):
        hip = _HIP
        if hip is not None:
            if getattr(self, "exe", None) and self.exe.value:
                hip.hipGraphExecDestroy(self.exe)
            if getattr(self, "graph", None) and self.graph.value:
                hip.hipGraphDestroy(self.graph)


# Runs of at most this many launches are timed as eager launches queued
# behind the hold kernel; longer runs as one replay of an uploaded HIP graph.
EAGER_MAX_STEPS = 64


def hold_us(steps: int, eager: bool) -> int:
    """Length of the hold kernel ahead of a timed run of `steps` launches:
    longer than the host takes to enqueue them.  On the MI355X boxes a
    20-launch graph takes 40-170 us to submit and a 2000-launch one ~1.1 ms;
    an eager launch through xt.launch ~17 us."""
    return min(5000, 500 + 40 * steps) if eager else min(10**6, 500 + steps)


def hold(stream, us: int) -> None:
    rc = _ceiling_lib().xt_ceiling_hold(us, stream.cuda_stream)
    if rc:
        raise RuntimeError(f"hold kernel launch failed (hipError {rc})")


def timed(launch, n_sets: int, steps: int, warmup: int, stream, use_graph: bool, before_replay=None,
          precondition=None):
    """(average ms per launch of `launch(i)` over `steps` launches, i = input
    set; description of how they were timed).

    Runs of more than EAGER_MAX_STEPS launches are captured in a HIP graph and
    uploaded first (capture runs nothing).  Then, on `stream`: the optional
    `precondition()` work, `warmup` untimed eager launches and
    `before_replay()`; a device synchronisation; the hold kernel
    (xt_ceiling_hold); the start event, the timed launches (the graph's one
    replay, or the eager launches), the end event; a device synchronisation.

    The hold keeps the stream busy while the host enqueues the timed launches,
    so the start event fires when they are already queued and the events time
    the kernels, not the host's submission: without it a 20-launch C1 run
    measured 6.4-9.2 us per launch, against 4.1-4.5 us with it and 3.7-4.1 over
    2000 launches.  Short runs use eager launches because a graph's first
    replay costs each short launch about 0.3-0.4 us more than its later
    replays (C1, 20 launches: 4.55-4.65 us per launch on the first replay,
    4.13-4.17 eager behind the hold, 4.20-4.24 on a second replay; C2 and C4
    by 0.2-0.6 us), and a timed run replays its graph once; long runs use the
    graph, because a long queue of eager launches runs slower than a replay
    (C2, 200 launches: 44.9-45.7 us eager, 43.6-44.2 replayed)."""
    import time

    import torch

    eager = not use_graph or steps <= EAGER_MAX_STEPS
    graph, mode = None, "eager launches"
    if not eager:
        try:
            graph = HipGraph(launch, n_sets, steps, stream)
            mode = "one replay of a HIP graph uploaded before timing"
        except Exception as exc:  # capture unsupported: time eager launches
            print(f"[bench] graph capture failed ({exc}); timing eager launches", file=sys.stderr)
            eager = True
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        if precondition is not None:
            precondition()
        for i in range(warmup):
            launch(i % n_sets)
        if before_replay is not None:
            before_replay()
    torch.cuda.synchronize()
    us = hold_us(steps, eager)
    with torch.cuda.stream(stream):
        hold(stream, us)
        start.record(stream)
        t0 = time.perf_counter()
        if graph is not None:
            graph.replay()
        else:
            for i in range(steps):
                launch(i % n_sets)
        t1 = time.perf_counter()
        end.record(stream)
    torch.cuda.synchronize()
    enq = (t1 - t0) * 1e6
    if enq > us:
        print(f"[bench] the host took {enq:.0f} us to enqueue {steps} launches, longer than the {us} us hold: "
              "the timed region includes host submission", file=sys.stderr)
    mode += f" behind a {us} us hold kernel (host enqueue {enq:.0f} us)"
    return start.elapsed_time(end) / steps, mode


class Preconditioner:
    """Brings the GPU to the clock it sustains under a configuration's kind of
    load before that configuration is timed.  The power manager ramps the
    clock over the first ~30 ms of matrix-core load, and restarts the ramp
    after even 50 ms of idle: the first 20 launches of C3 take 170-180 us,
    the 200th 142 us.  Short timed runs (the driver's 20 steps) would
    otherwise measure the ramp.  The work is one of the ceiling kernels of
    include/xt_ceiling.h (never the configuration's own kernel), enqueued on
    the timing stream right before the warm-up launches."""

    MS = 100.0

    def __init__(self):
        import torch

        self.lib = _ceiling_lib()
        self.dev = torch.device("cuda:0")
        self.wgs = 512
        self.ops = {}
        self.res = torch.empty(self.wgs * 256, dtype=torch.float32, device=self.dev)
        n = 256 << 20
        self.copy_bytes = n
        self.src = torch.empty(n, dtype=torch.uint8, device=self.dev).random_()
        self.dst = torch.empty_like(self.src)

    def operands(self, kind: str):
        import torch

        if kind not in self.ops:
            rng = np.random.default_rng(11)
            nvals = self.wgs * 256 * 16 * 16
            if kind == "f16":
                h = rng.uniform(-1, 1, nvals // 2).astype(np.float16).view(np.uint8)
            elif kind == "bf16":
                h = bf16_bits(_f32(rng.normal(0, 0.02, nvals // 2))).view(np.uint8)
            else:
                h = rng.integers(-128, 128, nvals, dtype=np.int8).view(np.uint8)
            self.ops[kind] = torch.from_numpy(h).to(self.dev)
        return self.ops[kind]

    def mfma(self, kind: str, iters: int, stream_handle):
        k = {"f16": 0, "bf16": 1, "i8": 2}[kind]
        rc = self.lib.xt_ceiling_mfma(self.operands(kind).data_ptr(), self.res.data_ptr(), self.wgs, iters, k,
                                      stream_handle)
        if rc:
            raise RuntimeError(f"ceiling MFMA launch failed (hipError {rc})")

    def copy(self, src, dst, nbytes, stream_handle):
        rc = self.lib.xt_ceiling_copy(src, dst, nbytes, stream_handle)
        if rc:
            raise RuntimeError(f"ceiling copy launch failed (hipError {rc})")

    @staticmethod
    def touch(sets) -> None:
        """Reads one byte of every 64 KB of every rotating input set, in the
        order the timed launches use them, so that their page translations
        are warm (a short timed run otherwise pays a TLB miss on each page it
        is the first to touch since the sets were written) while almost none
        of their data enters the 256 MB Infinity Cache."""
        for st in sets:
            for t in st:
                t.view(-1).view(torch_uint8())[::65536].sum()

    def run(self, bound: str, dtype: str, stream) -> None:
        """About MS milliseconds of MFMA loop (matrix-bound configurations) or
        streaming copy (bandwidth-bound ones) on `stream`."""
        h = stream.cuda_stream
        if bound == "mfma":
            for _ in range(int(self.MS / 1.4)):  # one 4000-round launch is about 1.4 ms
                self.mfma(dtype, 4000, h)
        else:
            for _ in range(int(self.MS / 0.09)):  # one 256 MiB copy is about 90 us
                self.copy(self.src.data_ptr(), self.dst.data_ptr(), self.copy_bytes, h)


def alloc_sets(cfg) -> list:
    """The configuration's rotating input sets (>= ROTATE_BYTES in all), on
    the GPU.  main() allocates every configuration's sets before anything
    else: C4's 20-launch figure read 13.1-13.4 us on sets allocated before the
    pre-conditioning buffers and 15.0-15.5 us on sets allocated after them
    (the 2000-launch figure is the same either way)."""
    import torch

    module, host, dtypes, out, meta = cfg
    dev = torch.device("cuda:0")
    set_bytes = sum(h.nbytes for h in host)
    nsets = max(1, min(128, math.ceil(ROTATE_BYTES / set_bytes)))
    first = [to_device(h, d, dev) for h, d in zip(host, dtypes)]
    sets = [first] + [[t.clone() for t in first] for _ in range(nsets - 1)]
    torch.cuda.synchronize()
    return sets


def gpu_leg(name: str, cfg, sets: list, steps: int, warmup: int, use_graph: bool,
            pre: "Preconditioner | None") -> dict:
    import torch

    import xtile_amd as xt

    module, host, dtypes, out, meta = cfg
    plan = xt.plan(module)
    print(f"[bench] {name}: {plan['kernel']}", file=sys.stderr, flush=True)
    dev = torch.device("cuda:0")
    nsets = len(sets)
    stream = torch.cuda.Stream(device=dev)

    def launch(i):
        xt.launch(module, *sets[i], stream=stream)

    # eager reference of set 0; its output is cleared again just before the
    # timed region, so only the timed launches can have rewritten it
    with torch.cuda.stream(stream):
        launch(0)
    torch.cuda.synchronize()
    reference = to_host(sets[0][out], dtypes[out])

    def clear():
        sets[0][out].zero_()

    def precondition():
        pre.run(meta["bound"], meta["dtype"], stream)
        pre.touch(sets)

    ms, mode = timed(launch, nsets, steps, warmup, stream, use_graph, before_replay=clear,
                     precondition=precondition if pre is not None else None)
    replay = to_host(sets[0][out], dtypes[out])
    replay_ok = bool(np.array_equal(replay.view(np.uint8), reference.view(np.uint8)))
    sets.clear()
    torch.cuda.empty_cache()
    sec = ms * 1e-3
    value = plan["bytes"] / sec / 1e9 if meta["unit"] == "GB/s" else plan["flops"] / sec / 1e12
    if meta["bound"] == "mixed":
        # the ideal time is the longer of the HBM time of the algorithmic bytes
        # and the matrix time of each element type's FLOPs at its dense peak
        t_hbm = plan["bytes"] / (HBM_PEAK_GBS * 1e9)
        t_mm = sum(f / (MFMA_PEAK_TFLOPS[t] * 1e12) for t, f in meta["flops_by_type"].items())
        ideal = max(t_hbm, t_mm)
        achieved = plan["flops"] / sec / 1e12
        roof = {"bound": "mfma" if t_mm >= t_hbm else "hbm", "achieved": achieved,
                "peak": plan["flops"] / ideal / 1e12, "unit": "TFLOP/s", "frac": ideal / sec,
                "traffic": _traffic(name), "hbm_GBs": plan["bytes"] / sec / 1e9,
                "peak_note": "FLOPs / the ideal time max(bytes / 8 TB/s, f16 FLOPs / 2.5 PF + f32 FLOPs / 157.3 TF)"}
    elif meta["bound"] == "hbm":
        achieved = plan["bytes"] / sec / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": _traffic(name)}
    else:
        achieved = plan["flops"] / sec / 1e12
        peak = MFMA_PEAK_TFLOPS[meta["dtype"]]
        roof = {"bound": "mfma", "achieved": achieved, "peak": peak,
                "unit": "TOP/s" if meta["dtype"] == "i8" else "TFLOP/s",
                "frac": achieved / peak, "traffic": _traffic(name)}
    if name in ("c4", "c8"):  # report against the MFMA peak as well
        tf = plan["flops"] / sec / 1e12
        roof["mfma_tflops"] = tf
        roof["mfma_frac"] = tf / MFMA_PEAK_TFLOPS["f16"]
    return {
        "config": name,
        "workload": meta["workload"],
        "kernel": plan["kernel"],
        "value": value,
        "unit": meta["unit"],
        "ms_per_step": ms,
        "dtype": meta["dtype"],
        "data": meta["data"],
        "timing": f"{steps} {mode}, after {warmup} warm-up, {nsets} rotating input sets"
                  + (f", after {Preconditioner.MS:.0f} ms of device pre-conditioning ("
                     + ("MFMA loop" if meta["bound"] == "mfma" else "streaming copy")
                     + ", include/xt_ceiling.h) and a page-touch of every input set" if pre is not None else ""),
        "roofline": roof,
        "algo_bytes": plan["bytes"],
        "algo_flops": plan["flops"],
        "check": {"replay_equals_eager": replay_ok},
        "_reference": reference,
    }


_CEILING_LIB = None


def _ceiling_lib():
    global _CEILING_LIB
    if _CEILING_LIB is None:
        lib = ctypes.CDLL(str(ROOT / "xtile_amd" / "lib" / "libxt_ceiling.so"))
        lib.xt_ceiling_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.xt_ceiling_noop.argtypes = [ctypes.c_int, ctypes.c_void_p]
        lib.xt_ceiling_mfma.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_void_p]
        lib.xt_ceiling_hold.argtypes = [ctypes.c_uint, ctypes.c_void_p]
        for f in (lib.xt_ceiling_copy, lib.xt_ceiling_noop, lib.xt_ceiling_mfma, lib.xt_ceiling_hold):
            f.restype = ctypes.c_int
        _CEILING_LIB = lib
    return _CEILING_LIB


def ceilings(pre: Preconditioner) -> dict:
    """What this GPU attains, measured by the kernels of include/xt_ceiling.h
    in the same graph protocol as the tile programs: an MFMA issue loop per
    element type on the configurations' own operand distributions, a 256 MiB
    streaming copy (read + write, rotated over 2 GiB) and a copy and an empty
    kernel at C1's size (the launch floor of a 12.6 MB program).  Each is
    preceded by the same pre-conditioning as the configurations."""
    import torch

    dev = pre.dev
    stream = torch.cuda.Stream(device=dev)
    h = stream.cuda_stream
    out = {}
    iters = 40000
    for name in ("f16", "bf16", "i8"):
        ms, _ = timed(lambda i: pre.mfma(name, iters, h), 1, 4, 1, stream, True,
                      precondition=lambda: pre.run("mfma", name, stream))
        work = pre.wgs * 4 * iters * 8 * 32768 * (2 if name == "i8" else 1)
        out[f"mfma_{name}_T{'OP' if name == 'i8' else 'FLOP'}s"] = work / (ms * 1e-3) / 1e12
    # HBM streaming copy, 256 MiB, four pairs rotated
    n = 256 << 20
    src = [torch.empty(n, dtype=torch.uint8, device=dev).random_() for _ in range(4)]
    dst = [torch.empty_like(t) for t in src]
    ms, _ = timed(lambda i: pre.copy(src[i].data_ptr(), dst[i].data_ptr(), n, h), 4, 100, 10, stream, True,
                  precondition=lambda: pre.run("hbm", "f32", stream))
    out["hbm_copy_GBs"] = 2 * n / (ms * 1e-3) / 1e9
    del src, dst
    # C1's size: 12,582,912 bytes moved per launch (a 6 MiB copy), rotated over 86 pairs like C1's inputs
    n = 6 << 20
    src = [torch.empty(n, dtype=torch.uint8, device=dev).random_() for _ in range(86)]
    dst = [torch.empty_like(t) for t in src]
    ms, _ = timed(lambda i: pre.copy(src[i].data_ptr(), dst[i].data_ptr(), n, h), 86, 2000, 100, stream, True,
                  precondition=lambda: pre.run("hbm", "f32", stream))
    out["c1_size_copy_us"] = ms * 1e3
    out["c1_size_copy_GBs"] = 2 * n / (ms * 1e-3) / 1e9
    del src, dst

    def noop(i):
        rc = pre.lib.xt_ceiling_noop(512, h)
        if rc:
            raise RuntimeError(f"ceiling launch failed (hipError {rc})")

    ms, _ = timed(noop, 1, 2000, 100, stream, True)
    out["empty_kernel_512wg_us"] = ms * 1e3
    torch.cuda.empty_cache()
    out["note"] = ("include/xt_ceiling.h kernels, HIP graph replay: MFMA loop of 8 independent 32x32 MFMAs per "
                   "wave, 8 waves per CU, operands distributed like C3 (f16), C5 (bf16), C6 (i8); non-temporal "
                   "float4 copy, one pass of a full grid (eight vectors a thread at 256 MiB, two at C1's size); "
                   "empty kernel of 512 workgroups (C1's grid)")
    return out


def vendor(pre: "Preconditioner | None") -> dict:
    """hipBLASLt through torch on the GEMM configurations' shapes and types,
    in the same process and the same protocol as the configurations: the MFMA
    pre-conditioning loop, 10 warm-up calls, then 50 calls queued behind the
    hold kernel between two events (on a side stream)."""
    import torch

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    out = {}

    def rate(fn, flops, n=50, kind="f16"):
        precondition = (lambda: pre.run("mfma", kind, stream)) if pre is not None else None
        ms, _ = timed(lambda i: fn(), 1, n, 10, stream, True, precondition=precondition)
        return flops / (ms * 1e-3) / 1e12

    a = (torch.rand(4096, 4096, device=dev) * 2 - 1).half()
    b = (torch.rand(4096, 4096, device=dev) * 2 - 1).half()
    f = 2 * 4096**3
    out["hipblaslt_f16_4096_f16out_TFLOPs"] = rate(lambda: torch.mm(a, b), f)
    try:
        out["hipblaslt_f16_4096_f32out_TFLOPs"] = rate(lambda: torch.mm(a, b, out_dtype=torch.float32), f)
    except Exception as exc:  # the out_dtype overload is missing on some builds
        out["hipblaslt_f16_4096_f32out_TFLOPs"] = None
        out["f32out_error"] = str(exc)[:200]
    a = (torch.randn(4096, 4096, device=dev) * 0.02).bfloat16()
    b = (torch.randn(4096, 11008, device=dev) * 0.02).bfloat16()
    f = 2 * 4096 * 4096 * 11008
    out["hipblaslt_bf16_c5_bf16out_TFLOPs"] = rate(lambda: torch.mm(a, b), f, kind="bf16")
    try:
        out["hipblaslt_bf16_c5_f32out_TFLOPs"] = rate(lambda: torch.mm(a, b, out_dtype=torch.float32), f, kind="bf16")
    except Exception:
        out["hipblaslt_bf16_c5_f32out_TFLOPs"] = None
    a = torch.randint(-128, 128, (4096, 4096), dtype=torch.int8, device=dev)
    b = torch.randint(-128, 128, (4096, 4096), dtype=torch.int8, device=dev)
    try:
        out["hipblaslt_i8_4096_i32out_TOPs"] = rate(lambda: torch._int_mm(a, b), 2 * 4096**3, kind="i8")
    except Exception as exc:
        out["hipblaslt_i8_4096_i32out_TOPs"] = None
        out["i8_error"] = str(exc)[:200]
    del a, b
    torch.cuda.empty_cache()
    out["note"] = ("torch.mm (hipBLASLt); f32out = torch.mm(..., out_dtype=torch.float32), the configurations' own "
                   "types; i8 = torch._int_mm (i32 out, no epilogue); the same operands every call (no rotation); "
                   "MFMA pre-conditioning, 10 warm-up calls, 50 timed calls queued behind the hold kernel")
    return out


# -- CPU leg: the oracle as baseline and checker ---------------------------------------


def cpu_time(text: str, host, seconds: float, threads: int):
    """(seconds per run, repetitions, buffers after the first run) of the
    oracle over whole repetitions of `text`."""
    import oracle

    bufs = [np.array(h, copy=True) for h in host]
    first = None
    reps = 0
    t0 = time.perf_counter()
    while True:
        oracle.run(text, bufs, threads)
        if first is None:
            first = [np.array(b, copy=True) for b in bufs]
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return elapsed / reps, reps, first


_GRID = re.compile(r"xt\.grid = array<i32: (\d+), (\d+), (\d+)>")


def grid_subset(text: str, fraction: float):
    """The same program over a leading sub-grid holding about `fraction` of
    the Blocks (Blocks are independent and do equal work, so the rate per
    Block is that of the whole grid).  Returns (text, share of Blocks run)."""
    m = _GRID.search(text)
    g = [int(v) for v in m.groups()]
    axis = max(range(3), key=lambda a: g[a])
    keep = max(1, min(g[axis], math.ceil(g[axis] * fraction)))
    share = keep / g[axis]
    g[axis] = keep
    return text[: m.start()] + f"xt.grid = array<i32: {g[0]}, {g[1]}, {g[2]}>" + text[m.end():], share


def compare(kind: str, bar: float, got: np.ndarray, want: np.ndarray, dtype: str) -> tuple[bool, float]:
    if kind == "exact":
        return bool(np.array_equal(got.view(np.uint8), want.view(np.uint8))), 0.0
    if dtype == "bf16":
        got, want = (np.asarray(x, np.uint32) << 16 for x in (got, want))
        got, want = got.view(np.float32), want.view(np.float32)
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    if kind == "max_rel":
        err = float(np.max(np.abs(g - w) / np.maximum(np.abs(w), np.finfo(np.float32).tiny)))
    elif kind == "max_abs":
        err = float(np.max(np.abs(g - w)))
    else:
        err = float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-300))
    return err <= bar, err


def cpu_leg(name: str, cfg, result: dict, cpu_seconds: float) -> None:
    module, host, dtypes, out, meta = cfg
    threads = int(os.environ.get("XT_CPU_THREADS", min(16, os.cpu_count() or 1)))
    text = str(module)
    work = result["algo_bytes"] if meta["unit"] == "GB/s" else result["algo_flops"]
    scale = 1e9 if meta["unit"] == "GB/s" else 1e12
    print(f"[bench] {name}: oracle on {threads} threads", file=sys.stderr, flush=True)
    cpu_s, reps, first = cpu_time(text, host, cpu_seconds, threads)
    kind, bar = meta["check"]
    ok, err = compare(kind, bar, result["_reference"], first[out], dtypes[out])
    result["check"].update({"vs_oracle": kind, "bar": bar, "error": err, "ok": ok})
    # one thread, on a sub-grid sized to about 2 s
    sub, share = grid_subset(text, min(1.0, 2.0 / max(cpu_s * threads, 1e-9)))
    one_s, one_reps, _ = cpu_time(sub, host, 0.5, 1)
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    result["cpu_baseline"] = {
        "value": work / cpu_s / scale,
        "unit": meta["unit"],
        "cores": threads,
        "kind": "port",
        "sample": f"oracle/xt_oracle.c over the full workload, {reps} repetition(s), "
                  f"{cpu_s * 1e3:.1f} ms each, {threads} OpenMP threads (nproc={os.cpu_count()}, "
                  f"affinity={affinity})",
        "value_1thread": work * share / one_s / scale,
        "sample_1thread": f"{share:.4f} of the Blocks (a leading sub-grid), {one_reps} repetition(s), "
                          f"{one_s * 1e3:.1f} ms each, 1 thread",
    }


# -- the printed line ------------------------------------------------------------


def ceiling_of(result: dict, ceil: dict) -> None:
    """Adds roofline.ceiling (what this GPU attains for the configuration's
    bound, measured in the same run by the kernels of include/xt_ceiling.h)
    and roofline.frac_of_ceiling = achieved / ceiling.  C1's ceiling is a copy
    of C1's own byte count (the launch floor of a 12.6 MB program); the other
    bandwidth-bound configurations take the 256 MiB streaming copy; matrix-bound
    ones the MFMA loop of their element type."""
    roof = result["roofline"]
    if "peak_note" in roof:  # a mix of element types: the ideal time is the ceiling itself
        return
    if roof["bound"] == "hbm":
        if result["config"] == "c1":
            c, what = ceil["c1_size_copy_GBs"], "copy of C1's 12.6 MB"
        else:
            c, what = ceil["hbm_copy_GBs"], "256 MiB streaming copy"
    else:
        key = {"f16": "mfma_f16_TFLOPs", "bf16": "mfma_bf16_TFLOPs", "i8": "mfma_i8_TOPs"}[result["dtype"]]
        c, what = ceil[key], f"{result['dtype']} MFMA loop"
    roof["ceiling"] = c
    roof["ceiling_kind"] = what
    roof["frac_of_ceiling"] = roof["achieved"] / c


def _r(x, digits=4):
    """Round a float to `digits` significant digits for the printed line."""
    if isinstance(x, float) and math.isfinite(x) and x != 0.0:
        return float(f"{x:.{digits}g}")
    return x


def compact(d):
    """Numbers of a ceiling / vendor record, without its prose note."""
    if d is None:
        return None
    return {k: _r(v) for k, v in d.items() if k not in ("note",) and not k.endswith("_error")}


def compact_config(r: dict) -> dict:
    roof = r["roofline"]
    chk = r["check"]
    out = {
        "kernel": r["kernel"],
        "value": _r(r["value"]),
        "unit": r["unit"],
        "us_per_step": _r(r["ms_per_step"] * 1e3),
        "bound": roof["bound"],
        "frac": _r(roof["frac"], 3),
        "frac_of_ceiling": _r(roof.get("frac_of_ceiling"), 3),
        "traffic": roof.get("traffic"),
        "check": {"replay_equals_eager": chk["replay_equals_eager"], **(
            {"vs_oracle": chk["vs_oracle"], "error": _r(chk["error"], 3), "bar": chk["bar"], "ok": chk["ok"]}
            if "ok" in chk else {})},
    }
    if "mfma_frac" in roof:
        out["mfma_frac"] = _r(roof["mfma_frac"], 3)
    cpu = r.get("cpu_baseline")
    if cpu:
        out["cpu"] = {"value": _r(cpu["value"]), "cores": cpu["cores"], "value_1thread": _r(cpu["value_1thread"])}
    return out


def summary_line(r: dict) -> str:
    roof = r["roofline"]
    s = (f"{r['config']}: {r['ms_per_step'] * 1e3:8.2f} us/launch  {r['value']:9.1f} {r['unit']:7s} "
         f"{roof['frac']:.3f} of peak")
    if roof.get("frac_of_ceiling") is not None:
        s += f", {roof['frac_of_ceiling']:.3f} of the {roof['ceiling_kind']}"
    if "mfma_frac" in roof:
        s += f", {roof['mfma_frac']:.3f} of f16 MFMA peak"
    chk = r["check"]
    if "ok" in chk:
        s += f"; {chk['vs_oracle']} error {chk['error']:.2e} (bar {chk['bar']:g}) {'ok' if chk['ok'] else 'FAILED'}"
    return s + f"  [{r['kernel']}]"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 2000 launches keep every timed region >= 7 ms (C1) and the clock settled
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="all",
                    help="all (c1..c7 and c10), or a comma-separated list of c1..c10 (c8, c9: conv layers outside "
                         "the reference configurations, run only when named)")
    ap.add_argument("--cpu-seconds", type=float, default=5.0,
                    help="oracle time per configuration; 0 skips the CPU leg (and the oracle check)")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--detail", default=None, metavar="PATH",
                    help="also write every configuration's full record (timing protocol, CPU sample) as JSON")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the ceiling and vendor legs")
    ap.add_argument("--no-precondition", action="store_true",
                    help="time from whatever clock the GPU is at (no pre-conditioning; no ceilings)")
    ap.add_argument(
        "--copy-probe",
        type=float,
        default=0.0,
        metavar="MIB",
        help="only run a plain device copy of MIB MiB `steps` times (calibrates the "
        "rocprofv3 FETCH_SIZE / WRITE_SIZE counters against known bytes)",
    )
    args = ap.parse_args(argv)
    if args.copy_probe > 0:
        import torch

        n = int(args.copy_probe * (1 << 20)) // 4
        src = torch.arange(n, device="cuda:0", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n * 4, "launches": args.steps}), flush=True)
        return 0
    if args.gpus != 1:
        print(
            "bench.py measures one MI355X: the xtile tile programs run on a single GPU "
            "(multi-GPU sharding is a design note, not built); use --gpus 1",
            file=sys.stderr,
        )
        return 2
    names = ALL if args.config == "all" else args.config.split(",")
    headline = "c2" if "c2" in names else names[0]
    cfgs = {n: make_config(n) for n in names}
    print("[bench] inputs generated", file=sys.stderr, flush=True)
    dev_sets = {n: alloc_sets(cfgs[n]) for n in names}  # before any other GPU buffer
    pre = None if args.no_precondition else Preconditioner()
    ceil = None if args.no_ceilings or pre is None else ceilings(pre)
    results = {n: gpu_leg(n, cfgs[n], dev_sets.pop(n), args.steps, args.warmup, not args.no_graph, pre)
               for n in names}
    vend = None if args.no_ceilings or not ({"c3", "c5", "c6"} & set(names)) else vendor(pre)
    del pre
    if args.cpu_seconds > 0:
        for n in names:
            cpu_leg(n, cfgs[n], results[n], args.cpu_seconds)
    failed = [n for n in names if not results[n]["check"]["replay_equals_eager"]
              or not results[n]["check"].get("ok", True)]
    for r in results.values():
        r.pop("_reference")
    if failed:
        for n in failed:
            print(f"[bench] {n}: output check failed: {json.dumps(results[n]['check'])}", file=sys.stderr)
        return 1
    if ceil is not None:
        for r in results.values():
            ceiling_of(r, ceil)
    if args.detail:
        Path(args.detail).write_text(json.dumps({"attainable": ceil, "vendor": vend,
                                                 "per_config": [results[n] for n in names]}, indent=1))
    for n in names:
        print("[bench] " + summary_line(results[n]), file=sys.stderr)
    h = results[headline]
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": h["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": h["dtype"],
        "data": h["data"],
        "config": {"workload": h["workload"], "kernel": h["kernel"]},
        "roofline": h["roofline"],
        "cpu_baseline": h.get("cpu_baseline"),
        "check": h["check"],
        "timing": h["timing"],
        "attainable": compact(ceil),
        "vendor": compact(vend),
        "per_config": {n: compact_config(results[n]) for n in names},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
