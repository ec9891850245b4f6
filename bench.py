"""Benchmark of the xtile_amd HIP path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|c1|..|c7]

One step = one launch of the tile program over one batch of synthetic input
(numpy PCG64, seed = config index, shapes of BASELINE.json's configs).  The
headline line is C2 (row softmax fp32 8192x4096);
the six BASELINE.json configurations (C1-C6) and C7, a row layernorm run as a
fused tile program, are measured and reported under "per_config".

Timing: W untimed warm-up launches, then K launches captured in a HIP graph and
replayed once between two HIP events on the replay stream, with device
synchronisation on both sides; per-step time = elapsed / K.  Every step reads
a different input set (buffer rotation over >= 1 GiB) so inputs are not left
resident in the 256 MB Infinity Cache between steps.  Inputs are in HBM before
the timed region starts; no host transfer is timed.

roofline.achieved = algorithmic bytes (or FLOPs) of one launch / per-step
time; roofline.traffic = measured HBM bytes per launch from the rocprofv3
FETCH_SIZE / WRITE_SIZE summaries under profiles/ (null when absent).

cpu_baseline = the oracle (oracle/xt_oracle.c, the loop-lowered C executor of
the same xt program) timed on this host's cores over whole repetitions of the
same workload for about --cpu-seconds.
"""

from __future__ import annotations

import argparse
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
MFMA_PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0, "i8": 5000.0}  # dense; i8 in TOP/s
ROTATE_BYTES = 1 << 30


def _f32(a):
    return np.asarray(a, dtype=np.float32)


def make_config(name: str):
    """(module, host inputs, dtypes, out index, meta) for one configuration."""
    from oracle import f32_to_bf16_bits
    from xtile_amd import kernels as K

    if name == "c1":
        rng = np.random.default_rng(1)
        a = _f32(rng.uniform(-1, 1, (1024, 1024)))
        b = _f32(rng.uniform(-1, 1, (1024, 1024)))
        return K.CONFIGS["c1_add"](), [a, b, np.zeros_like(a)], ["f32"] * 3, {
            "workload": "c1_add: C = A + B fp32 1024x1024, 32x64 tiles, grid (32,16,1)",
            "unit": "GB/s",
            "bound": "hbm",
            "dtype": "f32",
            "data": "synthetic: numpy PCG64 seed=1, uniform[-1,1]",
        }
    if name == "c2":
        rng = np.random.default_rng(2)
        x = _f32(rng.normal(0.0, 2.0, (8192, 4096)))
        return K.CONFIGS["c2_softmax"](), [x, np.zeros_like(x)], ["f32"] * 2, {
            "workload": "c2_softmax: row softmax fp32 8192x4096, one 1x4096 row per Block, grid (8192,1,1)",
            "unit": "GB/s",
            "bound": "hbm",
            "dtype": "f32",
            "data": "synthetic: numpy PCG64 seed=2, normal(0,2)",
        }
    if name == "c7":
        rng = np.random.default_rng(7)
        x = _f32(rng.normal(0.0, 1.5, (8192, 4096)))
        g = _f32(rng.normal(1.0, 0.2, (1, 4096)))
        b = _f32(rng.normal(0.0, 0.2, (1, 4096)))
        n = np.full((1, 1), 1.0 / 4096, np.float32)
        e = np.full((1, 1), 1e-5, np.float32)
        return K.layernorm(8192, 4096, 1), [x, g, b, n, e, np.zeros_like(x)], ["f32"] * 6, {
            "workload": "c7_layernorm: row layernorm fp32 8192x4096 (a program outside the four benchmark "
                        "families, run as a fused tile program), one 1x4096 row per Block, grid (8192,1,1)",
            "unit": "GB/s",
            "bound": "hbm",
            "dtype": "f32",
            "data": "synthetic: numpy PCG64 seed=7, x normal(0,1.5), gamma normal(1,0.2), beta normal(0,0.2)",
        }
    if name == "c3":
        rng = np.random.default_rng(3)
        a = rng.uniform(-1, 1, (4096, 4096)).astype(np.float16)
        b = rng.uniform(-1, 1, (4096, 4096)).astype(np.float16)
        return K.CONFIGS["c3_matmul_f16"](), [a, b, np.zeros((4096, 4096), np.float32)], [
            "f16",
            "f16",
            "f32",
        ], {
            "workload": "c3_matmul_f16: C = A @ B, M=N=K=4096, f16 in, f32 acc/out, 128x128 Block tiles, B shared=1, grid (32,32,1)",
            "unit": "TFLOP/s",
            "bound": "mfma",
            "dtype": "f16",
            "data": "synthetic: numpy PCG64 seed=3, uniform[-1,1] -> f16",
        }
    if name == "c4":
        rng = np.random.default_rng(4)
        x = rng.normal(0, 0.1, (32, 56, 56, 64)).astype(np.float16)
        f = rng.normal(0, 0.1, (3, 3, 64, 64)).astype(np.float16)
        return K.CONFIGS["c4_conv2d_f16"](), [x, f, np.zeros((32, 56, 56, 64), np.float32)], [
            "f16",
            "f16",
            "f32",
        ], {
            "workload": "c4_conv2d_f16: NHWC 32x56x56x64 * 3x3x64x64, stride 1, pad 1, f16 in, f32 out, 1x4x56x64 Block tiles, filter shared=2, grid (32,14,1)",
            "unit": "TFLOP/s",
            "bound": "hbm",
            "dtype": "f16",
            "data": "synthetic: numpy PCG64 seed=4, normal(0,0.1) -> f16",
        }
    if name == "c5":
        rng = np.random.default_rng(5)
        a = f32_to_bf16_bits(_f32(rng.normal(0, 0.02, (4096, 4096))))
        b = f32_to_bf16_bits(_f32(rng.normal(0, 0.02, (4096, 11008))))
        return K.CONFIGS["c5_matmul_bf16"](), [a, b, np.zeros((4096, 11008), np.float32)], [
            "bf16",
            "bf16",
            "f32",
        ], {
            "workload": "c5_matmul_bf16: C = A @ B, M=4096 N=11008 K=4096, bf16 in (RNE), f32 out, 256x128 Block tiles, A shared=1, grid (86,16,1)",
            "unit": "TFLOP/s",
            "bound": "mfma",
            "dtype": "bf16",
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
            "i8", "i8", "i8", "f32", "f32"
        ], {
            "workload": "c6_matmul_i8: kernels/matmul.py, C = int8(A @ B * scale + bias), M=N=K=4096, "
            "i8 in, i32 acc, f32 epilogue, i8 out, 64x64 Block tiles, B/scale/bias shared=1, grid (64,64,1)",
            "unit": "TOP/s",
            "bound": "mfma",
            "dtype": "i8",
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


def gpu_time(module, host, dtypes, steps: int, warmup: int, use_graph: bool):
    """Average ms per launch over `steps` launches, rotating input sets."""
    import torch

    import xtile_amd as xt
    from tests.gpu_util import to_device

    dev = torch.device("cuda:0")
    set_bytes = sum(h.nbytes for h in host)
    nsets = max(1, min(128, math.ceil(ROTATE_BYTES / set_bytes)))
    first = [to_device(h, d, dev) for h, d in zip(host, dtypes)]
    sets = [first] + [[t.clone() for t in first] for _ in range(nsets - 1)]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for i in range(warmup):
            xt.launch(module, *sets[i % nsets])
    torch.cuda.synchronize()
    mode = "eager"
    graph = None
    if use_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(steps):
                    xt.launch(module, *sets[i % nsets])
            graph.replay()
            torch.cuda.synchronize()
            mode = "hip_graph"
        except Exception as exc:  # capture unsupported: fall back to eager launches
            print(f"[bench] graph capture failed ({exc}); timing eager launches", file=sys.stderr)
            graph = None
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        if graph is not None:
            graph.replay()
        else:
            for i in range(steps):
                xt.launch(module, *sets[i % nsets])
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    out = sets[0]
    return ms, mode, nsets, out


def cpu_time(text: str, host, seconds: float, threads: int):
    """Seconds per run of the oracle over whole repetitions of `text`."""
    import oracle

    bufs = [np.array(h, copy=True) for h in host]
    reps = 0
    t0 = time.perf_counter()
    while True:
        oracle.run(text, bufs, threads)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return elapsed / reps, reps


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


def attainable():
    """What a plain device copy and the vendor GEMM reach on this box: the
    practical ceilings beside the published peaks."""
    import torch

    dev = torch.device("cuda:0")
    out = {}
    n = (256 << 20) // 4
    src = [torch.rand(n, device=dev) for _ in range(4)]
    dst = [torch.empty_like(t) for t in src]
    for i in range(8):
        dst[i % 4].copy_(src[i % 4])
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(40):
        dst[i % 4].copy_(src[i % 4])
    end.record()
    torch.cuda.synchronize()
    out["hbm_copy_GBs"] = 40 * 2 * n * 4 / (start.elapsed_time(end) * 1e-3) / 1e9
    del src, dst
    a = (torch.rand(4096, 4096, device=dev) * 2 - 1).half()
    b = (torch.rand(4096, 4096, device=dev) * 2 - 1).half()
    for _ in range(10):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    start.record()
    for _ in range(200):
        torch.matmul(a, b)
    end.record()
    torch.cuda.synchronize()
    out["torch_matmul_f16_4096_TFLOPs"] = 200 * 2 * 4096**3 / (start.elapsed_time(end) * 1e-3) / 1e12
    out["note"] = ("device copy of 256 MiB (read + write bytes) and torch.matmul (hipBLASLt) "
                   "f16 4096^3 with f16 output, same process")
    return out


def measure(name: str, steps: int, warmup: int, cpu_seconds: float, use_graph: bool) -> dict:
    import xtile_amd as xt

    module, host, dtypes, meta = make_config(name)
    plan = xt.plan(module)
    print(f"[bench] {name}: {plan['kernel']}", file=sys.stderr, flush=True)
    ms, mode, nsets, _ = gpu_time(module, host, dtypes, steps, warmup, use_graph)
    sec = ms * 1e-3
    if meta["unit"] == "GB/s":
        value = plan["bytes"] / sec / 1e9
    else:
        value = plan["flops"] / sec / 1e12
    if meta["bound"] == "hbm":
        achieved = plan["bytes"] / sec / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": _traffic(name)}
    else:
        achieved = plan["flops"] / sec / 1e12
        peak = MFMA_PEAK_TFLOPS[meta["dtype"]]
        roof = {"bound": "mfma", "achieved": achieved, "peak": peak,
                "unit": "TOP/s" if meta["dtype"] == "i8" else "TFLOP/s",
                "frac": achieved / peak, "traffic": _traffic(name)}
    if name == "c4":  # report against the MFMA peak as well
        tf = plan["flops"] / sec / 1e12
        roof["mfma_tflops"] = tf
        roof["mfma_frac"] = tf / MFMA_PEAK_TFLOPS["f16"]
    result = {
        "config": name,
        "workload": meta["workload"],
        "kernel": plan["kernel"],
        "value": value,
        "unit": meta["unit"],
        "ms_per_step": ms,
        "dtype": meta["dtype"],
        "data": meta["data"],
        "timing": f"{mode}, {steps} launches, {nsets} rotating input sets",
        "roofline": roof,
        "algo_bytes": plan["bytes"],
        "algo_flops": plan["flops"],
    }
    if cpu_seconds > 0:
        threads = int(os.environ.get("XT_CPU_THREADS", min(16, os.cpu_count() or 1)))
        text = str(module)
        work = plan["bytes"] if meta["unit"] == "GB/s" else plan["flops"]
        scale = 1e9 if meta["unit"] == "GB/s" else 1e12
        cpu_s, reps = cpu_time(text, host, cpu_seconds, threads)
        # one thread, on a sub-grid sized to about 2 s
        sub, share = grid_subset(text, min(1.0, 2.0 / max(cpu_s * threads, 1e-9)))
        one_s, one_reps = cpu_time(sub, host, 0.5, 1)
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
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 2000 launches keep every timed region >= 7 ms (C1) and the clock settled:
    # 200-launch bursts read up to 10% slower and vary run to run with the
    # clock's ramp
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="all", help="all, or one of c1..c7")
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-graph", action="store_true")
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
    names = ["c1", "c2", "c3", "c4", "c5", "c6", "c7"] if args.config == "all" else [args.config]
    headline = "c2" if "c2" in names else names[0]
    results = {n: measure(n, args.steps, args.warmup, args.cpu_seconds, not args.no_graph) for n in names}
    h = results[headline]
    ceilings = attainable() if args.config == "all" else None
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
        "config": {"workload": h["workload"], "kernel": h["kernel"], "timing": h["timing"]},
        "roofline": h["roofline"],
        "cpu_baseline": h.get("cpu_baseline"),
        "attainable": ceilings,
        "per_config": [results[n] for n in names],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
