"""Clock and power of the GPU while one benchmark configuration runs back to back.

    python power_sample.py --config c3 [--seconds 3] > out.json
    python power_sample.py --config ceiling_mfma_f16   (bench.py's MFMA loop;
        also ceiling_mfma_bf16, ceiling_mfma_i8, ceiling_copy)

Runs the configuration's launch (bench.py's inputs, rotating input sets)
captured in a HIP graph of about 30 ms of launches (at least --per-graph)
and replayed back to back for --seconds, two replays queued at a time, while
the host samples the driver's GPU metrics table (amdsmi gpu_metrics: current
graphics clock per XCD, socket power, throttle status) every ~5 ms; the first
0.5 s (the clock's ramp) are left out of the medians.
Prints one JSON line.  Measurement tooling beside bench.py: the xtile_amd
package never imports it.
"""

from __future__ import annotations

import argparse
import json
import math
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", required=True)
    ap.add_argument("--seconds", type=float, default=3.0)
    ap.add_argument("--per-graph", type=int, default=100)
    args = ap.parse_args(argv)

    import amdsmi
    import torch

    import bench
    import xtile_amd as xt

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    if args.config.startswith("ceiling_"):
        # bench.py's ceiling kernels: ceiling_mfma_{f16,bf16,i8} (the MFMA loop) or ceiling_copy
        pre = bench.Preconditioner()
        kind = args.config.split("_")[-1]
        nsets = 1
        if args.config.startswith("ceiling_mfma_"):
            launch = lambda i: pre.mfma(kind, 4000, stream.cuda_stream)  # noqa: E731
        else:
            launch = lambda i: pre.copy(pre.src.data_ptr(), pre.dst.data_ptr(), pre.copy_bytes,  # noqa: E731
                                        stream.cuda_stream)
    else:
        module, host, dtypes, out, meta = bench.make_config(args.config)
        set_bytes = sum(h.nbytes for h in host)
        nsets = max(1, min(128, math.ceil(bench.ROTATE_BYTES / set_bytes)))
        first = [bench.to_device(h, d, dev) for h, d in zip(host, dtypes)]
        sets = [first] + [[t.clone() for t in first] for _ in range(nsets - 1)]
        launch = lambda i: xt.launch(module, *sets[i], stream=stream)  # noqa: E731
    # size one replay to about 30 ms of work, so that two queued replays keep
    # the GPU busy while the host samples
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        launch(0)
        e0.record(stream)
        for i in range(20):
            launch(i % nsets)
        e1.record(stream)
    torch.cuda.synchronize()
    per_launch_ms = e0.elapsed_time(e1) / 20
    per_graph = max(args.per_graph, int(30.0 / max(per_launch_ms, 1e-3)))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(per_graph):
            launch(i % nsets)
    torch.cuda.synchronize()

    amdsmi.amdsmi_init()
    handle = amdsmi.amdsmi_get_processor_handles()[0]
    samples = []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.time()
    replays = 0
    done = []
    with torch.cuda.stream(stream):
        start.record(stream)
        while time.time() - t0 < args.seconds:
            graph.replay()
            replays += 1
            ev = torch.cuda.Event()
            ev.record(stream)
            done.append(ev)
            # sample until the previous replay ends (this one is queued behind it)
            if len(done) >= 2:
                while not done[-2].query():
                    m = amdsmi.amdsmi_get_gpu_metrics_info(handle)
                    samples.append((time.time() - t0, m.get("current_gfxclks"), m.get("current_socket_power"),
                                    m.get("throttle_status")))
                    time.sleep(0.005)
        end.record(stream)
    torch.cuda.synchronize()
    amdsmi.amdsmi_shut_down()
    us = start.elapsed_time(end) * 1000.0 / (replays * per_graph)
    steady = [s for s in samples if s[0] >= 0.5] or samples
    clks = [[c for c in (s[1] or []) if isinstance(c, int) and 0 < c < 10000] for s in steady]
    clks = [c for c in clks if c]
    per_xcd = [round(statistics.median(col)) for col in zip(*clks)] if clks else None
    rec = {
        "config": args.config,
        "launches": replays * per_graph,
        "us_per_launch": round(us, 3),
        "gfxclk_MHz_median": round(statistics.median(c for row in clks for c in row)) if clks else None,
        "gfxclk_MHz_per_xcd": per_xcd,
        "socket_power_W_median": round(statistics.median(s[2] for s in steady if isinstance(s[2], (int, float))))
        if steady else None,
        "throttle_status": sorted({str(s[3]) for s in steady}),
        "samples": len(steady),
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
