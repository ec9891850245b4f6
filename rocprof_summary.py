"""Summarise rocprofv3 (rocpd SQLite) output for xtile_amd kernels.

    python rocprof_summary.py --trace T.db [--fetch F.db --write W.db
        --copy-fetch CF.db --copy-write CW.db --copy-mib 256] [--pmc P.db ...]
        [--kernel REGEX] [--power P.json] [--command "..."] > profiles/<config>_<kernel>.txt

Measurement tooling beside bench.py; the xtile_amd package never imports it.

Kernel-trace databases give per-kernel dispatch counts and durations, and for
the selected kernel the span of its longest run of back-to-back dispatches
divided by their count (the rate a stream of launches sustains under the
tracer, comparable with bench.py's per-step time).  The FETCH_SIZE /
WRITE_SIZE databases (one counter per pass) give KiB per dispatch; each
counter is scaled by the factor that makes it read the true byte count of a
plain device copy of --copy-mib MiB (which reads and writes exactly that many
bytes).  The scaled bytes are printed as `fetch_bytes` / `write_bytes` lines,
which bench.py reads as roofline.traffic.

Each --pmc database (any other counters, one pass each) is reduced per
dispatch of the selected kernel - counters summed over their instances - and
averaged over the dispatches.  SQ_BUSY_CYCLES is counted by each of the 32
shader engines (8 XCDs x 4) while it has work, so SQ_BUSY_CYCLES / 32 is the
dispatch's length in shader-clock cycles.  From it:
  - sq_busy_clock_GHz = (SQ_BUSY_CYCLES / 32) / traced dispatch duration
    (dispatches run one at a time under counter collection; a lower bound of
    the clock, since the traced duration includes the launch and drain);
  - counter_duration_us = (SQ_BUSY_CYCLES / 32) / the clock sampled while
    the kernel runs back to back (--power, power_sample.py);
  - mfma_busy_fraction = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x
    SQ_BUSY_CYCLES / 32), the share of the dispatch's cycles in which an
    average SIMD's matrix pipe is busy.
"""

from __future__ import annotations

import argparse
import collections
import json
import re
import sqlite3
import statistics

SIMDS = 1024  # 256 CUs x 4 SIMDs on MI355X


SHADER_ENGINES = 32  # 8 XCDs x 4 shader engines; each counts its own SQ_BUSY_CYCLES


def _kernels(db_path: str, pattern: str | None):
    db = sqlite3.connect(db_path)
    rows = db.execute("select name, duration, grid_x, workgroup_x, dispatch_id from kernels").fetchall()
    if pattern:
        rows = [r for r in rows if re.search(pattern, r[0])]
    return rows


def _span_rate(db_path: str, pattern: str):
    """(us per dispatch, count) over the longest run of consecutive dispatches
    (in dispatch order, no other kernel between them) of the selected kernel:
    (end of the last - start of the first) / count."""
    db = sqlite3.connect(db_path)
    try:
        rows = db.execute("select name, start, end from kernels order by start").fetchall()
    except sqlite3.Error:
        return None
    best, first, n = (0, 0, 0), 0, 0  # (count, start of the first, end of the last)
    for name, st, en in rows:
        if re.search(pattern, name):
            if n == 0:
                first = st
            n += 1
            if n > best[0]:
                best = (n, first, en)
        else:
            n = 0
    if best[0] < 2:
        return None
    return (best[2] - best[1]) / 1000.0 / best[0], best[0]


def _per_dispatch(db_path: str, pattern: str | None):
    """{dispatch_id: ({counter: reduced value}, duration_ns)} for the selected kernel."""
    db = sqlite3.connect(db_path)
    rows = db.execute("select dispatch_id, name, counter_name, counter_value, duration from pmc_events").fetchall()
    vals: dict = collections.defaultdict(lambda: collections.defaultdict(list))
    dur = {}
    for d, name, cn, v, du in rows:
        if pattern and not re.search(pattern, name):
            continue
        vals[d][cn].append(float(v))
        dur[d] = du
    out = {}
    for d, cs in vals.items():
        out[d] = ({cn: sum(v) for cn, v in cs.items()}, dur[d])
    return out


def _counter(db_path: str, counter: str, pattern: str | None):
    per = _per_dispatch(db_path, pattern)
    return [cs[counter] for cs, _ in per.values() if counter in cs]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace", required=True)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-mib", type=float, default=256.0)
    ap.add_argument("--pmc", action="append", default=[], help="a counter-collection database (repeatable)")
    ap.add_argument("--kernel", default=None, help="regex selecting the kernel of interest")
    ap.add_argument("--command", action="append", default=[], help="command lines to record")
    ap.add_argument("--bench-log", default=None, help="stdout of the traced bench.py run")
    ap.add_argument("--power", default=None, help="JSON line written by power_sample.py for this config")
    ap.add_argument("--trace-eager", default=None,
                    help="a kernel-trace database of bench.py's eager 20-launch protocol (--steps 20 --warmup 5)")
    args = ap.parse_args(argv)

    power = json.loads(open(args.power).read().strip().splitlines()[-1]) if args.power else None
    out = []
    for c in args.command:
        out.append(f"# command: {c}")
    rows = _kernels(args.trace, None)
    by_name: dict[str, list] = {}
    for name, dur, gx, wx, _ in rows:
        by_name.setdefault(name, []).append((dur, gx, wx))
    out.append("# kernel-trace (durations in microseconds)")
    out.append(f"{'kernel':44s} {'calls':>6s} {'avg_us':>9s} {'median_us':>9s} {'min_us':>9s} {'max_us':>9s}  grid(threads)")
    for name, items in sorted(by_name.items(), key=lambda kv: -sum(d for d, _, _ in kv[1])):
        durs = [d / 1000.0 for d, _, _ in items]
        grids = sorted({g for _, g, _ in items})
        out.append(
            f"{name[:44]:44s} {len(durs):6d} {statistics.mean(durs):9.2f} {statistics.median(durs):9.2f} "
            f"{min(durs):9.2f} {max(durs):9.2f}  {','.join(map(str, grids))}"
        )
    if args.kernel:
        sel = [d / 1000.0 for n, d, *_ in rows if re.search(args.kernel, n)]
        if sel:
            out.append(f"selected_kernel: {args.kernel}")
            out.append(f"selected_avg_us: {statistics.mean(sel):.3f}")
            out.append(f"selected_median_us: {statistics.median(sel):.3f}")
            span = _span_rate(args.trace, args.kernel)
            if span:
                out.append(f"selected_back_to_back_us_per_dispatch: {span[0]:.3f}  (span of the longest run of "
                           f"{span[1]} consecutive dispatches / count)")
    if args.trace_eager and args.kernel:
        eager = [d / 1000.0 for n, d, *_ in _kernels(args.trace_eager, args.kernel)]
        if len(eager) >= 20:
            timed = eager[-20:]  # the timed launches come last
            out.append(f"eager_protocol_avg_us: {statistics.mean(timed):.3f}  (the last 20 dispatches of the eager "
                       f"20-launch run: its timed launches)")
    if args.bench_log:
        lines = [ln for ln in open(args.bench_log).read().splitlines() if ln.startswith('{"metric"')]
        if lines:
            rec = json.loads(lines[-1])
            out.append(
                f"bench_us_per_launch_same_run: {rec['ms_per_step'] * 1000.0:.3f}  "
                f"(bench.py's own HIP-event timing of its {rec['steps']} timed launches)"
            )
    if args.fetch and args.write:
        fetch = _counter(args.fetch, "FETCH_SIZE", args.kernel)
        write = _counter(args.write, "WRITE_SIZE", args.kernel)
        f_scale = w_scale = 1.0
        true_kib = args.copy_mib * 1024.0
        if args.copy_fetch and args.copy_write:
            cf = _counter(args.copy_fetch, "FETCH_SIZE", "copyBuffer")
            cw = _counter(args.copy_write, "WRITE_SIZE", "copyBuffer")
            if cf and cw:
                f_scale = true_kib / statistics.mean(cf)
                w_scale = true_kib / statistics.mean(cw)
                out.append(
                    f"# copy calibration: {args.copy_mib:g} MiB device copy reads FETCH_SIZE="
                    f"{statistics.mean(cf):.1f} KiB (factor {f_scale:.4f}), WRITE_SIZE="
                    f"{statistics.mean(cw):.1f} KiB (factor {w_scale:.4f})"
                )
        if fetch and write:
            fk, wk = statistics.mean(fetch), statistics.mean(write)
            out.append(f"fetch_kib_per_dispatch: {fk:.1f}  (raw, {len(fetch)} dispatches)")
            out.append(f"write_kib_per_dispatch: {wk:.1f}  (raw, {len(write)} dispatches)")
            out.append(f"fetch_bytes: {fk * 1024.0 * f_scale:.0f}")
            out.append(f"write_bytes: {wk * 1024.0 * w_scale:.0f}")
    for db in args.pmc:
        per = _per_dispatch(db, args.kernel)
        if not per:
            continue
        names = sorted({cn for cs, _ in per.values() for cn in cs})
        out.append(f"# counters per dispatch of the selected kernel ({len(per)} dispatches, {db.split('/')[-2]})")
        for cn in names:
            vals = [cs[cn] for cs, _ in per.values() if cn in cs]
            out.append(f"{cn}: {statistics.mean(vals):.0f}")
        durs = [d / 1000.0 for _, d in per.values()]
        out.append(f"pmc_dispatch_avg_us: {statistics.mean(durs):.3f}")
        cyc = [(cs["SQ_BUSY_CYCLES"] / SHADER_ENGINES, cs, d) for cs, d in per.values() if cs.get("SQ_BUSY_CYCLES")]
        if cyc:
            out.append(f"sq_busy_cycles_per_engine: {statistics.mean(c for c, _, _ in cyc):.0f}  "
                       f"(SQ_BUSY_CYCLES / {SHADER_ENGINES} shader engines)")
            clk = [c / d for c, _, d in cyc if d]
            if clk:
                out.append(f"sq_busy_clock_GHz: {statistics.mean(clk):.3f}  ((SQ_BUSY_CYCLES / {SHADER_ENGINES}) / "
                           "traced duration of the serialised dispatch)")
            if power and power.get("gfxclk_MHz_median"):
                ghz = power["gfxclk_MHz_median"] / 1000.0
                out.append(f"counter_duration_us: {statistics.mean(c for c, _, _ in cyc) / ghz / 1000.0:.3f}  "
                           f"((SQ_BUSY_CYCLES / {SHADER_ENGINES}) / the sampled {ghz:.3f} GHz)")
            busy = [cs["SQ_VALU_MFMA_BUSY_CYCLES"] / (c * SIMDS) for c, cs, _ in cyc
                    if "SQ_VALU_MFMA_BUSY_CYCLES" in cs]
            if busy:
                out.append(f"mfma_busy_fraction: {statistics.mean(busy):.3f}  (SQ_VALU_MFMA_BUSY_CYCLES / "
                           f"(1024 SIMDs x SQ_BUSY_CYCLES / {SHADER_ENGINES}))")
    if power:
        rec = power
        out.append("# clock and power while the kernel runs back to back (power_sample.py)")
        for k in ("launches", "us_per_launch", "gfxclk_MHz_median", "gfxclk_MHz_per_xcd", "socket_power_W_median",
                  "throttle_status", "samples"):
            if k in rec:
                out.append(f"{k}: {rec[k]}")
    print("\n".join(out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
