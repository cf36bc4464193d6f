"""Text summaries of rocprofv3 output for the kernels of the decode step.

  python -m tt_symbiote_amd.rocprof_summary trace <results.db> [--top N]
      per-kernel dispatch count and average / min / max / total duration, from the SQLite
      database written by ``rocprofv3 --kernel-trace``;

  python -m tt_symbiote_amd.rocprof_summary timeline <results.db> --last N
      the last N dispatches in start order (e.g. the replays of a captured step): per kernel
      the mean duration and the mean idle gap between the previous dispatch's end and its
      start, and the window's busy fraction;

  python -m tt_symbiote_amd.rocprof_summary pmc --kernel NAME --fetch F.csv --write W.csv
          --calib-fetch CF.csv --calib-write CW.csv --calib-kernel NAME --calib-bytes N [--json]
      HBM bytes per dispatch of kernel NAME from two ``rocprofv3 --pmc FETCH_SIZE`` /
      ``--pmc WRITE_SIZE`` runs (counter values in KiB per dispatch), each scaled by what the
      same counter reads per dispatch for a plain copy kernel that reads and writes N bytes;

  python -m tt_symbiote_amd.rocprof_summary clock --trace T.csv --counters C.csv
          [--kernel NAME ...] [--flops NAME=FLOPS ...]
      from one ``rocprofv3 --kernel-trace --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES ...``
      run: per kernel the shader clock over its dispatches and its MFMA use against the
      MI355X bf16 peak (2.5 PFLOP/s at 2.4 GHz) and against the peak at that measured clock.
"""
from __future__ import annotations

import argparse
import csv
import json
import sqlite3
import statistics
import sys
from collections import defaultdict


def kernel_stats(db_path: str):
    db = sqlite3.connect(db_path)
    rows = db.execute(
        "select s.kernel_name, count(*), avg(d.end - d.start), sum(d.end - d.start), "
        "min(d.end - d.start), max(d.end - d.start) from rocpd_kernel_dispatch d "
        "join rocpd_info_kernel_symbol s on d.kernel_id = s.id "
        "group by s.kernel_name order by sum(d.end - d.start) desc").fetchall()
    db.close()
    return rows


def print_trace(db_path: str, top: int) -> None:
    print(f"{'calls':>6} {'avg us':>9} {'min us':>9} {'max us':>9} {'total ms':>9}  kernel")
    for name, n, avg, tot, mn, mx in kernel_stats(db_path)[:top]:
        print(f"{n:6d} {avg / 1e3:9.1f} {mn / 1e3:9.1f} {mx / 1e3:9.1f} {tot / 1e6:9.2f}  "
              f"{name[:110]}")


def print_timeline(db_path: str, last: int) -> None:
    db = sqlite3.connect(db_path)
    rows = db.execute(
        "select s.kernel_name, d.start, d.end from rocpd_kernel_dispatch d "
        "join rocpd_info_kernel_symbol s on d.kernel_id = s.id order by d.start").fetchall()
    db.close()
    rows = rows[-last:]
    dur = defaultdict(list)
    gap = defaultdict(list)
    order = []
    for i, (name, st, en) in enumerate(rows):
        if name not in dur:
            order.append(name)
        dur[name].append(en - st)
        if i:
            gap[name].append(max(0, st - rows[i - 1][2]))
    span = rows[-1][2] - rows[0][1]
    busy = sum(en - st for _, st, en in rows)
    print(f"window: {len(rows)} dispatches, {span / 1e3:.1f} us, busy {busy / 1e3:.1f} us "
          f"({100.0 * busy / span:.1f}%)")
    print(f"{'calls':>6} {'avg us':>9} {'gap us':>9}  kernel (in order of first start)")
    for name in order:
        g = gap[name]
        print(f"{len(dur[name]):6d} {statistics.mean(dur[name]) / 1e3:9.2f} "
              f"{(statistics.mean(g) / 1e3 if g else 0.0):9.2f}  {name[:100]}")


def counter_per_dispatch(csv_path: str, counter: str) -> dict:
    """{kernel name: [counter value of each dispatch]} (values summed over the rows of one
    dispatch, e.g. per-XCD instances)."""
    per_dispatch = defaultdict(float)
    names = {}
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            key = row["Dispatch_Id"]
            per_dispatch[key] += float(row["Counter_Value"])
            names[key] = row["Kernel_Name"]
    out = defaultdict(list)
    for key, v in per_dispatch.items():
        out[names[key]].append(v)
    return out


def print_counters(csv_paths, kernels) -> None:
    """For each kernel whose name contains one of ``kernels``: every counter of the CSVs, as the
    median over its dispatches of the sum over a dispatch's rows (per-XCD / per-SE instances)
    and of their maximum (GRBM_GUI_ACTIVE is a per-instance clock: use its max)."""
    sums = defaultdict(lambda: defaultdict(lambda: defaultdict(float)))
    maxs = defaultdict(lambda: defaultdict(lambda: defaultdict(float)))
    for path in csv_paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"]
                if not any(k in name for k in kernels):
                    continue
                v = float(row["Counter_Value"])
                key = (row["Dispatch_Id"], row.get("Grid_Size", ""))
                sums[name][row["Counter_Name"]][key] += v
                cur = maxs[name][row["Counter_Name"]]
                cur[key] = max(cur[key], v)
    for name in sorted(sums):
        print(name[:110])
        for c in sorted(sums[name]):
            s_med = statistics.median(sums[name][c].values())
            m_med = statistics.median(maxs[name][c].values())
            print(f"  {c:32s} sum {s_med:16.0f}   max {m_med:14.0f}   "
                  f"({len(sums[name][c])} dispatches)")


def _match(table: dict, needle: str) -> list:
    hits = [k for k in table if needle in k]
    if not hits:
        raise SystemExit(f"no kernel matching {needle!r}")
    if len(hits) > 1:
        hits.sort(key=len)
    return table[hits[0]]


def pmc_traffic(args) -> dict:
    fetch = statistics.median(_match(counter_per_dispatch(args.fetch, "FETCH_SIZE"), args.kernel))
    write = statistics.median(_match(counter_per_dispatch(args.write, "WRITE_SIZE"), args.kernel))
    cf = statistics.median(_match(counter_per_dispatch(args.calib_fetch, "FETCH_SIZE"),
                                  args.calib_kernel))
    cw = statistics.median(_match(counter_per_dispatch(args.calib_write, "WRITE_SIZE"),
                                  args.calib_kernel))
    f_fetch = args.calib_bytes / cf
    f_write = args.calib_bytes / cw
    return {
        "kernel": args.kernel,
        "fetch_size_kib_per_dispatch": fetch,
        "write_size_kib_per_dispatch": write,
        "calibration": {"kernel": args.calib_kernel, "bytes_read_and_written": args.calib_bytes,
                        "fetch_size_kib": cf, "write_size_kib": cw,
                        "fetch_bytes_per_unit": f_fetch, "write_bytes_per_unit": f_write},
        "hbm_read_bytes": fetch * f_fetch,
        "hbm_write_bytes": write * f_write,
        "traffic_bytes": fetch * f_fetch + write * f_write,
    }


XCDS = 8                 # GRBM_GUI_ACTIVE is counted per XCD and summed by rocprofv3
PEAK_CLOCK_GHZ = 2.4     # the clock of the published 2.5 PFLOP/s dense bf16 peak
BF16_FLOPS_PER_MFMA_CYCLE = 1024   # per SIMD: v_mfma_f32_16x16x32_bf16 is 16384 flops over 16
                                   # busy cycles, v_mfma_f32_32x32x16_bf16 32768 over 32


def _dispatch_table(trace_csv: str, counter_csv: str) -> list:
    """[(kernel name, duration ns, {counter: value summed over the dispatch's rows})]"""
    dur, names = {}, {}
    with open(trace_csv, newline="") as f:
        for row in csv.DictReader(f):
            dur[row["Dispatch_Id"]] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
            names[row["Dispatch_Id"]] = row["Kernel_Name"]
    counters = defaultdict(lambda: defaultdict(float))
    with open(counter_csv, newline="") as f:
        for row in csv.DictReader(f):
            counters[row["Dispatch_Id"]][row["Counter_Name"]] += float(row["Counter_Value"])
    return [(names[k], dur[k], dict(c)) for k, c in counters.items() if dur.get(k, 0) > 0]


def profiler_window_cycles(table: list) -> tuple:
    """Least-squares fit GRBM_GUI_ACTIVE = a + b * duration over the dispatches that issue no
    MFMA: ``a`` is the part of the counter window outside the kernel (the profiler starts and
    stops the counters around each dispatch), ``b`` the mean summed clock of those kernels."""
    pts = [(d, c["GRBM_GUI_ACTIVE"]) for _, d, c in table
           if "GRBM_GUI_ACTIVE" in c and c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) == 0]
    n = len(pts)
    if n < 3:
        return 0.0, 0.0
    mx = sum(d for d, _ in pts) / n
    my = sum(g for _, g in pts) / n
    sxx = sum((d - mx) ** 2 for d, _ in pts)
    b = sum((d - mx) * (g - my) for d, g in pts) / sxx
    return my - b * mx, b


def clock_report(trace_csv: str, counter_csv: str, kernels, flops: dict) -> None:
    table = _dispatch_table(trace_csv, counter_csv)
    a, b = profiler_window_cycles(table)
    print(f"counter window outside the kernel: {a:.0f} GRBM cycles (fit over the dispatches "
          f"without MFMA: {b / XCDS:.3f} GHz per XCD)")
    per = defaultdict(list)
    for name, d, c in table:
        if kernels and not any(k in name for k in kernels):
            continue
        per[name].append((d, c))
    print(f"{'calls':>5} {'us':>8} {'GHz':>6} {'(raw)':>6} {'MFMA TF/s':>10} {'/2.5PF':>7} "
          f"{'/clk-pk':>7} {'algo TF/s':>10} {'/2.5PF':>7} {'/clk-pk':>7}  kernel")
    for name, lst in sorted(per.items(), key=lambda kv: -statistics.median(x[0] for x in kv[1])):
        t = statistics.median(d for d, _ in lst) * 1e-9
        g = statistics.median(c.get("GRBM_GUI_ACTIVE", 0.0) for _, c in lst)
        busy = statistics.median(c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for _, c in lst)
        clk = (g - a) / XCDS / t * 1e-9
        raw = g / XCDS / t * 1e-9
        peak = 2.5e15
        clk_peak = peak * clk / PEAK_CLOCK_GHZ
        ex = busy * BF16_FLOPS_PER_MFMA_CYCLE / t
        line = (f"{len(lst):5d} {t * 1e6:8.1f} {clk:6.3f} {raw:6.3f} {ex / 1e12:10.1f} "
                f"{ex / peak:7.3f} {ex / clk_peak:7.3f}")
        algo = [v for k, v in flops.items() if k in name]
        if algo:
            al = algo[0] / t
            line += f" {al / 1e12:10.1f} {al / peak:7.3f} {al / clk_peak:7.3f}"
        else:
            line += f" {'':>10} {'':>7} {'':>7}"
        print(f"{line}  {name.split('(')[0][:60]}")


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("db")
    t.add_argument("--top", type=int, default=25)
    tl = sub.add_parser("timeline")
    tl.add_argument("db")
    tl.add_argument("--last", type=int, default=100)
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+")
    c.add_argument("--kernel", action="append", required=True)
    p = sub.add_parser("pmc")
    p.add_argument("--kernel", required=True)
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--calib-fetch", required=True)
    p.add_argument("--calib-write", required=True)
    p.add_argument("--calib-kernel", required=True)
    p.add_argument("--calib-bytes", type=float, required=True)
    p.add_argument("--json", action="store_true")
    k = sub.add_parser("clock")
    k.add_argument("--trace", required=True)
    k.add_argument("--counters", required=True)
    k.add_argument("--kernel", action="append", default=[])
    k.add_argument("--flops", action="append", default=[],
                   help="NAME=FLOPS: algorithmic flops per dispatch of the kernel matching NAME")
    args = ap.parse_args(argv)
    if args.cmd == "clock":
        flops = {}
        for item in args.flops:
            key, _, val = item.rpartition("=")
            flops[key] = float(val)
        clock_report(args.trace, args.counters, args.kernel, flops)
        return
    if args.cmd == "trace":
        print_trace(args.db, args.top)
        return
    if args.cmd == "timeline":
        print_timeline(args.db, args.last)
        return
    if args.cmd == "counters":
        print_counters(args.csv, args.kernel)
        return
    res = pmc_traffic(args)
    if args.json:
        json.dump(res, sys.stdout, indent=1)
        print()
        return
    c = res["calibration"]
    print(f"kernel {res['kernel']}")
    print(f"  FETCH_SIZE {res['fetch_size_kib_per_dispatch']:.0f} (nominal KiB) per dispatch x "
          f"{c['fetch_bytes_per_unit']:.1f} B = {res['hbm_read_bytes'] / 1e6:.1f} MB read")
    print(f"  WRITE_SIZE {res['write_size_kib_per_dispatch']:.0f} (nominal KiB) per dispatch x "
          f"{c['write_bytes_per_unit']:.1f} B = {res['hbm_write_bytes'] / 1e6:.1f} MB written")
    print(f"  traffic {res['traffic_bytes'] / 1e6:.1f} MB per dispatch")
    print(f"calibration: {c['kernel']} moving {c['bytes_read_and_written'] / 2**20:.0f} MiB each "
          f"way reads FETCH_SIZE {c['fetch_size_kib']:.0f} / WRITE_SIZE {c['write_size_kib']:.0f}")


if __name__ == "__main__":
    main()
