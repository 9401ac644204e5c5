#!/usr/bin/env python3
"""Per-kernel statistics of a rocprofv3 CSV, over the last dispatches only.

A bench or profiling run launches each kernel many times: warmup steps, the
clock ramp (tens of milliseconds of back-to-back launches while the GPU's
clocks rise), then the timed steps. The profiler's own --stats summary
averages all of them; this tool keeps, per kernel, only the last N dispatches
(by start time), i.e. the timed, warm ones, so its figures can be set beside
the bench line of the same command.

    python trace_stats.py T_kernel_trace.csv [--last 200] [--match SUBSTR ...]
    python trace_stats.py S_counter_collection.csv [--last 200] [--match SUBSTR ...]

A kernel trace gives count, mean, median, min and max duration (ns) of the
last N dispatches of each kernel; a counter collection gives, per kernel and
counter, the mean value per dispatch over its last N dispatches. Kernel names
are demangled only as far as the CSV already has them. Output is a Markdown
table on stdout.
"""
from __future__ import annotations

import argparse
import csv
import statistics
import sys
from collections import defaultdict


def _short(name: str, width: int = 90) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def kernel_trace(rows, last: int, match) -> list[str]:
    per = defaultdict(list)
    for r in rows:
        name = r["Kernel_Name"]
        if match and not any(m in name for m in match):
            continue
        per[name].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    out = [f"| Kernel | Dispatches (all) | Last | Mean ns | Median ns | Min ns | Max ns |",
           "|---|---|---|---|---|---|---|"]
    for name, d in sorted(per.items(), key=lambda kv: -len(kv[1])):
        d.sort()
        tail = [x for _, x in d[-last:]]
        out.append(f"| `{_short(name)}` | {len(d)} | {len(tail)} | {statistics.fmean(tail):,.0f} | "
                   f"{statistics.median(tail):,.0f} | {min(tail):,} | {max(tail):,} |")
    return out


def counters(rows, last: int, match) -> list[str]:
    # one row per (dispatch, counter); keep each kernel's last N dispatches
    per = defaultdict(lambda: defaultdict(dict))      # kernel -> dispatch -> counter -> value
    start = {}
    for r in rows:
        name = r["Kernel_Name"]
        if match and not any(m in name for m in match):
            continue
        did = int(r["Dispatch_Id"])
        per[name][did][r["Counter_Name"]] = float(r["Counter_Value"])
        start[(name, did)] = int(r["Start_Timestamp"])
    out = ["| Kernel | Counter | Dispatches (all) | Last | Mean per dispatch |", "|---|---|---|---|---|"]
    for name, ds in sorted(per.items(), key=lambda kv: -len(kv[1])):
        ids = sorted(ds, key=lambda i: start[(name, i)])[-last:]
        names = sorted({c for i in ids for c in ds[i]})
        for c in names:
            vals = [ds[i][c] for i in ids if c in ds[i]]
            out.append(f"| `{_short(name, 60)}` | {c} | {len(ds)} | {len(vals)} | {statistics.fmean(vals):,.1f} |")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("csv")
    ap.add_argument("--last", type=int, default=200, help="dispatches kept per kernel (the last ones)")
    ap.add_argument("--match", nargs="*", default=None, help="keep kernels whose name contains one of these")
    args = ap.parse_args(argv)
    with open(args.csv, newline="") as f:
        rows = list(csv.DictReader(f))
    if not rows:
        print("no rows", file=sys.stderr)
        return 1
    lines = counters(rows, args.last, args.match) if "Counter_Name" in rows[0] else kernel_trace(rows, args.last, args.match)
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
