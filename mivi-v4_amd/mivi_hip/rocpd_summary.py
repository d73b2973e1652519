"""Text summaries of rocprofv3 result databases (rocpd SQLite).

    python -m mivi_hip.rocpd_summary DB [--filter SUBSTR] [--pmc [--by-grid]]

Kernel mode prints dispatch count and duration statistics per kernel name.
With --pmc it prints, per kernel name, the mean per-dispatch value of every
collected counter (FETCH_SIZE / WRITE_SIZE are reported by rocprofv3 in KiB);
--by-grid splits each kernel's dispatches by grid size (e.g. the decode
launches of a kernel from its prefill launches).
"""
from __future__ import annotations

import argparse
import collections
import sqlite3
import statistics


def kernel_stats(db: str, filt: str = ""):
    cur = sqlite3.connect(db).cursor()
    rows = cur.execute("select name, duration from kernels").fetchall()
    g = collections.defaultdict(list)
    for name, dur in rows:
        if filt in name:
            g[name].append(dur)
    out = []
    for name, d in sorted(g.items(), key=lambda kv: -sum(kv[1])):
        out.append(dict(name=name, count=len(d), mean_us=statistics.mean(d) / 1e3,
                        median_us=statistics.median(d) / 1e3, min_us=min(d) / 1e3,
                        total_ms=sum(d) / 1e6))
    return out


def pmc_stats(db: str, filt: str = "", by_grid: bool = False):
    cur = sqlite3.connect(db).cursor()
    rows = cur.execute("select kernel_name, counter_name, value, dispatch_id, grid_size_x, grid_size_y "
                       "from counters_collection").fetchall()
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    for name, counter, value, disp, gx, gy in rows:
        if filt in name:
            grid = (gx, gy) if by_grid else None
            per[(name, grid, counter)][disp] += value  # summed over the counter's instances
    out = []
    for (name, grid, counter), d in sorted(per.items(), key=lambda kv: (kv[0][0], kv[0][1] or (0, 0), kv[0][2])):
        vals = list(d.values())
        out.append(dict(name=name, grid=grid, counter=counter, dispatches=len(vals), mean=statistics.mean(vals),
                        median=statistics.median(vals)))
    return out


def per_period(db: str, marker: str, periods: int):
    """Breakdown of the last `periods` repetitions of a kernel sequence that
    ends with the kernel whose name contains `marker` (e.g. one decode step)."""
    cur = sqlite3.connect(db).cursor()
    rows = cur.execute("select name, duration, grid_x, start, end from kernels order by start").fetchall()
    ends = [i for i, r in enumerate(rows) if marker in r[0]]
    if len(ends) < periods + 1:
        raise SystemExit(f"only {len(ends)} '{marker}' kernels")
    win = rows[ends[-periods - 1] + 1: ends[-1] + 1]
    wall = (win[-1][4] - win[0][3]) / periods / 1e3
    busy = sum(r[1] for r in win) / periods / 1e3
    print(f"per period: wall {wall:.1f} us, kernels {len(win) / periods:.1f}, GPU busy {busy:.1f} us, "
          f"idle between kernels {wall - busy:.1f} us")
    g = collections.OrderedDict()
    for name, dur, gx, st, en in win:
        short = name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:70]
        g.setdefault((short, gx // 256), []).append(dur)
    print(f"{'per period':>10s} {'median_us':>10s} {'us/period':>10s} {'wgs':>6s}  kernel")
    for (short, wgs), d in sorted(g.items(), key=lambda kv: -sum(kv[1])):
        print(f"{len(d) / periods:10.1f} {statistics.median(d) / 1e3:10.2f} {sum(d) / periods / 1e3:10.1f} "
              f"{wgs:6d}  {short}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--filter", default="")
    ap.add_argument("--pmc", action="store_true")
    ap.add_argument("--by-grid", action="store_true", help="with --pmc: one line per (kernel, grid size)")
    ap.add_argument("--period-marker", default="", help="per-repetition breakdown ending at this kernel")
    ap.add_argument("--periods", type=int, default=32)
    a = ap.parse_args()
    if a.period_marker:
        per_period(a.db, a.period_marker, a.periods)
    elif a.pmc:
        for r in pmc_stats(a.db, a.filter, a.by_grid):
            grid = f"grid {r['grid'][0]}x{r['grid'][1]}  " if r["grid"] else ""
            print(f"{r['counter']:16s} dispatches {r['dispatches']:6d}  mean {r['mean']:14.2f}  "
                  f"median {r['median']:14.2f}  {grid}{r['name'][:110]}")
    else:
        print(f"{'count':>6s} {'mean_us':>10s} {'median_us':>10s} {'min_us':>9s} {'total_ms':>9s}  kernel")
        for r in kernel_stats(a.db, a.filter):
            print(f"{r['count']:6d} {r['mean_us']:10.2f} {r['median_us']:10.2f} {r['min_us']:9.2f} "
                  f"{r['total_ms']:9.2f}  {r['name'][:140]}")


if __name__ == "__main__":
    main()
