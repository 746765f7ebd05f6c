"""Per-kernel summaries of rocprofv3 results databases (`*_results.db`).

    python -m dwim_amd.rocprof_summary trace RUN_results.db [--top N] [--match S] [--after K]
    python -m dwim_amd.rocprof_summary pmc RUN_results.db [--match S]

`trace` (from `rocprofv3 --kernel-trace`): for each kernel name and grid
size, the dispatch count, mean / median duration in µs and total ms.  With
--after K only the dispatches that start after the last dispatch of a kernel
whose name contains K count (e.g. the decode steps after a prefill), and the
window's wall time and busy share are printed.
`pmc` (from `rocprofv3 --pmc C`): for each kernel name and grid size and
each counter, the dispatch count and the mean value per dispatch.
"""
from __future__ import annotations

import argparse
import collections
import re
import sqlite3
import statistics


def _short(name: str) -> str:
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    return name if len(name) <= 90 else name[:87] + "..."


def trace(db: str, top: int, match: str | None, after: str | None = None) -> str:
    c = sqlite3.connect(db)
    rows = c.execute("select name, grid_x, start, end from kernels").fetchall()
    window = ""
    if after:
        last = max((e for name, _, _, e in rows if after in name), default=None)
        if last is None:
            return f"no dispatch of a kernel matching {after!r}"
        rows = [r for r in rows if r[2] > last]
        if rows:
            span = max(r[3] for r in rows) - min(r[2] for r in rows)
            busy = sum(r[3] - r[2] for r in rows)
            window = f"window after the last {after}: {span / 1e6:.3f} ms wall, GPU busy {busy / max(span, 1):.1%}"
    agg = collections.defaultdict(list)
    for name, grid, s, e in rows:
        if match and match not in name:
            continue
        agg[(_short(name), grid)].append((e - s) / 1000.0)
    total = sum(sum(v) for v in agg.values())
    out = [f"{'calls':>7} {'mean us':>9} {'median us':>9} {'total ms':>9} {'share':>6}  grid  kernel"]
    for (name, grid), ds in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:top]:
        out.append(f"{len(ds):7d} {statistics.fmean(ds):9.2f} {statistics.median(ds):9.2f} {sum(ds) / 1e3:9.3f} "
                   f"{sum(ds) / total:6.1%}  {grid}  {name}")
    out.append(f"all kernels: {sum(len(v) for v in agg.values())} dispatches, {total / 1e3:.3f} ms")
    if window:
        out.append(window)
    return "\n".join(out)


def pmc(db: str, match: str | None) -> str:
    c = sqlite3.connect(db)
    rows = c.execute("select kernel_name, grid_size, counter_name, value from counters_collection").fetchall()
    agg = collections.defaultdict(list)
    for name, grid, counter, value in rows:
        if match and match not in name:
            continue
        agg[(_short(name), grid, counter)].append(value)
    out = [f"{'calls':>6} {'counter':>11} {'mean':>14} {'median':>14}  grid  kernel"]
    for (name, grid, counter), vs in sorted(agg.items()):
        out.append(f"{len(vs):6d} {counter:>11} {statistics.fmean(vs):14.2f} {statistics.median(vs):14.2f}  "
                   f"{grid}  {name}")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["trace", "pmc"])
    ap.add_argument("db")
    ap.add_argument("--top", type=int, default=40)
    ap.add_argument("--match")
    ap.add_argument("--after")
    a = ap.parse_args()
    print(trace(a.db, a.top, a.match, a.after) if a.mode == "trace" else pmc(a.db, a.match))


if __name__ == "__main__":
    main()
