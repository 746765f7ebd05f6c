"""Per-kernel summaries of rocprofv3 results databases (`*_results.db`).

    python -m dwim_amd.rocprof_summary trace RUN_results.db [--top N] [--match S] [--after K] [--split N]
    python -m dwim_amd.rocprof_summary pmc RUN_results.db [--match S] [--split N]

`trace` (from `rocprofv3 --kernel-trace`): for each kernel name and grid
size, the dispatch count, mean / median duration in µs and total ms.  With
--after K only the dispatches that start after the last dispatch of a kernel
whose name contains K count (e.g. the decode steps after a prefill), and the
window's wall time and busy share are printed.
`pmc` (from `rocprofv3 --pmc C`): for each kernel name and grid size and
each counter, the dispatch count and the mean value per dispatch.
With --split N each kernel's dispatches, in dispatch order, are summarized in
groups of N (group g: its dispatches N·g .. N·g + N − 1), so that a workload
that runs N calls of each case in turn gets a row a case.
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


def _group(key: tuple, seen: dict, split: int | None) -> tuple:
    """key, or with split, key and the dispatch's group among key's."""
    if not split:
        return key
    i = seen.get(key, 0)
    seen[key] = i + 1
    return key + (i // split,)


def trace(db: str, top: int, match: str | None, after: str | None = None, split: int | None = None) -> str:
    c = sqlite3.connect(db)
    rows = c.execute("select name, grid_x, start, end from kernels order by start").fetchall()
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
    seen: dict = {}
    for name, grid, s, e in rows:
        if match and match not in name:
            continue
        agg[_group((_short(name), grid), seen, split)].append((e - s) / 1000.0)
    total = sum(sum(v) for v in agg.values())
    out = [f"{'calls':>7} {'mean us':>9} {'median us':>9} {'total ms':>9} {'share':>6}  grid  kernel"]
    order = sorted(agg.items(), key=lambda kv: kv[0]) if split else sorted(agg.items(), key=lambda kv: -sum(kv[1]))
    for key, ds in order[:top]:
        name, grid = key[0], key[1]
        tag = f" [group {key[2]}]" if split else ""
        out.append(f"{len(ds):7d} {statistics.fmean(ds):9.2f} {statistics.median(ds):9.2f} {sum(ds) / 1e3:9.3f} "
                   f"{sum(ds) / total:6.1%}  {grid}  {name}{tag}")
    out.append(f"all kernels: {sum(len(v) for v in agg.values())} dispatches, {total / 1e3:.3f} ms")
    if window:
        out.append(window)
    return "\n".join(out)


def pmc(db: str, match: str | None, split: int | None = None) -> str:
    c = sqlite3.connect(db)
    cols = [d[0] for d in c.execute("select * from counters_collection limit 1").description]
    order = next((k for k in ("dispatch_id", "start", "correlation_id") if k in cols), "rowid")
    rows = c.execute("select kernel_name, grid_size, counter_name, value from counters_collection "
                     f"order by {order}").fetchall()
    agg = collections.defaultdict(list)
    seen: dict = {}
    for name, grid, counter, value in rows:
        if match and match not in name:
            continue
        agg[_group((_short(name), grid, counter), seen, split)].append(value)
    out = [f"{'calls':>6} {'counter':>11} {'mean':>14} {'median':>14}  grid  kernel"]
    for key, vs in sorted(agg.items()):
        name, grid, counter = key[0], key[1], key[2]
        tag = f" [group {key[3]}]" if split else ""
        out.append(f"{len(vs):6d} {counter:>11} {statistics.fmean(vs):14.2f} {statistics.median(vs):14.2f}  "
                   f"{grid}  {name}{tag}")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["trace", "pmc"])
    ap.add_argument("db")
    ap.add_argument("--top", type=int, default=40)
    ap.add_argument("--match")
    ap.add_argument("--after")
    ap.add_argument("--split", type=int)
    a = ap.parse_args()
    print(trace(a.db, a.top, a.match, a.after, a.split) if a.mode == "trace" else pmc(a.db, a.match, a.split))


if __name__ == "__main__":
    main()
