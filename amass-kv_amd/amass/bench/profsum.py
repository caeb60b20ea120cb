"""Summarise rocprofv3 SQLite output into a short text table.

    python3 -m amass.bench.profsum DB [DB ...] [--match SUBSTR ...] [--top N]

For a kernel-trace database it prints, per kernel name, the dispatch count and the
average / median / total duration; for a ``--pmc`` database it prints, per kernel
name, the per-dispatch average of every collected counter.  Only the standard
rocpd views (``kernels``, ``counters_collection``) are read.
"""
from __future__ import annotations

import argparse
import re
import sqlite3
import statistics
import sys
from collections import defaultdict


def short_name(name: str) -> str:
    """Drop the argument list and return type of a demangled kernel name."""
    s = name.strip()
    depth, cut = 0, len(s)
    for i, ch in enumerate(s):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    s = s[:cut]
    return re.sub(r"^void\s+", "", s)


def _wanted(name: str, match) -> bool:
    return not match or any(m in name for m in match)


def trace_table(db: sqlite3.Connection, match, top: int) -> list[str]:
    rows = db.execute("select name, duration from kernels").fetchall()
    by = defaultdict(list)
    for name, dur in rows:
        n = short_name(name)
        if _wanted(n, match):
            by[n].append(dur)
    if not by:
        return []
    out = [f"{'calls':>7s} {'avg_us':>10s} {'med_us':>10s} {'total_ms':>10s}  kernel"]
    for n, d in sorted(by.items(), key=lambda kv: -sum(kv[1]))[:top]:
        out.append(f"{len(d):7d} {sum(d) / len(d) / 1e3:10.2f} "
                   f"{statistics.median(d) / 1e3:10.2f} {sum(d) / 1e6:10.3f}  {n[:110]}")
    return out


def pmc_table(db: sqlite3.Connection, match, top: int) -> list[str]:
    rows = db.execute("select kernel_name, grid_size, dispatch_id, counter_name, value "
                      "from counters_collection").fetchall()
    if not rows:
        return []
    per = defaultdict(lambda: defaultdict(float))      # (kernel, dispatch) -> counter -> sum
    for kname, grid, disp, cname, val in rows:
        n = short_name(kname)
        if _wanted(n, match):
            per[(f"{n} [grid {grid}]", disp)][cname] += float(val)
    agg = defaultdict(lambda: defaultdict(list))
    for (n, _), cs in per.items():
        for c, v in cs.items():
            agg[n][c].append(v)
    counters = sorted({c for cs in agg.values() for c in cs})
    out = ["per-dispatch averages (kernel [grid size], then dispatches and counters)",
           f"{'disp':>6s} " + " ".join(f"{c:>16s}" for c in counters)]
    order = sorted(agg.items(), key=lambda kv: -max(len(v) for v in kv[1].values()))
    for n, cs in order[:top]:
        nd = max(len(v) for v in cs.values())
        vals = " ".join(f"{(sum(cs[c]) / len(cs[c]) if cs.get(c) else float('nan')):16.1f}"
                        for c in counters)
        out.append(n)
        out.append(f"{nd:6d} {vals}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("db", nargs="+")
    ap.add_argument("--match", nargs="*", default=[])
    ap.add_argument("--top", type=int, default=20)
    a = ap.parse_args(argv)
    for path in a.db:
        db = sqlite3.connect(path)
        print(f"== {path}")
        lines = pmc_table(db, a.match, a.top) or trace_table(db, a.match, a.top)
        print("\n".join(lines) if lines else "(no matching rows)")
        db.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
