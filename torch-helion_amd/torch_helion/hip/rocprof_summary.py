"""Summarise a ``rocprofv3 --kernel-trace`` database (rocpd SQLite output).

    python -m torch_helion.hip.rocprof_summary RESULTS.db [--period P --reps R --labels k0,k1,... --match th::
                                                           --skip N]

Prints a markdown table of every kernel symbol (calls, average / total time,
share of the traced kernel time). Several program kernels can share one
compiled symbol (the persistent GEMM serves every projection of a block), so
``--period P --reps R`` also reports the average duration of each position
of the last R repetitions of a P-launch sequence at the end of the trace --
the per-kernel timing pass of ``torch_helion.hip.bench.bench_program`` ends
every workload with exactly such repetitions of the program's launch list.
Only dispatches whose symbol contains ``--match`` (default ``th::``, this
library's kernels) enter the sequence view, so host copies and torch fills
after the timed region do not shift it. ``--skip N`` drops the last N of those
matched dispatches first, so the window can end before a later leg of the same
run (another launch list timed after the one of interest).
"""

from __future__ import annotations

import argparse
import sqlite3
import statistics
from collections import defaultdict


def load(db_path: str) -> list[tuple[str, int, int, int]]:
    """(name, start ns, end ns, grid_x) of every kernel dispatch, in start order."""
    db = sqlite3.connect(db_path)
    rows = db.execute("select name, start, end, grid_x from kernels order by start").fetchall()
    db.close()
    return [(r[0], int(r[1]), int(r[2]), int(r[3])) for r in rows]


def table(rows) -> str:
    total = sum(e - s for _, s, e, _ in rows) or 1
    agg: dict[str, list[int]] = defaultdict(list)
    for name, s, e, _ in rows:
        agg[name].append(e - s)
    out = ["| kernel | calls | avg us | total ms | share |", "|---|---:|---:|---:|---:|"]
    for name, ds in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| `{name[:96]}` | {len(ds)} | {statistics.mean(ds) / 1e3:.2f} | {sum(ds) / 1e6:.3f} | "
                   f"{sum(ds) / total:.1%} |")
    return "\n".join(out)


def sequence(rows, period: int, reps: int, labels: list[str] | None) -> str:
    tail = rows[-period * reps:]
    if len(tail) < period * reps:
        return "(trace shorter than period x reps)"
    out = ["| position | kernel symbol | avg us | min us | max us |", "|---|---|---:|---:|---:|"]
    for i in range(period):
        ds = [tail[r * period + i][2] - tail[r * period + i][1] for r in range(reps)]
        names = {tail[r * period + i][0] for r in range(reps)}
        name = names.pop() if len(names) == 1 else "(differs between repetitions)"
        lab = labels[i] if labels and i < len(labels) else str(i)
        out.append(f"| {lab} | `{name[:80]}` | {statistics.mean(ds) / 1e3:.2f} | {min(ds) / 1e3:.2f} | "
                   f"{max(ds) / 1e3:.2f} |")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("db")
    ap.add_argument("--period", type=int, default=0)
    ap.add_argument("--reps", type=int, default=0)
    ap.add_argument("--labels", default="")
    ap.add_argument("--match", default="th::")
    ap.add_argument("--skip", type=int, default=0)
    a = ap.parse_args(argv)
    rows = load(a.db)
    print(f"{len(rows)} kernel dispatches, {sum(e - s for _, s, e, _ in rows) / 1e6:.3f} ms of kernel time\n")
    print(table(rows))
    if a.period and a.reps:
        skip = f" ending {a.skip} matched dispatches before the last" if a.skip else ""
        print(f"\nlast {a.reps} repetitions of the {a.period}-launch sequence{skip}:\n")
        seq = [r for r in rows if a.match in r[0]]
        seq = seq[:len(seq) - a.skip] if a.skip else seq
        print(sequence(seq, a.period, a.reps, a.labels.split(",") if a.labels else None))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
