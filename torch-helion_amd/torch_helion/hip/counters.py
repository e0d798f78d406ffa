"""Per-kernel hardware counters of a program run, from ``rocprofv3 --pmc`` CSV output.

    python -m torch_helion.hip.counters RUN_DIR PASS.csv [PASS.csv ...] --period P [--reps R]

``rocprofv3 --pmc`` writes one row per (dispatch, counter). Only this
library's dispatches (symbols in namespace ``th::``) are kept; the last
``reps`` repetitions of a ``period``-dispatch sequence at the end of the run
(bench_program's per-kernel timing pass ends every workload with such
repetitions of the program's launch list) are averaged per position, and the
positions are named after the program's launches (``kernels/launches.json``)
when every launch is one dispatch. Several passes (one per counter group: the
hardware collects a few counters per run) merge by position.

Derived figures, per position, when the counters are present:
* ``mfma_util`` = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE / XCDs):
  the MFMA busy cycles summed over every SIMD (on gfx950 each
  v_mfma_f32_32x32x16_bf16 adds its 32 cycles) over the SIMD-cycles the
  kernel had (GRBM_GUI_ACTIVE is summed over the XCDs);
* ``clock_ghz`` = GRBM_GUI_ACTIVE / XCDs / dispatch duration: the clock the
  part held during the kernel;
FETCH_SIZE / WRITE_SIZE are kept in KiB as read (on this part FETCH_SIZE reads
half the bytes of a calibrated copy, WRITE_SIZE all of them).
The result goes to ``10_device_counters.json`` in the run directory. With
``--by-symbol`` the tool prints a markdown table instead of the positions:
one row per kernel symbol (template arguments kept, parameters dropped),
averaged over its positions; positions of one symbol whose dispatches last more
than ``--split-us`` (default: never) form a row of their own, marked "long".
"""

from __future__ import annotations

import argparse
import csv
import json
from collections import defaultdict
from pathlib import Path


def read_passes(paths: list[Path], match: str = "th::") -> list[tuple[str, dict[str, float]]]:
    """Dispatches in order: (kernel symbol, {counter: value}) merged over the passes by index
    (each dispatch also carries ``duration_us`` from its timestamps)."""
    merged: list[tuple[str, dict[str, float]]] | None = None
    for p in paths:
        per: dict[int, tuple[str, dict[str, float]]] = {}
        with open(p, newline="") as f:
            for r in csv.DictReader(f):
                if match not in r["Kernel_Name"]:
                    continue
                d = int(r["Dispatch_Id"])
                name, vals = per.setdefault(d, (r["Kernel_Name"], defaultdict(float)))
                vals[r["Counter_Name"]] += float(r["Counter_Value"])
                vals["duration_us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        seq = [per[d] for d in sorted(per)]
        if merged is None:
            merged = [(n, dict(v)) for n, v in seq]
        else:
            # the same program replayed: align the passes from the end
            k = min(len(merged), len(seq))
            merged = merged[-k:]
            for i in range(k):
                merged[i][1].update(seq[len(seq) - k + i][1])
    return merged or []


def per_position(seq, period: int, reps: int, simds: int = 1024, xcds: int = 8) -> list[dict]:
    tail = seq[-period * reps:]
    if len(tail) < period * reps:
        raise ValueError(f"only {len(seq)} dispatches for {reps} repetitions of {period}")
    out = []
    for j in range(period):
        rows = [tail[r * period + j] for r in range(reps)]
        names = {n for n, _ in rows}
        keys = set().union(*(v.keys() for _, v in rows))
        avg = {k: sum(v.get(k, 0.0) for _, v in rows) / reps for k in sorted(keys)}
        gui = avg.get("GRBM_GUI_ACTIVE")
        if gui:
            if "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
                avg["mfma_util"] = avg["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * gui / xcds)
            if avg.get("duration_us"):
                avg["clock_ghz"] = gui / xcds / (avg["duration_us"] * 1e3)
        out.append({"position": j, "symbol": sorted(names)[0][:120], "consistent": len(names) == 1, **avg})
    return out


def by_symbol(pos: list[dict], split_us: float | None = None) -> str:
    """Markdown table of the positions grouped by kernel symbol, longest total first."""
    groups: dict[str, list[dict]] = {}
    for p in pos:
        sym = p.get("symbol", "?")
        sym = sym[5:] if sym.startswith("void ") else sym
        sym = sym[: sym.index("(")] if "(" in sym else sym
        if split_us is not None and p.get("duration_us", 0.0) > split_us:
            sym += " (long)"
        groups.setdefault(sym, []).append(p)

    def avg(ps: list[dict], k: str) -> float:
        v = [x[k] for x in ps if k in x]
        return sum(v) / len(v) if v else float("nan")

    rows = sorted(groups.items(), key=lambda kv: -avg(kv[1], "duration_us") * len(kv[1]))
    out = ["| kernel symbol | per run | avg us (under counters) | MFMA util | clock GHz | FETCH_SIZE MiB (as read) "
           "| WRITE_SIZE MiB |", "|---|---:|---:|---:|---:|---:|---:|"]
    for sym, ps in rows:
        out.append(f"| `{sym}` | {len(ps)} | {avg(ps, 'duration_us'):.1f} | {100 * avg(ps, 'mfma_util'):.1f}% | "
                   f"{avg(ps, 'clock_ghz'):.2f} | {avg(ps, 'FETCH_SIZE') / 1024:.1f} | {avg(ps, 'WRITE_SIZE') / 1024:.1f} |")
    return "\n".join(out)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("run_dir", type=Path)
    ap.add_argument("csv", nargs="+", type=Path)
    ap.add_argument("--period", type=int, required=True, help="dispatches of one program run")
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--by-symbol", action="store_true", help="print a markdown table per kernel symbol")
    ap.add_argument("--split-us", type=float, default=None, help="with --by-symbol: longer dispatches get their own row")
    a = ap.parse_args()
    from ..cost_models.hw_spec import HardwareSpec

    hw = HardwareSpec.load(None)
    pos = per_position(read_passes(a.csv), a.period, a.reps, simds=hw.compute_units * int(hw.raw.get("simds_per_cu", 4)),
                       xcds=hw.xcds)
    launches_file = a.run_dir / "kernels" / "launches.json"
    if launches_file.exists():
        launches = json.loads(launches_file.read_text())
        if len(launches) == a.period:
            for p, l in zip(pos, launches):
                p["kernel"] = l["kernel"]
    (a.run_dir / "10_device_counters.json").write_text(json.dumps(pos, indent=2))
    if a.by_symbol:
        print(by_symbol(pos, a.split_us))
        return 0
    for p in pos:
        print({k: (round(v, 4) if isinstance(v, float) else v) for k, v in p.items() if k != "symbol"})
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
