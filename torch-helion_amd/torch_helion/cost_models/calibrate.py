"""Fit the roofline cost model's per-kind efficiencies to measured kernel times.

The reference calibrates nothing on hardware: its analytic model ranks
candidates in mesh cycles and Loom reports an optimum per kernel
(reference cost_models/analytic.py:109-256; docs/cost_models.md:51-88 compare
the two). Here each kernel's ideal time is its roofline at 100% of the
MI355X peaks (``max(MFMA time, HBM time)`` with tile and wave quantisation,
roofline.py), and the model predicts

    us = ideal / efficiency[category] + waves * tile_us[category] + fixed_us[category]

with one efficiency per kernel category (bf16 / fp32 GEMM, attention, SSD,
conv1d, embedding, normalisation) and, for the GEMMs, a fixed cost per wave of
output tiles, scaled by the tile's area against 256 x 256 (pipeline fill and
epilogue: what makes a K = 1024 GEMM slower per FLOP than a K = 4096 one, and
a 64-row tile cheaper per wave than a 256-row one). ``fit`` takes runs that carry both the program
(``06_opir.json``) and measured per-kernel times (``11_bench.json``, written by
the bench stage or bench.py) and returns

* ``launch_overhead_us``: the median time of kernels whose ideal time is
  under 1 µs (their time is launch and latency, not work), the fixed part of
  every category without a fit of its own;
* for GEMM categories, ``efficiency``, ``tile_us`` and ``fixed_us`` from a
  non-negative least-squares fit of measured on (ideal, waves, 1) over all of
  the category's kernels, weighted by 1 / measured (relative error);
* for the others, ``efficiency``: the median of ideal / (measured - overhead)
  over the category's kernels whose ideal time is at least 20 µs (5 µs for the
  HBM-bound categories: conv1d, embedding, normalisation);
* ``merged_launch_factor``: the median of measured / predicted over merged
  sibling launches (several GEMM kernels on one lhs run as one th_gemm,
  priced by roofline.merged_gemm_cost with the bf16 GEMM fit), the factor the
  planner's merge-or-split decision applies to a merged launch.

``python -m torch_helion.cost_models.calibrate RUN_DIR... [--write HWSPEC]``
prints the fit and the predicted-vs-measured table, and with ``--write``
stores the fit in the hardware spec's ``calibration`` block.
"""

from __future__ import annotations

import argparse
import json
import statistics
from pathlib import Path
from typing import Any

from ..optimizer.opir import Program
from .hw_spec import HardwareSpec
from .roofline import category, kernel_cost


def _unit_spec(hw: HardwareSpec) -> HardwareSpec:
    """The same hardware at 100% efficiency and no launch overhead, uncalibrated."""
    raw = {k: v for k, v in hw.raw.items() if k != "calibration"}
    return HardwareSpec(hw.path, hw.name, hw.compute_units, hw.xcds, hw.clock_ghz, hw.lds_bytes,
                        hw.hbm_bandwidth_gbs, dict(hw.peak_tflops), {"mfma": 1.0, "hbm": 1.0, "vector": 1.0}, 0.0, raw)


def samples(run_dirs: list[Path], hw: HardwareSpec) -> list[dict[str, Any]]:
    """One record per measured kernel: name, category, ideal µs (100% roofline), measured µs."""
    unit = _unit_spec(hw)
    out = []
    for d in run_dirs:
        d = Path(d)
        prog = Program.from_json(d / "06_opir.json")
        bench = json.loads((d / "11_bench.json").read_text())
        specs = {k.name: k for k in prog.kernels}
        for name, m in bench["kernels"].items():
            if name not in specs:
                rec = _merged_sample(name, m, specs, prog, unit)
                if rec is not None:
                    out.append({"run": d.name, **rec})
                continue
            if len(m.get("entries", [])) > 1:
                # a kernel lowered to several launches (a normalised-lhs th_rmsnorm before its
                # th_gemm): its time is not one launch of the modelled kernel
                continue
            spec = specs[name]
            c = kernel_cost(spec, prog.tensors, unit)
            # (the per-wave term counts waves of 256 x 256-equivalent tiles)
            out.append({"run": d.name, "kernel": name, "category": category(spec, prog.tensors),
                        "ideal_us": max(c.t_mfma_us, c.t_hbm_us),
                        "waves": c.waves * c.detail.get("wave_scale", 1.0), "measured_us": float(m["us"]),
                        "bound": c.bound})
    return out


def _merged_sample(name: str, m: dict[str, Any], specs: dict[str, Any], prog: Program,
                   unit: HardwareSpec) -> dict[str, Any] | None:
    """A merged sibling launch ("k0_gemm+k2_gemm"): one th_gemm over the concatenated
    weights of several GEMM kernels, priced as roofline.merged_gemm_cost prices it; or a
    grouped convolution ("k1_conv1d+k4_conv1d"): one th_conv1d_causal over the members'
    channels, whose ideal time is the sum of theirs (HBM-bound, bytes add)."""
    from ..hip.epilogue import match_epilogue
    from .roofline import merged_gemm_cost

    names = name.split("+")
    if len(names) < 2 or any(n not in specs for n in names):
        return None
    members = [specs[n] for n in names]
    if all(sp.kind == "conv1d" for sp in members) and m.get("entries") == ["th_conv1d_causal"]:
        costs = [kernel_cost(sp, prog.tensors, unit) for sp in members]
        return {"kernel": name, "category": "conv1d", "ideal_us": sum(max(c.t_mfma_us, c.t_hbm_us) for c in costs),
                "waves": 0.0, "measured_us": float(m["us"]), "bound": "hbm"}
    if m.get("entries") != ["th_gemm"]:
        return None
    if any(sp.kind != "gemm" or category(sp, prog.tensors) != "gemm_bf16" for sp in members):
        return None
    used = [len({o.a for o in match_epilogue(sp).outs}) for sp in members]
    c = merged_gemm_cost(members, used, prog.tensors, unit)
    return {"kernel": name, "category": "gemm_bf16_merged", "ideal_us": max(c.t_mfma_us, c.t_hbm_us),
            "waves": c.waves * c.detail.get("wave_scale", 1.0), "measured_us": float(m["us"]), "bound": c.bound}


def fit(recs: list[dict[str, Any]]) -> dict[str, Any]:
    # (GEMM categories fit a fixed part of their own below)
    small = [r["measured_us"] for r in recs if r["ideal_us"] < 1.0 and not r["category"].startswith("gemm")]
    overhead = statistics.median(small) if small else 4.0
    eff: dict[str, float] = {}
    tile: dict[str, float] = {}
    counts: dict[str, int] = {}
    fixed: dict[str, float] = {}
    for cat in sorted({r["category"] for r in recs} - {"gemm_bf16_merged"}):
        rows = [r for r in recs if r["category"] == cat]
        if cat.startswith("gemm") and len(rows) >= 4 and len({r["waves"] for r in rows}) > 1:
            # every GEMM of the category, small ones included (their time is mostly the fixed
            # part): non-negative least squares of measured on (ideal, tile waves, 1)
            import numpy as np
            from scipy.optimize import nnls

            a = np.array([[r["ideal_us"], r["waves"], 1.0] for r in rows])
            y = np.array([r["measured_us"] for r in rows])
            # relative errors matter as much for a 10 us kernel as for a 3 ms one
            w = 1.0 / y
            (inv_eff, per_wave, c0), _ = nnls(a * w[:, None], y * w)
            counts[cat] = len(rows)
            eff[cat] = round(min(1.0, 1.0 / inv_eff), 4) if inv_eff > 0 else 1.0
            tile[cat] = round(float(per_wave), 3)
            fixed[cat] = round(float(c0), 2)
            continue
        # MFMA categories: kernels with at least 20 µs of ideal work; HBM ones: 5 µs
        floor = 20.0 if cat.startswith(("gemm", "attention", "ssd")) else 5.0
        big = [r for r in rows if r["ideal_us"] >= floor]
        if not big:
            continue
        counts[cat] = len(big)
        eff[cat] = round(statistics.median(min(1.0, r["ideal_us"] / max(r["measured_us"] - overhead, 1e-3))
                                           for r in big), 4)
    out = {"launch_overhead_us": round(overhead, 2), "efficiency": eff, "tile_us": tile, "fixed_us": fixed,
           "kernels_fitted": counts, "runs": sorted({r["run"] for r in recs})}
    # merged sibling launches: the bf16 GEMM fit of their shape times one fitted factor
    merged = [r for r in recs if r["category"] == "gemm_bf16_merged"]
    if merged and "gemm_bf16" in eff:
        base = {**out, "merged_launch_factor": 1.0}
        out["merged_launch_factor"] = round(statistics.median(r["measured_us"] / predict(r, base) for r in merged), 3)
        counts["gemm_bf16_merged"] = len(merged)
    return out


def predict(rec: dict[str, Any], calib: dict[str, Any]) -> float:
    cat, factor = rec["category"], 1.0
    if cat == "gemm_bf16_merged":
        cat, factor = "gemm_bf16", calib.get("merged_launch_factor", float("nan"))
    e = calib["efficiency"].get(cat)
    if e is None:
        return float("nan")
    return factor * (rec["ideal_us"] / e + rec["waves"] * calib.get("tile_us", {}).get(cat, 0.0) +
                     calib.get("fixed_us", {}).get(cat, calib["launch_overhead_us"]))


def report(recs: list[dict[str, Any]], calib: dict[str, Any]) -> str:
    lines = ["| run | kernel | category | ideal us | predicted us | measured us | measured / predicted |",
             "|---|---|---|---:|---:|---:|---:|"]
    for r in recs:
        p = predict(r, calib)
        lines.append(f"| {r['run']} | {r['kernel']} | {r['category']} | {r['ideal_us']:.1f} | {p:.1f} | "
                     f"{r['measured_us']:.1f} | {r['measured_us'] / p:.2f} |")
    return "\n".join(lines)


def accuracy(recs: list[dict[str, Any]], calib: dict[str, Any]) -> dict[str, Any]:
    """Median and worst |log(measured / predicted)| over the kernels the fit covers, and the
    predicted against the measured sum per run."""
    import math

    errs = [abs(math.log(r["measured_us"] / predict(r, calib))) for r in recs
            if not math.isnan(predict(r, calib))]
    runs = {}
    for r in recs:
        p = predict(r, calib)
        if math.isnan(p):
            p = r["measured_us"]   # no fit for this category: counted as measured
        t = runs.setdefault(r["run"], [0.0, 0.0])
        t[0] += p
        t[1] += r["measured_us"]
    return {"kernels": len(errs), "median_abs_log_err": round(statistics.median(errs), 3) if errs else None,
            "max_abs_log_err": round(max(errs), 3) if errs else None,
            "per_run_predicted_over_measured": {k: round(v[0] / v[1], 3) for k, v in runs.items()}}


def write(hwspec_path: Path, calib: dict[str, Any], source: str) -> None:
    d = json.loads(Path(hwspec_path).read_text())
    d["calibration"] = {**calib, "source": source}
    Path(hwspec_path).write_text(json.dumps(d, indent=2) + "\n")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("runs", nargs="+", type=Path, help="results/<run> directories with 06_opir.json and 11_bench.json")
    ap.add_argument("--hwspec", type=Path, default=None)
    ap.add_argument("--write", action="store_true", help="store the fit in the hardware spec")
    ap.add_argument("--source", default="fitted by torch_helion.cost_models.calibrate on bench.py runs")
    a = ap.parse_args()
    hw = HardwareSpec.load(a.hwspec)
    recs = samples(a.runs, hw)
    calib = fit(recs)
    calib["accuracy"] = accuracy(recs, calib)
    print(json.dumps(calib, indent=2))
    print(report(recs, calib))
    if a.write:
        write(hw.path, calib, a.source)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
