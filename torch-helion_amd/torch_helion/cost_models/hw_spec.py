"""Hardware description for the cost model and planner.

The reference reads a Loom ADL/MLIR mesh description plus perf YAMLs
(reference: cost_models/hw_spec.py:88-166). The MI355X entry is a plain JSON
file (``hwspec/mi355x.json``): CU count, XCDs, clock, LDS, HBM bandwidth and
dense MFMA peaks per dtype, which is all a roofline model needs.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

DEFAULT_HW_SPEC = Path(__file__).resolve().parents[1] / "hwspec" / "mi355x.json"


@dataclass
class HardwareSpec:
    path: Path
    name: str
    compute_units: int
    xcds: int
    clock_ghz: float
    lds_bytes: int
    hbm_bandwidth_gbs: float
    peak_tflops: dict[str, float]
    efficiency: dict[str, float] = field(default_factory=dict)
    launch_overhead_us: float = 4.0
    raw: dict[str, Any] = field(default_factory=dict)

    @property
    def calibration(self) -> dict[str, Any]:
        """Per-category efficiencies and launch overhead fitted to measured kernel times
        (cost_models/calibrate.py); empty when the spec carries none."""
        return self.raw.get("calibration", {})

    @staticmethod
    def load(path: str | Path | None = None) -> "HardwareSpec":
        p = Path(path) if path else DEFAULT_HW_SPEC
        if p.suffix != ".json" or not p.exists():
            # a Loom mesh description (the reference's default) has no MI355X meaning
            p = DEFAULT_HW_SPEC
        d = json.loads(p.read_text())
        return HardwareSpec(p, d["name"], int(d["compute_units"]), int(d.get("xcds", 1)), float(d["clock_ghz"]),
                            int(d["lds_bytes_per_cu"]), float(d["hbm_bandwidth_gbs"]), dict(d["peak_tflops"]),
                            dict(d.get("efficiency", {})), float(d.get("launch_overhead_us", 4.0)), d)

    @property
    def cores(self) -> int:
        return self.compute_units

    @property
    def l1_bytes(self) -> int:
        return self.lds_bytes

    @property
    def mesh(self) -> tuple[int, int]:
        return (self.xcds, self.compute_units // max(self.xcds, 1))

    def peak_flops(self, dtype: str) -> float:
        return self.peak_tflops.get(dtype, self.peak_tflops["float32"]) * 1e12

    def hbm_bytes_per_s(self) -> float:
        return self.hbm_bandwidth_gbs * 1e9

    def summary(self) -> dict[str, Any]:
        return {"path": str(self.path), "name": self.name, "compute_units": self.compute_units, "xcds": self.xcds,
                "clock_ghz": self.clock_ghz, "lds_bytes_per_cu": self.lds_bytes,
                "hbm_bandwidth_gbs": self.hbm_bandwidth_gbs, "peak_tflops": self.peak_tflops,
                "efficiency": self.efficiency, "launch_overhead_us": self.launch_overhead_us,
                "calibration": self.calibration}
