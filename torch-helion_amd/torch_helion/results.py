"""Results directory of one compilation (reference: src/torch_helion/results.py:1-53).

    results/<run_name>/
      00_model.txt  01_fx_graph.txt  01_fx_op_histogram.json
      02_opgraph_raw.{json,txt}  03_opgraph_canonical.{json,txt}  03_pass_log.json
      04_hw_spec.json  05_plan/{candidates.json,plan.md}  06_opir.{json,txt}
      07_validation.json         device parity: HIP run vs the eager model
      08_reference_check.json    CPU interpreter vs the eager model
      09_cost_report.{md,json}   roofline estimate per kernel
      11_bench.json              (bench=True) measured us, tokens/s, roofline fraction
      kernels/<kernel>.json      the HIP launch plan of each kernel
      timings.json
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any


class ResultsWriter:
    def __init__(self, run_dir: Path) -> None:
        self.run_dir = Path(run_dir)
        self.run_dir.mkdir(parents=True, exist_ok=True)
        self.files: list[Path] = []

    def path(self, name: str) -> Path:
        p = self.run_dir / name
        p.parent.mkdir(parents=True, exist_ok=True)
        return p

    def write_text(self, name: str, text: str) -> Path:
        p = self.path(name)
        p.write_text(text)
        self.files.append(p)
        return p

    def write_json(self, name: str, obj: Any) -> Path:
        return self.write_text(name, json.dumps(obj, indent=2, default=_default))

    def listing(self) -> list[str]:
        return sorted(str(p.relative_to(self.run_dir)) for p in self.run_dir.rglob("*") if p.is_file())


def _default(o: Any) -> Any:
    if hasattr(o, "to_dict"):
        return o.to_dict()
    if isinstance(o, Path):
        return str(o)
    if isinstance(o, (set, tuple)):
        return list(o)
    return str(o)
