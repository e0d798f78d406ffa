"""Measure the device's MFMA and HBM peaks and record them beside the published ones.

The hardware spec's ``peak_tflops`` and ``hbm_bandwidth_gbs`` are AMD's published
MI355X figures (dense MFMA per dtype, 8 TB/s); the roofline fractions bench.py
reports divide by those. This runs the peak probe (``hwspec/probe.hip``, built
into ``lib/th_probe`` by ``hip.build.build_probe``) in a child process and, with
``--write``, stores what it measured in the spec's ``measured`` block:

* ``mfma_tflops``: dense rate of the three MFMA instructions the kernels issue
  (32x32x16 and 16x16x32 bf16, 32x32x2 fp32), register operands, every SIMD busy;
* ``hbm_read_gbs`` / ``hbm_copy_gbs``: 16-byte streaming loads over 4 GiB (16x the
  Infinity Cache) and a 2 GiB copy counting read plus write bytes.

The cost model keeps pricing against the published peaks (a fitted efficiency per
kernel category absorbs the gap); the measured block says how large that gap is
for the hardware itself, apart from any kernel of this library.

``python -m torch_helion.cost_models.measure_peaks [--write] [--hwspec PATH]``
"""

from __future__ import annotations

import argparse
import json
import subprocess
from pathlib import Path

from ..hip.build import PROBE_PATH
from .hw_spec import HardwareSpec


def measure(probe: Path = PROBE_PATH, timeout: float = 120.0) -> dict:
    """Run the probe (a separate process: it initialises the GPU itself) and parse its JSON line."""
    if not Path(probe).exists():
        raise FileNotFoundError(f"{probe} is not built (torch_helion.hip.build.build_probe)")
    r = subprocess.run([str(probe)], capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"{probe} exited with {r.returncode}: {r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def with_fractions(m: dict, hw: HardwareSpec) -> dict:
    """The measured figures plus each one's ratio to the published peak it corresponds to."""
    pub_bf16, pub_f32 = hw.peak_tflops["bfloat16"], hw.peak_tflops["float32"]
    frac = {
        "bfloat16_32x32x16": m["mfma_tflops"]["bfloat16_32x32x16"] / pub_bf16,
        "bfloat16_16x16x32": m["mfma_tflops"]["bfloat16_16x16x32"] / pub_bf16,
        "float32_32x32x2": m["mfma_tflops"]["float32_32x32x2"] / pub_f32,
        "hbm_read": m["hbm_read_gbs"] / hw.hbm_bandwidth_gbs,
        "hbm_copy": m["hbm_copy_gbs"] / hw.hbm_bandwidth_gbs,
    }
    return {**m, "fraction_of_published": {k: round(v, 3) for k, v in frac.items()}}


def write(hwspec_path: Path, measured: dict) -> None:
    d = json.loads(Path(hwspec_path).read_text())
    d["measured"] = measured
    Path(hwspec_path).write_text(json.dumps(d, indent=2) + "\n")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--hwspec", type=Path, default=None)
    ap.add_argument("--write", action="store_true", help="store the figures in the spec's 'measured' block")
    a = ap.parse_args()
    hw = HardwareSpec.load(a.hwspec)
    m = with_fractions(measure(), hw)
    print(json.dumps(m, indent=2))
    if a.write:
        write(hw.path, m)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
