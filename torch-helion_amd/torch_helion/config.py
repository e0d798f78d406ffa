"""Compile-time configuration (reference: src/torch_helion/config.py:16-66).

Every reference field is kept with its meaning; the Loom-only ones
(``verify_with_loom``, ``loom_*``, ``check_frontend``) are accepted and
ignored by the HIP backend. New fields select the backend and device, the
MI355X hardware spec, the numeric checks and the benchmark stage.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parents[2]
DEFAULT_HW_SPEC = Path(__file__).resolve().parent / "hwspec" / "mi355x.json"
DEFAULT_RESULTS_DIR = REPO_ROOT / "results"


@dataclass
class CompileConfig:
    run_name: str = "run"
    hw_spec: Path = field(default_factory=lambda: Path(os.environ.get("TORCH_HELION_HW_SPEC", DEFAULT_HW_SPEC)))
    results_dir: Path = field(default_factory=lambda: Path(os.environ.get("TORCH_HELION_RESULTS", DEFAULT_RESULTS_DIR)))
    planner_mode: str = "exhaustive"
    tile_alignment: int = 32
    max_tile: int = 512
    kernel_launch_overhead: float = 4.0          # microseconds per kernel (MI355X)
    verify_with_loom: bool = False
    loom_njobs: int = 8
    loom_topk_candidates: int = 1
    check_frontend: bool = False
    validate_workers: int = 4
    save_params: bool = False
    dtype: str = "float16"
    # --- MI355X backend
    backend: str = "hip"                          # "hip" (device) or "none" (front end only)
    device: int = 0
    verify_passes: bool | None = None             # None: only when the graph is small enough for the CPU
    reference_check: bool | None = None           # interpreter vs eager on the CPU; None: small graphs only
    device_check: bool = True                     # HIP run vs eager model (needs a GPU)
    tolerance: float = 2e-2
    bench: bool = False
    bench_warmup: int = 10
    bench_reps: int = 50
    cpu_threads: int = 0                          # 0: all cores in the process affinity
    ssd_chunk: int = 0                            # 0: 64 for sequences up to 1024, else 256
    fuse_rope: bool = True
    fp32_outputs: bool = True                     # producers of program outputs also write an fp32 copy
    residual_fp32: bool = True                    # residual operands of GEMM epilogues travel in fp32
    merge_siblings: bool | None = None            # GEMM kernels sharing an lhs run as one launch (column windows);
                                                  # None: where the planner prices one launch below the separate
                                                  # ones (optimizer/planner.py price_launch_merges; reported in
                                                  # 05_plan/plan.md); True / False: always / never
    cpu_flop_budget: float = 2e10                 # graphs above this skip CPU-side checks in "auto" mode
    reuse_buffers: bool = True                    # intermediates share device buffers by liveness
    merge_convs: bool = True                      # the depthwise convolutions feeding one SSD run as one launch
    norm_gain: str = "fold"                       # "fold": RMSNorm gains folded into the GEMM weights (the
                                                  # reference's lowering); "activation": the device normalises
                                                  # the activations with the gain (th_rmsnorm, from the fp32
                                                  # residual) and multiplies by the model's own weights; the
                                                  # bf16 rounding of g*W then never happens (deep stacks)

    @property
    def run_dir(self) -> Path:
        return Path(self.results_dir) / self.run_name

    def hw_spec_dir(self) -> Path:
        return Path(self.hw_spec).resolve().parent
