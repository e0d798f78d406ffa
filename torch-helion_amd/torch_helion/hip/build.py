"""Build ``libth_hip.so`` (the gfx950 kernel library) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object under ``_build/`` and the
objects are linked into ``torch_helion/lib/libth_hip.so``. The library is
loaded with ctypes after ``import torch``, so it binds to the HIP runtime torch
already mapped (same SONAME), giving one runtime per process.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parents[1]          # torch_helion/
PROJECT = PKG_ROOT.parent                               # torch-helion_amd/
REPO = PROJECT.parent
CSRC = PROJECT / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = PROJECT / "_build"
LIB_PATH = PKG_ROOT / "lib" / "libth_hip.so"
PROBE_SRC = PKG_ROOT / "hwspec" / "probe.hip"
PROBE_PATH = PKG_ROOT / "lib" / "th_probe"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    # packed-fp32 VALU forms are kept out of every code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the HIP backend needs ROCm to build")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-4000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every kernel source and link the shared library. Always rebuilds."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_PATH.parent.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of libth_hip.so failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


def build_probe(verbose: bool = False) -> Path:
    """Compile the peak probe (MFMA rate, HBM stream bandwidth; hwspec/probe.hip) into an
    executable beside the library. cost_models.measure_peaks runs it."""
    PROBE_PATH.parent.mkdir(parents=True, exist_ok=True)
    tmp = PROBE_PATH.with_suffix(".tmp")
    cmd = [hipcc(), *[f for f in HIPCC_FLAGS if f != "-fPIC"], str(PROBE_SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC.name}:\n{r.stderr[-4000:]}")
    os.replace(tmp, PROBE_PATH)
    if verbose:
        print(f"built {PROBE_PATH}")
    return PROBE_PATH


if __name__ == "__main__":
    build(verbose=True)
    build_probe(verbose=True)
