"""Shared test set-up: import paths and the ``gpu`` marker.

``gpu`` tests need an MI355X (gfx950) and the built ``libth_hip.so``; the
CPU suite (``-m "not gpu"``) covers the oracle, the front end, the lowering
and the C ABI's host-side validation.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "torch-helion_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libth_hip.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def announce(msg: str) -> None:
    """Name the GPU case about to run (so a crash log says which)."""
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from torch_helion.hip import abi

    abi.init_device(0)
    return torch.device("cuda", 0)
