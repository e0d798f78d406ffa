"""Benchmark targets (the reference's models/ registry, models/__init__.py:14-49)."""

from __future__ import annotations

import importlib
from typing import Any

TARGETS: dict[str, tuple[str, str, str]] = {
    "llama_block": ("targets.llama_block", "build_llama_block",
                    "one Llama-style decoder block: RMSNorm, QKV + RoPE, attention, SwiGLU MLP"),
    "mamba": ("targets.mamba", "build_mamba_model", "a Mamba-2 backbone: stacked SSD blocks with a final norm"),
    "mamba_block": ("targets.mamba", "build_mamba_block", "a single Mamba-2 block, the smallest useful SSD target"),
}


def available() -> list[str]:
    return list(TARGETS)


def describe() -> str:
    width = max(len(n) for n in TARGETS)
    return "\n".join(f"  {n:<{width}}  {d}" for n, (_, _, d) in TARGETS.items())


def resolve(name: str) -> tuple[Any, str]:
    if name not in TARGETS:
        raise KeyError(name)
    mod, fac, _ = TARGETS[name]
    return getattr(importlib.import_module(mod), fac), f"{mod}:{fac}"
