"""Planner: choose the sibling-GEMM grouping with the cost model
(reference: optimizer/planner.py:83-164).

The freedom left after canonicalisation is which sibling GEMMs share a
kernel. ``exhaustive`` enumerates every set partition of each sibling set
(Bell-number many, sets up to 6), ``greedy`` only all-merged vs all-split.
Each candidate is partitioned, checked for MI355X legality and costed with
the roofline model (``us`` per kernel plus launch overhead); the cheapest
legal candidate wins, ties broken by fewer kernels.

When the product of the per-set choices exceeds ``max_candidates`` (a deep
model: a 24-layer Mamba-2 has 48 sibling sets), the reference enumerates
only the first 512 combinations, which never varies the early layers. Here
such graphs are planned by coordinate descent instead: starting from the
first option of every set, each set in turn takes whichever of its options
lowers the program cost with the others held, so every set is decided.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from itertools import product
from typing import Any

from ..capture.opgraph import OpGraph
from ..cost_models.hw_spec import HardwareSpec
from ..cost_models.roofline import CostModelError, kernel_cost, merged_gemm_cost
from .legality import check_program
from .opir import Program
from .partition import Grouping, PartitionError, build_program, sibling_sets


@dataclass
class Candidate:
    index: int
    grouping: Grouping
    program: Program | None
    legal: bool
    total_cycles: float          # microseconds on MI355X (key kept from the reference)
    kernel_cycles: dict[str, float] = field(default_factory=dict)
    violations: list[str] = field(default_factory=list)
    error: str | None = None

    @property
    def total_us(self) -> float:
        return self.total_cycles

    def to_dict(self) -> dict[str, Any]:
        return {"index": self.index, "grouping": self.grouping, "legal": self.legal, "total_us": self.total_cycles,
                "kernel_us": self.kernel_cycles, "kernels": [k.name for k in self.program.kernels] if self.program else [],
                "violations": self.violations, "error": self.error}


@dataclass
class PlanResult:
    best: Candidate
    candidates: list[Candidate]

    @property
    def program(self) -> Program:
        assert self.best.program is not None
        return self.best.program


def set_partitions(items: list[str]) -> list[list[list[str]]]:
    if not items:
        return [[]]
    first, rest = items[0], items[1:]
    out = []
    for part in set_partitions(rest):
        out.append([[first]] + part)
        for i in range(len(part)):
            out.append(part[:i] + [[first] + part[i]] + part[i + 1:])
    return out


MAX_CANDIDATES = 512


def set_options(g: OpGraph, mode: str = "exhaustive") -> list[list[list[list[str]]]]:
    """Per sibling set, the partitions of it the planner may choose from."""
    per_set = []
    for s in sibling_sets(g):
        if mode == "exhaustive" and len(s) <= 6:
            per_set.append(set_partitions(s))
        else:
            per_set.append([[list(s)], [[m] for m in s]] if len(s) > 1 else [[list(s)]])
    return per_set


def grouping_of(combo) -> Grouping:
    grouping: Grouping = {}
    gid = 0
    for part in combo:
        for block in part:
            for m in block:
                grouping[m] = gid
            gid += 1
    return grouping


def enumerate_groupings(g: OpGraph, mode: str = "exhaustive", max_candidates: int = MAX_CANDIDATES) -> list[Grouping]:
    groupings: list[Grouping] = []
    for combo in product(*set_options(g, mode)):
        groupings.append(grouping_of(combo))
        if len(groupings) >= max_candidates:
            break
    return groupings


def kernel_signature(spec, tensors) -> str:
    """Structural key of a kernel (its name aside) for cost memoisation."""
    body = [(b.op, tuple(b.inputs), json.dumps(b.attrs, sort_keys=True, default=str)) for b in spec.epilogue]
    key = (spec.kind, spec.k_extent, tuple(sorted(spec.grid.items())), spec.sumsq,
           tuple((gm.acc, gm.rhs) for gm in spec.gemms), tuple(body),
           json.dumps(spec.attrs, sort_keys=True, default=str),
           tuple((a.name, a.role, tuple(a.view or ()), tuple(tensors[a.tensor].shape), tensors[a.tensor].dtype)
                 for a in spec.args),
           tuple(o.value for o in spec.outputs))
    return repr(key)


def cost_program(program: Program, hw: HardwareSpec, config=None, memo: dict[str, Any] | None = None) -> tuple[float, dict[str, float]]:
    total, per = 0.0, {}
    memo = {} if memo is None else memo
    for spec in program.kernels:
        key = kernel_signature(spec, program.tensors)
        cb = memo.get(key)
        if cb is None:
            cb = memo[key] = kernel_cost(spec, program.tensors, hw)
        spec.tiles = dict(cb.tiles)
        spec.cost = {"us": cb.us, "cycles": cb.us, "bound": cb.bound, "flops": cb.flops, "bytes": cb.bytes,
                     "breakdown": cb.to_dict()}
        per[spec.name] = cb.us
        total += cb.us
    return total, per


def _evaluate(g: OpGraph, grouping: Grouping, index: int, hw: HardwareSpec, config, name: str,
              memo: dict[str, Any]) -> Candidate:
    try:
        program = build_program(g, grouping, name=name)
    except PartitionError as e:
        return Candidate(index, grouping, None, False, float("inf"), error=str(e))
    rep = check_program(program)
    if not rep.ok:
        return Candidate(index, grouping, program, False, float("inf"), violations=[str(v) for v in rep.violations])
    try:
        total, per = cost_program(program, hw, config, memo)
    except CostModelError as e:
        return Candidate(index, grouping, program, False, float("inf"), error=str(e))
    return Candidate(index, grouping, program, True, total, per)


def _better(a: Candidate, b: Candidate) -> bool:
    if not a.legal:
        return False
    return not b.legal or (a.total_cycles, len(a.program.kernels)) < (b.total_cycles, len(b.program.kernels))


def plan(g: OpGraph, hw: HardwareSpec, config, name: str = "program") -> PlanResult:
    mode = getattr(config, "planner_mode", "exhaustive")
    candidates: list[Candidate] = []
    memo: dict[str, Any] = {}
    options = set_options(g, mode)
    n_combos = 1
    for o in options:
        n_combos *= len(o)
    if n_combos <= MAX_CANDIDATES:
        for i, grouping in enumerate(enumerate_groupings(g, mode)):
            candidates.append(_evaluate(g, grouping, i, hw, config, name, memo))
    else:
        choice = [0] * len(options)
        cur = _evaluate(g, grouping_of([o[0] for o in options]), 0, hw, config, name, memo)
        candidates.append(cur)
        for si, opts in enumerate(options):
            for oi in range(1, len(opts)):
                trial = list(choice)
                trial[si] = oi
                c = _evaluate(g, grouping_of([o[j] for o, j in zip(options, trial)]), len(candidates), hw, config,
                              name, memo)
                candidates.append(c)
                if _better(c, cur):
                    cur, choice = c, trial
    legal = [c for c in candidates if c.legal]
    if not legal:
        details = "\n".join(f"  candidate {c.index}: {c.error or c.violations}" for c in candidates[:10])
        raise PartitionError(f"no legal partition among {len(candidates)} candidates:\n{details}")
    best = min(legal, key=lambda c: (c.total_cycles, len(c.program.kernels)))
    best.program.metadata["plan"] = {"candidates": len(candidates), "legal": len(legal), "total_us": best.total_cycles,
                                     "total_cycles": best.total_cycles, "kernel_us": best.kernel_cycles,
                                     "launch_overhead_us": hw.launch_overhead_us}
    return PlanResult(best, candidates)


# ---------------------------------------------------------------- launch merges
# After the partition, a backend may still run several GEMM kernels as one
# launch: kernels that multiply the same lhs by different weights (projections
# the partition kept apart because their widths or epilogue ops differ) become
# one GEMM over the concatenated weights, each output on its own column window.
# Which groups CAN merge is structural (the HIP runtime's _plan_sibling_merges);
# whether they SHOULD is decided here with the cost model: the group's kernels
# as separate launches (each with its launch overhead and its own wave and tile
# quantisation) against one launch of the concatenated width.


@dataclass
class LaunchMerge:
    members: list[str]
    split_us: float
    merged_us: float

    @property
    def merged(self) -> bool:
        return self.merged_us < self.split_us

    def to_dict(self) -> dict[str, Any]:
        return {"members": self.members, "split_us": self.split_us, "merged_us": self.merged_us,
                "merged": self.merged}


def price_launch_merges(program: Program, groups: list[list[tuple[str, int]]], hw: HardwareSpec) -> list[LaunchMerge]:
    """Each group (kernel name, accumulators it contributes) priced split and merged."""
    kern = {k.name: k for k in program.kernels}
    out = []
    for g in groups:
        specs = [kern[n] for n, _ in g]
        split = sum(kernel_cost(sp, program.tensors, hw).us for sp in specs)
        merged = merged_gemm_cost(specs, [u for _, u in g], program.tensors, hw).us
        out.append(LaunchMerge([n for n, _ in g], split, merged))
    return out


def launch_merge_report(merges: list[LaunchMerge]) -> str:
    lines = ["## Launch merges (HIP backend)", "",
             "Sibling GEMM kernels reading one lhs, priced as separate launches and as one launch over",
             "their concatenated weights (calibrated cost model, launch overhead included).", "",
             "| kernels | split us | merged us | decision |", "|---|---:|---:|---|"]
    for m in merges:
        lines.append(f"| {' + '.join(m.members)} | {m.split_us:,.1f} | {m.merged_us:,.1f} | "
                     f"{'merged' if m.merged else 'split'} |")
    if not merges:
        lines.append("| (none: no two GEMM kernels share an lhs) | | | |")
    return "\n".join(lines)
