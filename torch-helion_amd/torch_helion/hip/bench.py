"""Timing of a DeviceProgram: whole-program and per-kernel, with HIP events.

Events are recorded on the stream the kernels are launched on (torch's
current stream, which every launch in :mod:`torch_helion.hip.ops` uses), so
they bracket exactly the kernels. Algorithmic work per kernel comes from the
roofline cost model (FLOPs for MFMA-bound kernels, bytes for HBM-bound ones).
"""

from __future__ import annotations

import statistics
from typing import Any

import torch

from ..cost_models.hw_spec import HardwareSpec
from ..cost_models.roofline import kernel_cost


def bench_program(dp, inputs, hw: HardwareSpec, warmup: int = 10, reps: int = 50, graph: bool = True) -> dict[str, Any]:
    """Whole-forward time (replaying the captured HIP graph when ``graph``, so
    host launch overhead is out of the timed region) and per-kernel times
    (each launch bracketed by its own events)."""
    dp.set_inputs(list(inputs))
    stream = torch.cuda.current_stream(dp.device)
    if graph and dp.graph is None:
        dp.capture()
    forward = dp.replay if graph else dp.launch_all
    for _ in range(warmup):
        forward()
    torch.cuda.synchronize(dp.device)

    # whole program: one event pair per forward
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    for i in range(reps):
        starts[i].record(stream)
        forward()
        ends[i].record(stream)
    torch.cuda.synchronize(dp.device)
    per_fwd = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))

    # per kernel (launch granularity)
    n = len(dp.launches)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
          for _ in range(max(1, reps // 2))]
    for rep in ev:
        for (s, e), l in zip(rep, dp.launches):
            s.record(stream)
            l.run()
            e.record(stream)
    torch.cuda.synchronize(dp.device)
    kernels: dict[str, dict[str, Any]] = {}
    specs = {k.name: k for k in dp.program.kernels}
    for j, l in enumerate(dp.launches):
        times = [rep[j][0].elapsed_time(rep[j][1]) * 1e3 for rep in ev]
        entry = kernels.setdefault(l.kernel, {"kind": l.kind, "entries": [], "us": 0.0})
        entry["entries"].append(l.entry)
        entry["us"] += statistics.mean(times)
    for name, entry in kernels.items():
        # a launch that merged sibling kernels ("k0_gemm+k2_gemm") carries their summed work
        members = [specs[n] for n in name.split("+")]
        costs = [kernel_cost(sp, dp.program.tensors, hw) for sp in members]
        cb = costs[0]
        if len(costs) > 1:
            bound = "mfma" if any(c.bound == "mfma" for c in costs) else costs[0].bound
            cb = type(cb)(**{**cb.__dict__, "flops": sum(c.flops for c in costs), "bytes": sum(c.bytes for c in costs),
                             "bound": bound})
        dtype = _kernel_dtype(members[0], dp.program)
        entry.update({"flops": cb.flops, "bytes": cb.bytes, "bound": cb.bound})
        sec = entry["us"] * 1e-6
        if cb.bound == "mfma":
            entry["achieved_tflops"] = cb.flops / sec / 1e12
            entry["peak_tflops"] = hw.peak_tflops.get(dtype, hw.peak_tflops["float32"])
            entry["frac"] = entry["achieved_tflops"] / entry["peak_tflops"]
        else:
            entry["achieved_gbs"] = cb.bytes / sec / 1e9
            entry["peak_gbs"] = hw.hbm_bandwidth_gbs
            entry["frac"] = entry["achieved_gbs"] / entry["peak_gbs"]
    total_flops = sum(k["flops"] for k in kernels.values())
    med = statistics.median(per_fwd)
    return {
        "us_median": med,
        "us_p10": per_fwd[max(0, int(0.1 * len(per_fwd)) - 1)],
        "us_p90": per_fwd[min(len(per_fwd) - 1, int(0.9 * len(per_fwd)))],
        "reps": reps,
        "warmup": warmup,
        "graph": bool(graph),
        "kernels": kernels,
        "total_flops": total_flops,
        "sum_kernel_us": sum(k["us"] for k in kernels.values()),
    }


def _kernel_dtype(spec, program) -> str:
    for a in spec.args:
        if a.role in ("lhs", "q", "x"):
            return program.tensors[a.tensor].dtype
    return "float32"
