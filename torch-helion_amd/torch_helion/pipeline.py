"""compile_model: PyTorch model -> OpGraph -> OpIR -> MI355X HIP kernels.

::

    from torch_helion import compile_model, CompileConfig
    res = compile_model(model, example_args, CompileConfig(run_name="llama_block"))
    print(res.program.summary())
    out = res.run(*example_args)            # on the GPU, through libth_hip.so

Stages as in the reference (reference: pipeline.py:60-145): capture,
canonicalize, plan, codegen (here: HIP launch plans + device binding),
reference_check (CPU interpreter vs eager), then the MI355X additions:
device_check (HIP run vs the eager model in fp32) and an optional bench.
"""

from __future__ import annotations

import copy
import logging
import math
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Sequence

import torch

from .capture import CapturedFx, OpGraph, capture
from .codegen.emit import emit_program
from .codegen.interpret import program_outputs
from .config import CompileConfig
from .cost_models.hw_spec import HardwareSpec
from .optimizer.evaluate import max_rel_err
from .optimizer.opir import Program
from .optimizer.passes import canonicalize
from .optimizer.planner import PlanResult, plan
from .results import ResultsWriter

log = logging.getLogger("torch_helion")


@dataclass
class CompileResult:
    config: CompileConfig
    run_dir: Path
    fx: CapturedFx
    raw_graph: OpGraph
    graph: OpGraph
    hw: HardwareSpec
    plan: PlanResult
    program: Program
    kernel_files: dict[str, Path]
    validation: dict[str, Any] = field(default_factory=dict)
    reference_check: dict[str, Any] = field(default_factory=dict)
    loom_results: dict[str, Any] = field(default_factory=dict)
    timings: dict[str, float] = field(default_factory=dict)
    device_program: Any = None
    bench: dict[str, Any] = field(default_factory=dict)

    @property
    def estimated_cycles(self) -> float:
        """Estimated program time (µs on MI355X; key name kept from the reference)."""
        return self.program.metadata.get("plan", {}).get("total_us", float("nan"))

    def run(self, *args) -> list[torch.Tensor]:
        if self.device_program is None:
            raise RuntimeError("no device program: compile with backend='hip' on a machine with an MI355X")
        return self.device_program.run(list(args))


def _graph_flops(g: OpGraph) -> float:
    total = 0.0
    for n in g:
        if n.op in ("matmul", "batch_matmul") and len(n.inputs) == 2:
            total += 2.0 * math.prod(n.type.shape) * g[n.inputs[0]].type.shape[-1]
    return total


def eager_reference(model: torch.nn.Module, args: Sequence[Any], batch_slice: int | None = None) -> list[torch.Tensor]:
    """The model in fp32 on the CPU (optionally on the first ``batch_slice``
    sequences only: every config here is independent across the batch)."""
    m = copy.deepcopy(model).float().cpu().eval()
    xs = []
    for a in args:
        if isinstance(a, torch.Tensor):
            a = a.detach().cpu()
            if batch_slice is not None:
                a = a[:batch_slice]
            xs.append(a.float() if a.is_floating_point() else a)
        else:
            xs.append(a)
    with torch.inference_mode():
        out = m(*xs)
    return list(out) if isinstance(out, (list, tuple)) else [out]


def compile_model(model: torch.nn.Module, example_args: Sequence[Any], config: CompileConfig | None = None) -> CompileResult:
    config = config or CompileConfig()
    if getattr(model, "is_decode_step", False):
        # a decode step (one token per sequence against a KV cache, e4m3 weights): its OpIR
        # is derived from the block's own S = 1 capture (torch_helion/decode.py)
        from .decode import compile_decode

        return compile_decode(model, example_args, config)
    rw = ResultsWriter(config.run_dir)
    timings: dict[str, float] = {}

    class stage:
        def __init__(self, name: str) -> None:
            self.name = name

        def __enter__(self):
            self.t = time.time()
            log.info("stage %s", self.name)

        def __exit__(self, *exc):
            timings[self.name] = time.time() - self.t

    with stage("capture"):
        fx, raw = capture(model, example_args)
        rw.write_text("00_model.txt", f"{model!r}\n\nconfig: {config!r}\n")
        rw.write_text("01_fx_graph.txt", fx.text())
        rw.write_json("01_fx_op_histogram.json", fx.op_histogram())
        raw.to_json(rw.path("02_opgraph_raw.json"))
        rw.write_text("02_opgraph_raw.txt", raw.summary())

    small = _graph_flops(raw) <= config.cpu_flop_budget
    verify = small if config.verify_passes is None else config.verify_passes
    with stage("canonicalize"):
        graph, pass_log = canonicalize(raw, verify_inputs=list(example_args) if verify else None,
                                       tolerance=config.tolerance, ssd_chunk=config.ssd_chunk)
        graph.to_json(rw.path("03_opgraph_canonical.json"))
        rw.write_text("03_opgraph_canonical.txt", graph.summary())
        rw.write_json("03_pass_log.json", pass_log)

    with stage("plan"):
        hw = HardwareSpec.load(config.hw_spec)
        rw.write_json("04_hw_spec.json", hw.summary())
        result = plan(graph, hw, config, name=config.run_name)
        program = result.program
        rw.write_json("05_plan/candidates.json", [c.to_dict() for c in result.candidates])
        rw.write_text("05_plan/plan.md", plan_report(result, hw, config))
        program.to_json(rw.path("06_opir.json"))
        rw.write_text("06_opir.txt", program.summary())

    device_program = None
    with stage("codegen"):
        kernel_files = emit_program(program, config, rw.path("kernels"))
        if config.save_params:
            torch.save({n: graph.params[n] for n in program.params}, rw.path("params.pt"))
        if config.backend == "hip":
            from .hip.runtime import DeviceProgram

            if config.norm_gain not in ("fold", "activation"):
                raise ValueError(f"CompileConfig.norm_gain must be 'fold' or 'activation', not {config.norm_gain!r}")
            device_program = DeviceProgram(program, graph.params, config.device, fuse_rope=config.fuse_rope,
                                           fp32_outputs=config.fp32_outputs, residual_fp32=config.residual_fp32,
                                           merge_siblings=config.merge_siblings,
                                           fold_sources=graph.fold_sources if config.norm_gain == "activation"
                                           else None, reuse_buffers=config.reuse_buffers,
                                           merge_convs=config.merge_convs, hw=hw)
            rw.write_json("kernels/launches.json", [{"kernel": l.kernel, "entry": l.entry, "info": l.info}
                                                    for l in device_program.launches])
            if device_program.launch_merges:
                from .optimizer.planner import launch_merge_report

                program.metadata["launch_merges"] = [m.to_dict() for m in device_program.launch_merges]
                rw.write_text("05_plan/plan.md", plan_report(result, hw, config) + "\n\n" +
                              launch_merge_report(device_program.launch_merges) + "\n")
                program.to_json(rw.path("06_opir.json"))

    reference_check: dict[str, Any] = {}
    do_ref = small if config.reference_check is None else config.reference_check
    if do_ref:
        with stage("reference_check"):
            with torch.no_grad():
                ref = model(*example_args)
            outs = program_outputs(program, graph.params, list(example_args))
            refs = ref if isinstance(ref, (list, tuple)) else [ref]
            errs = [max_rel_err(o.reshape(-1), r.reshape(-1)) for o, r in zip(outs, refs)]
            reference_check = {"max_rel_err": max(errs), "per_output": errs, "tolerance": config.tolerance,
                               "ok": max(errs) <= config.tolerance}
            rw.write_json("08_reference_check.json", reference_check)

    validation: dict[str, Any] = {}
    if device_program is not None and config.device_check:
        with stage("device_check"):
            validation = device_check(model, example_args, device_program, config, small)
            rw.write_json("07_validation.json", validation)

    rw.write_json("09_cost_report.json", cost_report_json(program, hw, config))
    rw.write_text("09_cost_report.md", cost_report_md(program, hw, config))

    res = CompileResult(config, rw.run_dir, fx, raw, graph, hw, result, program, kernel_files, validation,
                        reference_check, {}, timings, device_program)
    if config.bench and device_program is not None:
        from .hip.bench import bench_program

        with stage("bench"):
            res.bench = bench_program(device_program, example_args, hw, warmup=config.bench_warmup,
                                      reps=config.bench_reps)
            write_device_results(rw.run_dir, program, hw, res.bench)
    rw.write_json("timings.json", timings)
    return res


def device_check(model, example_args, dp, config: CompileConfig, small: bool) -> dict[str, Any]:
    """HIP run vs the eager model in fp32 (first sequence only for large graphs)."""
    dp.run(list(example_args))
    outs = dp.outputs(fp32=True)
    torch.cuda.synchronize()
    batch_slice = None if small else 1
    refs = eager_reference(model, example_args, batch_slice)
    res: dict[str, Any] = {"batch_slice": batch_slice, "outputs": []}
    ok = True
    for o, r in zip(outs, refs):
        o = o.float().cpu()
        if batch_slice is not None:
            o = o[:batch_slice]
        o = o.reshape(r.shape)
        rel = max_rel_err(o.reshape(-1), r.reshape(-1))
        mab = float((o - r).abs().max())
        dtype = str(dp.program.tensors[dp.program.outputs[0]].dtype)
        # fp32: 1e-4 relative; bf16/fp16: the reference's normalised max_rel_err bound
        # (max|a-b| / max|b|, pipeline.py:115-117 of the reference), max-abs reported beside it
        passed = (rel <= 1e-4) if dtype == "float32" else (rel <= config.tolerance)
        ok &= passed
        res["outputs"].append({"max_rel_err": rel, "max_abs_err": mab, "dtype": dtype, "ok": passed,
                               "finite": bool(torch.isfinite(o).all())})
    res["ok"] = ok
    return res


# ------------------------------------------------------------------ reports
def plan_report(result: PlanResult, hw: HardwareSpec, config: CompileConfig) -> str:
    lines = [f"# Partition plan ({config.run_name})", "",
             f"Hardware: {hw.name} ({hw.compute_units} CUs, {hw.hbm_bandwidth_gbs:.0f} GB/s HBM)",
             f"Candidates: {len(result.candidates)} (legal: {sum(c.legal for c in result.candidates)}), "
             f"planner mode: {config.planner_mode}", "",
             "| # | kernels | est. us | legal | note |", "|---|---|---|---|---|"]
    for c in sorted(result.candidates, key=lambda c: (not c.legal, c.total_cycles)):
        note = c.error or "; ".join(c.violations[:2]) or ("best" if c is result.best else "")
        est = f"{c.total_cycles:,.1f}" if c.legal else "-"
        lines.append(f"| {c.index} | {len(c.program.kernels) if c.program else '-'} | {est} | {'yes' if c.legal else 'no'} | {note} |")
    lines += ["", "## Chosen program", "", "```", result.program.summary(), "```"]
    return "\n".join(lines)


def write_device_results(run_dir: Path, program: Program, hw: HardwareSpec, bench: dict[str, Any]) -> None:
    """11_bench.json (the measurement) and 10_device_results.{json,md}: per kernel the measured
    µs next to the cost model's prediction (calibrated where the hardware spec carries a fit),
    the achieved rate and its fraction of the roofline. 10_* takes the place of the
    reference's 10_loom_results.json (Loom's optimum per kernel)."""
    from .cost_models.roofline import category, kernel_cost

    rw = ResultsWriter(run_dir)
    rw.write_json("11_bench.json", bench)
    specs = {k.name: k for k in program.kernels}
    rows = []
    for name, m in bench["kernels"].items():
        members = [specs[n] for n in name.split("+") if n in specs]
        pred = sum(kernel_cost(sp, program.tensors, hw).us for sp in members)
        rows.append({"kernel": name, "kind": m["kind"], "category": category(members[0], program.tensors),
                     "entries": m["entries"], "measured_us": m["us"], "predicted_us": pred,
                     "measured_over_predicted": m["us"] / pred if pred else None, "bound": m.get("bound"),
                     "achieved": m.get("achieved_tflops", m.get("achieved_gbs")),
                     "unit": "TFLOP/s" if "achieved_tflops" in m else "GB/s", "frac": m.get("frac")})
    total_pred = sum(r["predicted_us"] for r in rows)
    out = {"hw": hw.name, "calibrated": bool(hw.calibration), "forward_us_median": bench["us_median"],
           "sum_kernel_us": bench.get("sum_kernel_us"), "predicted_total_us": total_pred, "kernels": rows}
    rw.write_json("10_device_results.json", out)
    lines = [f"# Device results ({program.name})", "",
             f"Forward {bench['us_median']:,.1f} µs (graph replay, median); the cost model "
             f"({'calibrated' if hw.calibration else 'uncalibrated'}) predicts {total_pred:,.1f} µs.", "",
             "| kernel | category | measured µs | predicted µs | measured/predicted | achieved | roofline |",
             "|---|---|---:|---:|---:|---:|---:|"]
    for r in rows:
        ratio = f"{r['measured_over_predicted']:.2f}" if r["measured_over_predicted"] else "-"
        ach = f"{r['achieved']:,.0f} {r['unit']}" if r["achieved"] is not None else "-"
        frac = f"{100 * r['frac']:.1f}%" if r["frac"] is not None else "-"
        lines.append(f"| {r['kernel']} | {r['category']} | {r['measured_us']:,.1f} | {r['predicted_us']:,.1f} | "
                     f"{ratio} | {ach} | {frac} |")
    rw.write_text("10_device_results.md", "\n".join(lines) + "\n")


def cost_report_json(program: Program, hw: HardwareSpec, config: CompileConfig) -> dict[str, Any]:
    kernels = [{"name": k.name, "kind": k.kind, "tiles": k.tiles, "us": k.cost.get("us"), "bound": k.cost.get("bound"),
                "flops": k.cost.get("flops"), "bytes": k.cost.get("bytes")} for k in program.kernels]
    inter = program.intermediates()
    link = {t: program.tensors[t].nbytes for t in inter}
    return {"hw": hw.summary(), "kernels": kernels, "total_us": program.metadata.get("plan", {}).get("total_us"),
            "intermediate_tensors": link, "intermediate_bytes": sum(link.values())}


def cost_report_md(program: Program, hw: HardwareSpec, config: CompileConfig) -> str:
    total = program.metadata.get("plan", {}).get("total_us", 0.0)
    lines = [f"# Cost report ({program.name})", "",
             f"Hardware `{hw.name}`: {hw.compute_units} CUs, {hw.hbm_bandwidth_gbs:.0f} GB/s.",
             f"Estimated time: **{total:,.1f} us** (roofline, incl. {hw.launch_overhead_us} us per kernel).", "",
             "| kernel | kind | tiles | est. us | bound | GFLOP | MB |", "|---|---|---|---|---|---|---|"]
    for k in program.kernels:
        c = k.cost
        lines.append(f"| {k.name} | {k.kind} | {k.tiles} | {c.get('us', 0):,.1f} | {c.get('bound', '-')} | "
                     f"{c.get('flops', 0) / 1e9:,.2f} | {c.get('bytes', 0) / 1e6:,.1f} |")
    inter = program.intermediates()
    lines += ["", f"Kernel-to-kernel links: {len(inter)} intermediate tensors, "
              f"{sum(program.tensors[t].nbytes for t in inter):,} bytes through HBM.", ""]
    for t in inter:
        p = program.producer(t)
        lines.append(f"- `{t}` {program.tensors[t]}: {p.name if p else '?'} -> "
                     f"{', '.join(c.name for c in program.consumers(t)) or 'output'}")
    return "\n".join(lines) + "\n"
