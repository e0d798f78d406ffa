"""OpIR -> HIP launch plans (replaces the reference's Helion emitter,
codegen/emit.py:500-520, keeping its signature and ``{kernel: path}`` result).

For every KernelSpec one JSON file describes how the HIP backend runs it:
the C-ABI entry point, the tile the kernel will use, and the fused epilogue
catalogue entries (or the epilogue-VM fallback). Binding to device buffers
happens in :class:`torch_helion.hip.runtime.DeviceProgram`, which also
confirms RoPE re-fusion against the weight values.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any

from ..optimizer.opir import KernelSpec, Program


class CodegenError(RuntimeError):
    pass


_ENTRY = {"gemm": "th_gemm", "attention": "th_attention_prefill", "attention_decode": "th_attention_decode",
          "ssd": "th_ssd_chunked",
          "ssd_chunked": "th_ssd_chunked", "conv1d": "th_conv1d_causal", "embedding": "th_embedding"}


def launch_plan(spec: KernelSpec, program: Program) -> dict[str, Any]:
    from ..hip import abi
    from ..hip.epilogue import fused_acc_count, match_epilogue

    if spec.kind not in _ENTRY:
        raise CodegenError(f"{spec.name}: no HIP kernel for kind {spec.kind!r}")
    plan: dict[str, Any] = {"kernel": spec.name, "kind": spec.kind, "entry": _ENTRY[spec.kind], "tiles": spec.tiles,
                            "args": [{"name": a.name, "tensor": a.tensor, "role": a.role,
                                      "shape": list(program.tensors[a.tensor].shape),
                                      "dtype": program.tensors[a.tensor].dtype} for a in spec.args],
                            "outputs": [o.tensor for o in spec.outputs]}
    if spec.kind == "gemm":
        if not spec.gemms:
            plan["entry"] = "th_rmsnorm | th_epilogue_vm"
        else:
            m = match_epilogue(spec)
            names = {v: k for k, v in vars(abi).items() if k.startswith("EPI_")}
            plan["epilogue"] = ({"fused": True, "n_acc": fused_acc_count(spec), "rscale": m.rscale,
                                 "outputs": [{"tensor": o.tensor, "op": names.get(o.op, o.op), "a": o.a, "b": o.b,
                                              "extra": o.extra, "rope": o.rope} for o in m.outs]}
                                if m.fused else {"fused": False, "reason": m.reason, "fallback": "th_epilogue_vm"})
    return plan


def readme(program: Program, plans: dict[str, dict[str, Any]]) -> str:
    """kernels/README.md: what each launch plan is and how to run it (the reference's
    kernels/README.md explains how to run each generated kernel through Loom)."""
    lines = [f"# Kernels of `{program.name}`", "",
             "Each `<kernel>.json` is the HIP launch plan of one OpIR KernelSpec: the C-ABI entry point of",
             "`libth_hip.so` (declared in `include/th_hip.h`), the tile, every argument with its tensor, role,",
             "shape and dtype, and for GEMMs the fused epilogue (catalogue ops, or the epilogue-VM fallback).",
             "", "Run a plan on the GPU through the runtime, which binds device buffers and packs weights:", "",
             "```python", "from torch_helion import CompileConfig, compile_model",
             "res = compile_model(model, example_inputs, CompileConfig(backend=\"hip\"))",
             "res.device_program.run(list(example_inputs))      # every kernel, in program order",
             "[l for l in res.device_program.launches if l.kernel == \"k0_gemm\"]  # one kernel's C-ABI launches",
             "```", "",
             "A plan can also be driven from C with the descriptors of `include/th_hip.h` (one `th_*` call per",
             "plan; the caller owns every buffer).", "",
             "| kernel | kind | entry point | tiles | inputs -> outputs |", "|---|---|---|---|---|"]
    for spec in program.kernels:
        p = plans[spec.name]
        ins = ", ".join(f"{a['role']}={a['tensor']}" for a in p["args"])
        lines.append(f"| `{spec.name}` | {spec.kind} | `{p['entry']}` | {p['tiles']} | {ins} -> "
                     f"{', '.join(p['outputs'])} |")
    return "\n".join(lines) + "\n"


def emit_program(program: Program, config, out_dir: Path) -> dict[str, Path]:
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    files: dict[str, Path] = {}
    plans: dict[str, dict[str, Any]] = {}
    for spec in program.kernels:
        p = out_dir / f"{spec.name}.json"
        plans[spec.name] = launch_plan(spec, program)
        p.write_text(json.dumps(plans[spec.name], indent=2, default=str))
        files[spec.name] = p
    (out_dir / "README.md").write_text(readme(program, plans))
    return files
