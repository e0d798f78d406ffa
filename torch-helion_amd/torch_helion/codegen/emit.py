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


_ENTRY = {"gemm": "th_gemm", "attention": "th_attention_prefill", "ssd": "th_ssd_chunked",
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


def emit_program(program: Program, config, out_dir: Path) -> dict[str, Path]:
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    files: dict[str, Path] = {}
    for spec in program.kernels:
        p = out_dir / f"{spec.name}.json"
        p.write_text(json.dumps(launch_plan(spec, program), indent=2, default=str))
        files[spec.name] = p
    return files
