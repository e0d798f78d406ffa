"""CPU interpreter of the OpIR (reference: codegen/interpret.py:18-77).

Runs a Program kernel by kernel in fp32 with the op semantics of
:mod:`torch_helion.optimizer.evaluate`. ``compile_model`` uses it for the
``reference_check`` stage (interpreter vs eager model, as the reference
does); the device path never calls it.
"""

from __future__ import annotations

import torch

from ..optimizer.evaluate import eval_op
from ..optimizer.opir import KernelSpec, Program

_ROLES = {"ssd": ["c", "b", "x", "cum", "dt", "mask", "dskip"], "ssd_chunked": ["c", "b", "x", "dt", "A", "D"],
          "conv1d": ["x", "w"], "embedding": ["table", "ids"]}


def run_kernel(spec: KernelSpec, env: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    args = {a.name: env[a.tensor].float() if env[a.tensor].is_floating_point() else env[a.tensor] for a in spec.args}
    vals: dict[str, torch.Tensor] = {}
    if spec.kind == "gemm":
        lhs = args["lhs"]
        # e4m3 weights carry per-column scales (arg "<rhs>_scale"); an activation-side
        # RMSNorm gain (role "gain") multiplies the lhs columns, the sum of squares does not see it
        a_lhs = lhs * args["gain"] if "gain" in args else lhs
        for g in spec.gemms:
            w = args[g.rhs]
            if g.rhs + "_scale" in args:
                w = w * args[g.rhs + "_scale"]
            vals[g.acc] = a_lhs @ w
        if spec.sumsq:
            vals["sumsq"] = (lhs * lhs).sum(-1, keepdim=True)
    elif spec.kind == "attention":
        return {spec.outputs[0].tensor: eval_op("attention", [args["q"], args["k"], args["v"]], spec.attrs)}
    elif spec.kind == "attention_decode":
        return {spec.outputs[0].tensor: eval_op("attention_decode", [args[r] for r in
                                                                   ("q", "k_cache", "v_cache", "k_new", "v_new")],
                                                spec.attrs)}
    elif spec.kind in _ROLES:
        vals["acc"] = eval_op(spec.kind, [args[r] for r in _ROLES[spec.kind]], spec.attrs)
        if spec.kind == "embedding":
            vals["out"] = vals.pop("acc").reshape(-1, spec.attrs["dim"])
    else:
        raise ValueError(spec.kind)
    for a in spec.args:
        if a.role == "extra":
            vals[a.name] = args[a.name]
    for op in spec.epilogue:
        vals[op.name] = eval_op(op.op, [vals[i] for i in op.inputs], op.attrs)
    return {o.tensor: vals[o.value] for o in spec.outputs}


def run_program(program: Program, params: dict[str, torch.Tensor], inputs) -> dict[str, torch.Tensor]:
    if isinstance(inputs, (list, tuple)):
        inputs = dict(zip(program.inputs, inputs))
    env: dict[str, torch.Tensor] = {}
    for name in program.inputs:
        t = inputs[name].reshape(program.tensors[name].shape)
        env[name] = t.float() if t.is_floating_point() else t
    for name in program.params:
        env[name] = params[name].float() if params[name].is_floating_point() else params[name]
    for spec in program.kernels:
        env.update(run_kernel(spec, env))
    return env


def program_outputs(program: Program, params: dict[str, torch.Tensor], inputs) -> list[torch.Tensor]:
    env = run_program(program, params, inputs)
    shapes = program.metadata.get("output_shapes", {})
    return [env[o].reshape(shapes[o]) if o in shapes else env[o] for o in program.outputs]
