"""Compile an OpIR epilogue SSA into a th_epilogue_vm program.

Values live in fp32 slots of a workspace; a slot is reused once its value's
last reader has run, so the workspace is ``n_slots * M * N`` floats with
``n_slots`` the peak number of live values, not the number of ops.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from ..optimizer.opir import KernelSpec
from . import abi

_BIN = {"add": abi.VM_ADD, "sub": abi.VM_SUB, "mul": abi.VM_MUL, "div": abi.VM_DIV, "max": abi.VM_MAX,
        "powf": abi.VM_POW}
_UN = {"exp": abi.VM_EXP, "log": abi.VM_LOG}
_RED = {"row_sum": abi.VM_ROW_SUM, "row_max": abi.VM_ROW_MAX}


@dataclass
class VmProgram:
    operands: list[tuple[torch.Tensor, bool]] = field(default_factory=list)
    ops: list[tuple] = field(default_factory=list)
    outs: list[tuple[torch.Tensor, int]] = field(default_factory=list)
    n_slots: int = 0


class _Slots:
    def __init__(self) -> None:
        self.free: list[int] = []
        self.count = 0

    def take(self) -> int:
        if self.free:
            return self.free.pop()
        self.count += 1
        return self.count - 1

    def give(self, s: int) -> None:
        self.free.append(s)


def compile_vm(dp, spec: KernelSpec, acc_bufs: dict[str, torch.Tensor], sumsq: torch.Tensor | None,
               lhs: torch.Tensor | None, M: int, N: int) -> VmProgram:
    prog = VmProgram()
    # where each value comes from before any op runs
    sources: dict[str, tuple[torch.Tensor, bool]] = {}
    for name, buf in acc_bufs.items():
        sources[name] = (buf, False)
    if sumsq is not None:
        sources["sumsq"] = (sumsq.view(M, 1), True)
    for a in spec.args:
        if a.role == "extra":
            t = dp.operand(a.tensor)
            sources[a.name] = (t.reshape(M, -1), t.numel() == M)
    alias: dict[str, str] = {}

    def root(v: str) -> str:
        while v in alias:
            v = alias[v]
        return v

    body = []
    for op in spec.epilogue:
        if op.op == "broadcast":
            alias[op.name] = op.inputs[0]
        else:
            body.append(op)
    last_use: dict[str, int] = {}
    for idx, op in enumerate(body):
        for i in op.inputs:
            last_use[root(i)] = idx
    end = len(body)
    for o in spec.outputs:
        last_use[root(o.value)] = end

    slots = _Slots()
    slot_of: dict[str, int] = {}

    def ensure(v: str) -> int:
        v = root(v)
        if v in slot_of:
            return slot_of[v]
        if v == "sumsq" and "sumsq" not in sources:
            if lhs is None:
                raise abi.HipBackendError("vm", abi.TH_ERR_INVALID, "epilogue needs sumsq but there is no lhs", spec.name)
            s = slots.take()
            prog.operands.append((lhs, False))
            prog.ops.append((abi.VM_LOAD, s, len(prog.operands) - 1, -1, 0.0, 0))
            prog.ops.append((abi.VM_MUL, s, s, s, 0.0, 0))
            prog.ops.append((abi.VM_ROW_SUM, s, s, -1, 0.0, 0))
            slot_of[v] = s
            return s
        if v not in sources:
            raise abi.HipBackendError("vm", abi.TH_ERR_INVALID, f"value {v} has no source", spec.name)
        s = slots.take()
        prog.operands.append(sources[v])
        prog.ops.append((abi.VM_LOAD, s, len(prog.operands) - 1, -1, 0.0, 0))
        slot_of[v] = s
        return s

    for idx, op in enumerate(body):
        ins = [ensure(i) for i in op.inputs]
        for i in op.inputs:  # release inputs whose last reader is this op
            r = root(i)
            if last_use.get(r) == idx and r in slot_of:
                slots.give(slot_of.pop(r))
        dst = slots.take()
        a = op.attrs
        if op.op in _BIN:
            if "scalar" in a:
                mode = 2 if a.get("scalar_first") else 1
                prog.ops.append((_BIN[op.op], dst, ins[0], -1, float(a["scalar"]), mode))
            else:
                prog.ops.append((_BIN[op.op], dst, ins[0], ins[1], 0.0, 0))
        elif op.op in _UN:
            prog.ops.append((_UN[op.op], dst, ins[0], -1, 0.0, 0))
        elif op.op in _RED:
            prog.ops.append((_RED[op.op], dst, ins[0], -1, 0.0, 0))
        else:
            raise abi.HipBackendError("vm", abi.TH_ERR_UNSUPPORTED, f"epilogue op {op.op} is not registered", spec.name)
        slot_of[op.name] = dst
        if op.name not in last_use:
            slots.give(slot_of.pop(op.name))
    for o in spec.outputs:
        s = ensure(o.value)
        prog.outs.append((dp.buffers[o.tensor].view(M, -1), s))
        if o.tensor in dp.shadow:
            prog.outs.append((dp.shadow[o.tensor].view(M, -1), s))
    prog.n_slots = max(1, slots.count)
    if len(prog.ops) > abi.VM_MAX_OPS or len(prog.operands) > abi.VM_MAX_IN or len(prog.outs) > abi.VM_MAX_OUT:
        raise abi.HipBackendError("vm", abi.TH_ERR_UNSUPPORTED, "epilogue too large for the VM", spec.name)
    return prog
