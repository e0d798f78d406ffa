"""OpIR: the kernel-level program (reference: optimizer/opir.py:35-179).

A :class:`Program` is an ordered list of :class:`KernelSpec` over a flat
tensor table. The JSON layout (``Program.to_dict``) is the reference's, key
for key, so a ``06_opir.json`` written by the reference loads here and runs
on the HIP backend; the MI355X additions are new kernel kinds
(``ssd_chunked``, ``conv1d``) and new ``attrs`` keys (``causal``,
``kv_heads``, ``ngroups``, ``chunk``), never changes to existing fields.

Kinds
  gemm        acc_i = lhs @ rhs_i (shared lhs), optional ``sumsq`` of lhs rows,
              an epilogue SSA over registered ops, stores.
  attention   softmax(q k^T * scale) v over [B, S, H, d] views (+ causal, GQA).
  ssd         the reference's quadratic Mamba-2 scan (padded cum/dt operands).
  ssd_chunked the Mamba-2 scan from raw dt [T, H] and per-head A, D.
  conv1d      depthwise causal convolution over each sequence (+ SiLU).
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any

from ..capture.opgraph import TensorType


@dataclass
class KernelArg:
    name: str
    tensor: str
    role: str            # lhs | rhs | extra | q | k | v | c | b | x | cum | dt | mask | dskip | xskip | A | D | w
    view: list[int] | None = None


@dataclass
class BodyOp:
    name: str
    op: str
    inputs: list[str]
    attrs: dict[str, Any] = field(default_factory=dict)


@dataclass
class GemmSpec:
    acc: str
    rhs: str


@dataclass
class KernelOutput:
    tensor: str
    value: str


@dataclass
class KernelSpec:
    name: str
    kind: str
    args: list[KernelArg] = field(default_factory=list)
    outputs: list[KernelOutput] = field(default_factory=list)
    lhs: str | None = None
    k_extent: int = 0
    grid: dict[str, int] = field(default_factory=dict)
    gemms: list[GemmSpec] = field(default_factory=list)
    sumsq: bool = False
    epilogue: list[BodyOp] = field(default_factory=list)
    attrs: dict[str, Any] = field(default_factory=dict)
    constexprs: dict[str, float] = field(default_factory=dict)
    tiles: dict[str, int] = field(default_factory=dict)
    cost: dict[str, Any] = field(default_factory=dict)
    notes: list[str] = field(default_factory=list)

    def arg(self, name: str) -> KernelArg:
        for a in self.args:
            if a.name == name:
                return a
        raise KeyError(name)

    def input_tensors(self) -> list[str]:
        return [a.tensor for a in self.args]

    def output_tensors(self) -> list[str]:
        return [o.tensor for o in self.outputs]

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    @staticmethod
    def from_dict(d: dict[str, Any]) -> "KernelSpec":
        return KernelSpec(
            name=d["name"], kind=d["kind"],
            args=[KernelArg(**a) for a in d.get("args", [])],
            outputs=[KernelOutput(**o) for o in d.get("outputs", [])],
            lhs=d.get("lhs"), k_extent=d.get("k_extent", 0), grid=dict(d.get("grid", {})),
            gemms=[GemmSpec(**g) for g in d.get("gemms", [])], sumsq=d.get("sumsq", False),
            epilogue=[BodyOp(**b) for b in d.get("epilogue", [])], attrs=dict(d.get("attrs", {})),
            constexprs=dict(d.get("constexprs", {})), tiles=dict(d.get("tiles", {})),
            cost=dict(d.get("cost", {})), notes=list(d.get("notes", [])))


@dataclass
class Program:
    name: str
    inputs: list[str]
    outputs: list[str]
    tensors: dict[str, TensorType]
    kernels: list[KernelSpec]
    params: list[str] = field(default_factory=list)
    metadata: dict[str, Any] = field(default_factory=dict)

    def intermediates(self) -> list[str]:
        produced = {o for k in self.kernels for o in k.output_tensors()}
        return [t for t in produced if t not in self.outputs]

    def producer(self, tensor: str) -> KernelSpec | None:
        for k in self.kernels:
            if tensor in k.output_tensors():
                return k
        return None

    def consumers(self, tensor: str) -> list[KernelSpec]:
        return [k for k in self.kernels if tensor in k.input_tensors()]

    def to_dict(self) -> dict[str, Any]:
        return {"name": self.name, "inputs": self.inputs, "outputs": self.outputs,
                "tensors": {n: {"shape": list(t.shape), "dtype": t.dtype} for n, t in self.tensors.items()},
                "params": self.params, "kernels": [k.to_dict() for k in self.kernels], "metadata": self.metadata}

    def to_json(self, path: str | Path) -> None:
        Path(path).write_text(json.dumps(self.to_dict(), indent=2, default=str))

    @staticmethod
    def from_dict(d: dict[str, Any]) -> "Program":
        return Program(name=d["name"], inputs=list(d["inputs"]), outputs=list(d["outputs"]),
                       tensors={n: TensorType(tuple(t["shape"]), t["dtype"]) for n, t in d["tensors"].items()},
                       kernels=[KernelSpec.from_dict(k) for k in d["kernels"]],
                       params=list(d.get("params", [])), metadata=dict(d.get("metadata", {})))

    @staticmethod
    def from_json(path: str | Path) -> "Program":
        return Program.from_dict(json.loads(Path(path).read_text()))

    def summary(self) -> str:
        lines = [f"Program {self.name}: {len(self.kernels)} kernels, inputs={self.inputs}, outputs={self.outputs}"]
        for k in self.kernels:
            ins = ", ".join(f"{a.name}<-{a.tensor}" for a in k.args)
            outs = ", ".join(o.tensor for o in k.outputs)
            extra = (f" gemms={len(k.gemms)} sumsq={k.sumsq} epilogue={len(k.epilogue)}" if k.kind == "gemm"
                     else f" attrs={k.attrs}")
            est = k.cost.get("us")
            cost = f" est={est:,.1f}us tiles={k.tiles}" if est else ""
            lines.append(f"  [{k.kind}] {k.name}({ins}) -> {outs}{extra}{cost}")
        return "\n".join(lines)
