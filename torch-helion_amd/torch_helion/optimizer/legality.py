"""Kernel legality for the MI355X backend (reference: optimizer/legality.py:56-145).

The reference encodes Loom's constraints C1-C6 (every extent a multiple of
32, rank-2 operands only, a fixed registered-op set). On gfx950 the limits
are the kernels' own:

* gemm: operand shapes consistent; K a multiple of 8 (bf16/fp16) or 4 (fp32)
  for 16-byte loads; at most 6 accumulators before RoPE re-fusion; epilogue
  ops registered (anything registered runs, fused or on the epilogue VM);
* attention: head_dim 64 or 128 (bf16), 16/32/64/128 (fp32); heads a
  multiple of kv_heads;
* ssd / ssd_chunked: head_dim and state_dim multiples of 16, at most 128;
* conv1d: kernel width at most 8;
* embedding: integer ids, a parameter table, no epilogue.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from ..capture.opgraph import TensorType
from ..capture.ops import REGISTERED_BINARY, REGISTERED_REDUCE, REGISTERED_UNARY
from .opir import KernelSpec, Program

MAX_GEMM_ACC = 6


@dataclass
class Violation:
    kernel: str
    rule: str
    message: str

    def __str__(self) -> str:
        return f"[{self.kernel}] {self.rule}: {self.message}"


@dataclass
class LegalityReport:
    violations: list[Violation] = field(default_factory=list)

    @property
    def ok(self) -> bool:
        return not self.violations

    def add(self, kernel: str, rule: str, message: str) -> None:
        self.violations.append(Violation(kernel, rule, message))

    def __str__(self) -> str:
        return "legal" if self.ok else "\n".join(str(v) for v in self.violations)


def _k_align(dtype: str) -> int:
    return 4 if dtype == "float32" else 8


def check_kernel(spec: KernelSpec, tensors: dict[str, TensorType], report: LegalityReport | None = None) -> LegalityReport:
    rep = report or LegalityReport()
    k = spec.name
    if spec.kind == "gemm":
        T, N, K = spec.grid["rows"], spec.grid["cols"], spec.k_extent
        lhs = tensors[spec.arg("lhs").tensor]
        if lhs.shape != (T, K):
            rep.add(k, "shape", f"lhs {lhs.shape} != {(T, K)}")
        if K % _k_align(lhs.dtype):
            rep.add(k, "align", f"K={K} is not a multiple of {_k_align(lhs.dtype)} elements")
        if not spec.gemms and not spec.sumsq:
            rep.add(k, "empty", "kernel has neither a GEMM nor a row reduction")
        if len(spec.gemms) > MAX_GEMM_ACC:
            rep.add(k, "acc", f"{len(spec.gemms)} accumulators > {MAX_GEMM_ACC}")
        for g in spec.gemms:
            rhs = tensors[spec.arg(g.rhs).tensor]
            if rhs.shape != (K, N):
                rep.add(k, "shape", f"rhs {g.rhs} {rhs.shape} != {(K, N)}")
        for a in spec.args:
            if a.role == "extra" and tensors[a.tensor].shape != (T, N):
                rep.add(k, "shape", f"epilogue input {a.tensor} {tensors[a.tensor].shape} != {(T, N)}")
        for op in spec.epilogue:
            if op.op not in REGISTERED_BINARY | REGISTERED_UNARY | REGISTERED_REDUCE | {"broadcast"}:
                rep.add(k, "op", f"epilogue op {op.name} = {op.op} is not registered")
        for o in spec.outputs:
            if tensors[o.tensor].shape != (T, N):
                rep.add(k, "shape", f"output {o.tensor} {tensors[o.tensor].shape} != {(T, N)}")
    elif spec.kind == "attention":
        a = spec.attrs
        dt = tensors[spec.arg("q").tensor].dtype
        ok_hd = (64, 128) if dt != "float32" else (16, 32, 64, 128)
        if a["head_dim"] not in ok_hd:
            rep.add(k, "head_dim", f"head_dim {a['head_dim']} not in {ok_hd}")
        if a["heads"] % a.get("kv_heads", a["heads"]):
            rep.add(k, "gqa", f"heads {a['heads']} not a multiple of kv_heads {a.get('kv_heads')}")
    elif spec.kind in ("ssd", "ssd_chunked"):
        a = spec.attrs
        for label in ("head_dim", "state_dim"):
            if a[label] % 16 or a[label] > 128:
                rep.add(k, label, f"{label}={a[label]} must be a multiple of 16 and at most 128")
        if spec.kind == "ssd_chunked" and a["heads"] % a.get("ngroups", a["heads"]):
            rep.add(k, "groups", "heads not a multiple of ngroups")
        for op in spec.epilogue:
            if op.op not in REGISTERED_BINARY | REGISTERED_UNARY | {"broadcast"}:
                rep.add(k, "op", f"epilogue op {op.name} = {op.op} is not registered")
    elif spec.kind == "conv1d":
        if spec.attrs["kernel"] > 8:
            rep.add(k, "kernel", f"conv width {spec.attrs['kernel']} > 8")
    elif spec.kind == "embedding":
        a = spec.attrs
        table, ids = tensors[spec.arg("table").tensor], tensors[spec.arg("ids").tensor]
        if ids.dtype not in ("int64", "int32"):
            rep.add(k, "ids", f"token ids are {ids.dtype}, not int64/int32")
        if table.shape != (a["vocab"], a["dim"]) or math.prod(ids.shape) != a["tokens"]:
            rep.add(k, "shape", f"table {table.shape} / ids {ids.shape} do not match {a}")
        if spec.epilogue:
            rep.add(k, "epilogue", "an embedding gather hosts no epilogue")
    else:
        rep.add(k, "kind", f"unknown kernel kind {spec.kind}")
    return rep


def check_program(program: Program) -> LegalityReport:
    rep = LegalityReport()
    for spec in program.kernels:
        check_kernel(spec, program.tensors, rep)
    return rep
