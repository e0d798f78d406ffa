"""Match an OpIR epilogue SSA against th_gemm's fused output catalogue.

An epilogue (reference: optimizer/opir.py:43-48, evaluated by
codegen/interpret.py:27-34) is expanded into one expression tree per stored
output, with leaves ``acc_i``, ``sumsq`` and ``extra`` arguments. The tree is
then matched against the catalogue of ``th_epi_op`` (include/th_hip.h):

    r        = powf(add(mul(sumsq, 1/K), eps), -0.5)      (the RMS row scale)
    a_i      = acc_i  |  acc_i * r
    ACC      a_i
    SILU     a_i * sigmoid(a_i)           sigmoid = div(1, add(exp(mul(x,-1)), 1))
    SWIGLU   SILU(a_i) * a_j
    ADD      a_i + e         SOFTPLUS_ADD  log(add(exp(a_i + e), 1))     MUL  a_i * e
    ROPE     a_i * cos + a_j * sin  where w_j is w_i with its columns rotated
             (the reference's pre-rotated sibling, optimizer/passes.py:204-212):
             a_j is dropped and the rotation is done in the epilogue.

Anything else runs as a generic program on the epilogue VM (th_epilogue_vm).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import torch

from ..optimizer.opir import KernelSpec
from . import abi

Expr = tuple  # ("acc", i) | ("sumsq",) | ("extra", arg) | (op, attrs_key, *children)


def _freeze(attrs: dict[str, Any]) -> tuple:
    return tuple(sorted((k, v) for k, v in attrs.items() if k in ("scalar", "scalar_first")))


def build_trees(spec: KernelSpec) -> dict[str, Expr]:
    """value name -> expression tree for every value of the kernel."""
    env: dict[str, Expr] = {}
    for i, g in enumerate(spec.gemms):
        env[g.acc] = ("acc", i)
    env["sumsq"] = ("sumsq",)
    if spec.kind in ("ssd", "ssd_chunked", "conv1d"):
        env["acc"] = ("acc", 0)
    for a in spec.args:
        if a.role == "extra":
            env[a.name] = ("extra", a.name)
    for op in spec.epilogue:
        kids = tuple(env[i] for i in op.inputs)
        if op.op == "broadcast":
            env[op.name] = kids[0]  # a [T,1] column broadcast over the tile is transparent
        else:
            env[op.name] = (op.op, _freeze(op.attrs)) + kids
    return env


def _scalar(e: Expr, op: str, first: bool = False) -> tuple[float, Expr] | None:
    if len(e) == 3 and e[0] == op:
        attrs = dict(e[1])
        if "scalar" in attrs and bool(attrs.get("scalar_first", False)) == first:
            return float(attrs["scalar"]), e[2]
    return None


def match_rscale(e: Expr) -> tuple[float, float] | None:
    """(inv_k, eps) if ``e`` is powf(add(mul(sumsq, inv_k), eps), -0.5)."""
    p = _scalar(e, "powf")
    if p is None or p[0] != -0.5:
        return None
    a = _scalar(p[1], "add")
    if a is None:
        return None
    m = _scalar(a[1], "mul")
    if m is None or m[1] != ("sumsq",):
        return None
    return m[0], a[0]


def _binary(e: Expr, op: str) -> tuple[Expr, Expr] | None:
    if len(e) == 4 and e[0] == op and not dict(e[1]).get("scalar") and "scalar" not in dict(e[1]):
        return e[2], e[3]
    return None


@dataclass
class _Ctx:
    rscale: tuple[float, float] | None = None


def match_scaled_acc(e: Expr, ctx: _Ctx) -> tuple[int, bool] | None:
    """(acc index, scaled by r) for ``acc_i`` or ``acc_i * r``."""
    if e[0] == "acc":
        return e[1], False
    b = _binary(e, "mul")
    if b is None:
        return None
    for x, y in (b, b[::-1]):
        if x[0] == "acc":
            rs = match_rscale(y)
            if rs is not None and (ctx.rscale is None or ctx.rscale == rs):
                ctx.rscale = rs
                return x[1], True
    return None


def match_sigmoid_of(e: Expr) -> Expr | None:
    """x if ``e`` is div(1, add(exp(mul(x, -1)), 1))."""
    d = _scalar(e, "div", first=True)
    if d is None or d[0] != 1.0:
        return None
    a = _scalar(d[1], "add")
    if a is None or a[0] != 1.0 or a[1][0] != "exp":
        return None
    m = _scalar(a[1][2], "mul")
    if m is None or m[0] != -1.0:
        return None
    return m[1]


def match_silu(e: Expr) -> Expr | None:
    b = _binary(e, "mul")
    if b is None:
        return None
    for x, y in (b, b[::-1]):
        if match_sigmoid_of(y) == x:
            return x
    return None


@dataclass
class FusedOut:
    tensor: str
    op: int
    a: int
    b: int = -1
    extra: str | None = None                 # extra argument name (ADD / SOFTPLUS_ADD / MUL)
    rope: tuple[str, str] | None = None      # (cos arg, sin arg)


@dataclass
class EpiloguePlan:
    """Result of matching one kernel's epilogue."""

    fused: bool
    outs: list[FusedOut] = field(default_factory=list)
    scaled: dict[int, bool] = field(default_factory=dict)
    rscale: tuple[float, float] | None = None
    reason: str = ""


def match_output(e: Expr, ctx: _Ctx, scaled: dict[int, bool]) -> FusedOut | None:
    def acc(x: Expr) -> int | None:
        m = match_scaled_acc(x, ctx)
        if m is None:
            return None
        i, s = m
        if scaled.setdefault(i, s) != s:
            return None
        return i

    i = acc(e)
    if i is not None:
        return FusedOut("", abi.EPI_ACC, i)
    x = match_silu(e)
    if x is not None and (i := acc(x)) is not None:
        return FusedOut("", abi.EPI_SILU, i)
    b = _binary(e, "mul")
    if b is not None:
        for x, y in (b, b[::-1]):
            s = match_silu(x)
            if s is not None and (i := acc(s)) is not None and (j := acc(y)) is not None:
                return FusedOut("", abi.EPI_SWIGLU, i, j)
        for x, y in (b, b[::-1]):
            if y[0] == "extra" and (i := acc(x)) is not None:
                return FusedOut("", abi.EPI_MUL, i, extra=y[1])
    b = _binary(e, "add")
    if b is not None:
        for x, y in (b, b[::-1]):
            if y[0] == "extra" and (i := acc(x)) is not None:
                return FusedOut("", abi.EPI_ADD, i, extra=y[1])
        m1, m2 = _binary(b[0], "mul"), _binary(b[1], "mul")
        if m1 is not None and m2 is not None:
            def split(m):
                for x, y in (m, m[::-1]):
                    if y[0] == "extra" and (k := acc(x)) is not None:
                        return k, y[1]
                return None
            p1, p2 = split(m1), split(m2)
            if p1 is not None and p2 is not None:
                return FusedOut("", abi.EPI_ROPE_PAIR, p1[0], p2[0], rope=(p1[1], p2[1]))
    lg = e if (len(e) == 3 and e[0] == "log") else None
    if lg is not None:
        a1 = _scalar(lg[2], "add")
        if a1 is not None and a1[0] == 1.0 and a1[1][0] == "exp":
            inner = _binary(a1[1][2], "add")
            if inner is not None:
                for x, y in (inner, inner[::-1]):
                    if y[0] == "extra" and (i := acc(x)) is not None:
                        return FusedOut("", abi.EPI_SOFTPLUS_ADD, i, extra=y[1])
    return None


def match_epilogue(spec: KernelSpec) -> EpiloguePlan:
    """Structural match of every stored output of a gemm kernel."""
    trees = build_trees(spec)
    ctx = _Ctx()
    scaled: dict[int, bool] = {}
    outs: list[FusedOut] = []
    for o in spec.outputs:
        if o.value not in trees:
            return EpiloguePlan(False, reason=f"output {o.tensor} reads unknown value {o.value}")
        f = match_output(trees[o.value], ctx, scaled)
        if f is None:
            return EpiloguePlan(False, reason=f"output {o.tensor} is outside the fused catalogue")
        f.tensor = o.tensor
        outs.append(f)
    return EpiloguePlan(True, outs, scaled, ctx.rscale)


def fused_acc_count(spec: KernelSpec) -> int:
    """Accumulators th_gemm computes for ``spec`` when a RoPE pair's rotated
    accumulator is re-fused (structural estimate, no weight values)."""
    plan = match_epilogue(spec)
    if not plan.fused:
        return len(spec.gemms)
    rotated = {o.b for o in plan.outs if o.op == abi.EPI_ROPE_PAIR}
    used = {o.a for o in plan.outs} | {o.b for o in plan.outs if o.b >= 0}
    return max(1, len(used - rotated)) if used else len(spec.gemms)


# ------------------------------------------------------------ table checks
def periodic_table(t: torch.Tensor, row_period: int, col_period: int) -> torch.Tensor | None:
    """``t[:row_period, :col_period]`` if ``t[r, c] == that[r % rp, c % cp]``."""
    rows, cols = t.shape
    if rows % row_period or cols % col_period:
        return None
    base = t[:row_period, :col_period]
    view = t.reshape(rows // row_period, row_period, cols // col_period, col_period)
    if not torch.equal(view, base.reshape(1, row_period, 1, col_period).expand_as(view)):
        return None
    return base.contiguous()


def _divisors(n: int) -> list[int]:
    return [d for d in range(1, n + 1) if n % d == 0]


def rope_geometry(cos: torch.Tensor, sin: torch.Tensor, seq_hint: int | None = None) -> tuple[int, int] | None:
    """(row period, head dim) of expanded RoPE tables: the smallest column
    period (a multiple of 8) first, then the smallest row period for it."""
    rows, cols = cos.shape
    for hd in [d for d in _divisors(cols) if d % 8 == 0]:
        if periodic_table(cos, rows, hd) is None or periodic_table(sin, rows, hd) is None:
            continue
        c1, s1 = cos[:, :hd], sin[:, :hd]
        row_opts = [seq_hint] if seq_hint and rows % seq_hint == 0 else _divisors(rows)
        for rp in row_opts:
            if periodic_table(c1, rp, hd) is not None and periodic_table(s1, rp, hd) is not None:
                return rp, hd
    return None


def is_rotated_copy(w: torch.Tensor, w_rot: torch.Tensor, head_dim: int) -> bool:
    """True when ``w_rot == w @ R`` for the per-head rotate-half matrix R."""
    from ..optimizer.param_transforms import rotate_columns

    if w.shape != w_rot.shape or w.shape[1] % head_dim:
        return False
    return torch.equal(rotate_columns(w, w.shape[1] // head_dim, head_dim), w_rot)
