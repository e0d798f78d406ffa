"""Partition a canonical OpGraph into kernels (reference: optimizer/partition.py:99-300).

Anchors are reductions: a group of sibling GEMMs sharing one LHS and output
width (the planner's grouping decides which siblings share a kernel), an
``attention``, a scan (``ssd`` / ``ssd_chunked``), a ``conv1d``, an
``embedding`` gather, or a stand-alone row sum of squares. Every other
compute op joins the epilogue of the latest anchor whose output tile it
fits (an embedding hosts no epilogue); the RMS column chain
(``row_sumsq`` -> scalars) is cloned into each kernel that needs it. Values
crossing kernels become DRAM tensors. Deterministic for a given grouping.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ..capture.opgraph import OpGraph, OpNode, TensorType
from ..capture.ops import BINARY_OPS, UNARY_OPS
from .opir import BodyOp, GemmSpec, KernelArg, KernelOutput, KernelSpec, Program


class PartitionError(RuntimeError):
    pass


Grouping = dict[str, int]  # matmul node -> group id


def sibling_sets(g: OpGraph) -> list[list[str]]:
    """GEMMs sharing the same LHS tensor and output width, in graph order."""
    by_key: dict[tuple[str, int], list[str]] = {}
    for n in g:
        if n.op == "matmul":
            by_key.setdefault((n.inputs[0], n.type.shape[1]), []).append(n.name)
    return list(by_key.values())


def default_grouping(g: OpGraph, merge_siblings: bool = True) -> Grouping:
    grouping: Grouping = {}
    gid = 0
    for group in sibling_sets(g):
        for m in group:
            grouping[m] = gid
            if not merge_siblings:
                gid += 1
        if merge_siblings:
            gid += 1
    return grouping


@dataclass
class _Kernel:
    spec: KernelSpec
    owned: dict[str, str] = field(default_factory=dict)
    order_key: int = 0
    anchor_key: int = 0
    lhs_node: str | None = None
    extra_args: dict[str, str] = field(default_factory=dict)
    column_cache: dict[str, str] = field(default_factory=dict)


def _tile_frame(k: _Kernel) -> tuple[int, int]:
    a = k.spec.attrs
    if k.spec.kind in ("ssd", "ssd_chunked"):
        return (a["batch"] * a["seq"], a["heads"] * a["head_dim"])
    if k.spec.kind == "conv1d":
        return (a["batch"] * a["seq"], a["width"])
    if k.spec.kind == "embedding":
        return (a["tokens"], a["dim"])
    return (k.spec.grid["rows"], k.spec.grid["cols"])


def _column_source(g: OpGraph, name: str, memo: dict[str, str | None]) -> str | None:
    """If ``name`` derives only from ``row_sumsq(x)`` and scalars, return ``x``."""
    if name in memo:
        return memo[name]
    node = g[name]
    res: str | None = None
    if node.op == "row_sumsq":
        res = node.inputs[0]
    elif node.op in BINARY_OPS or node.op in UNARY_OPS:
        srcs = [_column_source(g, i, memo) for i in node.inputs]
        if srcs and all(s is not None for s in srcs) and len(set(srcs)) == 1:
            res = srcs[0]
    memo[name] = res
    return res


_EPILOGUE_KINDS = ("gemm", "ssd", "ssd_chunked", "conv1d")


def build_program(g: OpGraph, grouping: Grouping | None = None, name: str = "program") -> Program:
    grouping = grouping if grouping is not None else default_grouping(g)
    order = {n.name: i for i, n in enumerate(g)}
    kernels: list[_Kernel] = []
    by_group: dict[int, _Kernel] = {}
    owner: dict[str, _Kernel] = {}
    memo: dict[str, str | None] = {}
    tensors: dict[str, TensorType] = {n.name: n.type for n in g}

    def new_kernel(spec: KernelSpec, node: OpNode, lhs: str | None = None) -> _Kernel:
        k = _Kernel(spec, order_key=order[node.name], anchor_key=order[node.name], lhs_node=lhs)
        kernels.append(k)
        return k

    # --- anchors
    for n in g:
        if n.op == "matmul":
            lhs, rhs = n.inputs
            if g[rhs].kind not in ("param", "const") and g[lhs].kind not in ("param", "const"):
                raise PartitionError(f"{n.name}: neither GEMM operand is constant")
            gid = grouping[n.name]
            k = by_group.get(gid)
            if k is None:
                spec = KernelSpec(name="gemm", kind="gemm", lhs="lhs", k_extent=g[lhs].type.shape[1],
                                  grid={"rows": n.type.shape[0], "cols": n.type.shape[1]})
                spec.args.append(KernelArg("lhs", lhs, "lhs"))
                k = by_group[gid] = new_kernel(spec, n, lhs)
            if k.lhs_node != lhs or k.spec.grid["cols"] != n.type.shape[1]:
                raise PartitionError(f"{n.name}: grouped with GEMMs of a different LHS or width")
            arg = f"w{len(k.spec.gemms)}"
            k.spec.args.append(KernelArg(arg, rhs, "rhs"))
            acc = f"acc_{n.name}"
            k.spec.gemms.append(GemmSpec(acc, arg))
            k.owned[n.name] = acc
            owner[n.name] = k
        elif n.op == "attention":
            a = n.attrs
            spec = KernelSpec(name="attention", kind="attention", attrs=dict(a))
            hk = a.get("kv_heads", a["heads"])
            for role, src, h in zip(("q", "k", "v"), n.inputs, (a["heads"], hk, hk)):
                spec.args.append(KernelArg(role, src, role, [a["batch"], a["seq"], h, a["head_dim"]]))
            spec.outputs.append(KernelOutput(n.name, "out"))
            k = new_kernel(spec, n)
            k.owned[n.name] = "out"
            owner[n.name] = k
        elif n.op == "ssd":
            a = n.attrs
            spec = KernelSpec(name="ssd", kind="ssd", attrs=dict(a))
            hp = [a["batch"], a["seq"], a["heads"], a["head_dim"]]
            hn = [a["batch"], a["seq"], a["heads"], a["state_dim"]]
            hpad = [a["batch"], a["seq"], a["heads"], a["pad"]]
            for role, src, view in zip(("c", "b", "x", "cum", "dt", "mask", "dskip"), n.inputs,
                                       (hn, hn, hp, hpad, hpad, None, hp)):
                spec.args.append(KernelArg(role, src, role, view))
            spec.args.append(KernelArg("xskip", n.inputs[2], "xskip", hp))
            k = new_kernel(spec, n)
            k.owned[n.name] = "acc"
            owner[n.name] = k
        elif n.op == "ssd_chunked":
            a = n.attrs
            spec = KernelSpec(name="ssd_chunked", kind="ssd_chunked", attrs=dict(a))
            grp = a.get("ngroups", a["heads"])
            views = ([a["batch"], a["seq"], grp, a["state_dim"]], [a["batch"], a["seq"], grp, a["state_dim"]],
                     [a["batch"], a["seq"], a["heads"], a["head_dim"]], [a["batch"], a["seq"], a["heads"]], None, None)
            for role, src, view in zip(("c", "b", "x", "dt", "A", "D"), n.inputs, views):
                spec.args.append(KernelArg(role, src, role, view))
            k = new_kernel(spec, n)
            k.owned[n.name] = "acc"
            owner[n.name] = k
        elif n.op == "conv1d":
            spec = KernelSpec(name="conv1d", kind="conv1d", attrs=dict(n.attrs))
            spec.args.append(KernelArg("x", n.inputs[0], "x"))
            spec.args.append(KernelArg("w", n.inputs[1], "w"))
            k = new_kernel(spec, n)
            k.owned[n.name] = "acc"
            owner[n.name] = k
        elif n.op == "embedding":
            table, ids = n.inputs
            if g[table].kind not in ("param", "const"):
                raise PartitionError(f"{n.name}: the embedding table must be a parameter")
            vocab, dim = g[table].type.shape
            spec = KernelSpec(name="embedding", kind="embedding",
                              attrs={"vocab": vocab, "dim": dim, "tokens": n.type.shape[0]})
            spec.args.append(KernelArg("table", table, "table"))
            spec.args.append(KernelArg("ids", ids, "ids"))
            spec.outputs.append(KernelOutput(n.name, "out"))
            k = new_kernel(spec, n)
            k.owned[n.name] = "out"
            owner[n.name] = k
        elif n.op == "batch_matmul":
            raise PartitionError(f"{n.name}: stand-alone batch_matmul has no kernel template")

    # --- a row sum of squares with no GEMM home becomes a normalisation kernel
    lhs_nodes = {k.lhs_node for k in kernels if k.lhs_node}
    for n in g:
        if n.op != "row_sumsq" or n.inputs[0] in lhs_nodes:
            continue
        x = n.inputs[0]
        rows, cols = g[x].type.shape
        spec = KernelSpec(name="norm", kind="gemm", lhs="lhs", k_extent=cols, grid={"rows": rows, "cols": cols})
        spec.args.append(KernelArg("lhs", x, "lhs"))
        spec.sumsq = True
        k = new_kernel(spec, n, x)
        k.column_cache[n.name] = "sumsq"
        owner[n.name] = k
        lhs_nodes.add(x)

    # --- epilogues
    for n in g:
        if n.kind != "compute" or n.op in ("matmul", "attention", "ssd", "ssd_chunked", "conv1d", "embedding",
                                               "row_sumsq"):
            continue
        if _column_source(g, n.name, memo) is not None:
            continue
        if any(i in owner and owner[i].spec.kind == "attention" for i in n.inputs):
            raise PartitionError(f"{n.name}: elementwise consumer of an attention output must be absorbed by a GEMM")
        homes = [owner[i] for i in n.inputs if i in owner and owner[i].spec.kind in _EPILOGUE_KINDS]
        homes = [k for k in homes if _tile_frame(k) == n.type.shape]
        col_srcs = [c for c in (_column_source(g, i, memo) for i in n.inputs) if c is not None]
        if not homes and col_srcs:
            cands = [k for k in kernels if k.lhs_node in col_srcs and _tile_frame(k) == n.type.shape]
            if cands:
                homes = [max(cands, key=lambda k: k.order_key)]
            else:
                continue  # a broadcast of the column: cloned into whichever kernel reads it
        if not homes:
            raise PartitionError(f"{n.name} ({n.op}): elementwise op on DRAM tensors has no kernel to live in")
        home = max(homes, key=lambda k: k.anchor_key)
        home.order_key = max(home.order_key, order[n.name])
        args = [_input_name(g, i, home, memo) for i in n.inputs]
        home.spec.epilogue.append(BodyOp(n.name, n.op, args, dict(n.attrs)))
        home.owned[n.name] = n.name
        owner[n.name] = home

    # --- outputs: values read outside their kernel
    users: dict[str, list[OpNode]] = {}
    for n in g:
        for i in n.inputs:
            users.setdefault(i, []).append(n)
    readers: dict[str, set[int]] = {}
    for kk in kernels:
        for a in kk.spec.args:
            readers.setdefault(a.tensor, set()).add(id(kk))
    for value, k in list(owner.items()):
        if k.spec.kind in ("attention", "embedding") or value not in k.owned:
            continue
        needed = value in g.outputs or any(
            u.name not in k.owned for u in users.get(value, ()) if u.name in owner or u.op in ("attention", "matmul"))
        needed = needed or bool(readers.get(value, set()) - {id(k)})
        if needed and value not in k.spec.output_tensors():
            k.spec.outputs.append(KernelOutput(value, k.owned[value]))

    ordered = _order_kernels(kernels)
    for i, k in enumerate(ordered):
        k.spec.name = f"k{i}_{k.spec.kind}"
    params = sorted({a.tensor for k in ordered for a in k.spec.args if g[a.tensor].kind in ("param", "const")})
    prog = Program(name=name, inputs=list(g.inputs), outputs=list(g.outputs), tensors=tensors,
                   kernels=[k.spec for k in ordered], params=params, metadata=dict(g.metadata))
    prog.metadata["grouping"] = dict(grouping)
    return prog


def _input_name(g: OpGraph, src: str, home: _Kernel, memo: dict) -> str:
    """In-kernel value name for graph value ``src`` read by ``home``'s epilogue."""
    if src in home.owned:
        return home.owned[src]
    if _column_source(g, src, memo) is not None:
        return _clone_column(g, src, home, memo)
    node = g[src]
    if node.op == "broadcast" and _column_source(g, node.inputs[0], memo) is not None:
        inner = _clone_column(g, node.inputs[0], home, memo)
        key = f"bcast:{node.inputs[0]}:{node.attrs.get('shape')}"
        if key not in home.column_cache:
            bname = f"{node.name}__{len(home.column_cache)}"
            home.spec.epilogue.append(BodyOp(bname, "broadcast", [inner], dict(node.attrs)))
            home.column_cache[key] = bname
        home.owned[node.name] = home.column_cache[key]
        return home.column_cache[key]
    if src in home.extra_args:
        return home.extra_args[src]
    arg = f"in{len(home.extra_args)}"
    view = None
    if home.spec.kind == "ssd":
        a = home.spec.attrs
        view = [a["batch"], a["seq"], a["heads"], a["head_dim"]]
    home.spec.args.append(KernelArg(arg, src, "extra", view))
    home.extra_args[src] = arg
    return arg


def _clone_column(g: OpGraph, name: str, home: _Kernel, memo: dict) -> str:
    if name in home.column_cache:
        return home.column_cache[name]
    node = g[name]
    x = _column_source(g, name, memo)
    if node.op == "row_sumsq":
        if home.lhs_node != x:
            raise PartitionError(f"{home.spec.name}: needs the row sum of squares of {x} but its LHS is {home.lhs_node}")
        home.spec.sumsq = True
        home.column_cache[name] = "sumsq"
        return "sumsq"
    ins = [_clone_column(g, i, home, memo) for i in node.inputs]
    local = f"{name}__col"
    home.spec.epilogue.append(BodyOp(local, node.op, ins, dict(node.attrs)))
    home.column_cache[name] = local
    return local


def _order_kernels(kernels: list[_Kernel]) -> list[_Kernel]:
    """Topological order, earliest graph position first among the ready kernels
    (kernels are compared by identity: two kernels may hold equal specs)."""
    produced = {o.tensor: k for k in kernels for o in k.spec.outputs}
    done: list[_Kernel] = []
    done_ids: set[int] = set()
    remaining = sorted(kernels, key=lambda k: k.order_key)
    while remaining:
        left: list[_Kernel] = []
        for k in remaining:
            deps = [produced[a.tensor] for a in k.spec.args if a.tensor in produced and produced[a.tensor] is not k]
            if all(id(d) in done_ids for d in deps):
                done.append(k)
                done_ids.add(id(k))
            else:
                left.append(k)
        if len(left) == len(remaining):
            raise PartitionError("cyclic kernel dependencies")
        remaining = left
    return done
