"""Core-ATen FX graph -> raw OpGraph (reference: capture/fx_to_opgraph.py:80-335).

Each ATen node becomes one OpGraph node of the same shape; view-like nodes
become ``layout`` nodes. Parameters and buffers are attached with their
values. All semantic rewriting is left to the optimizer passes.

Added for the MI355X configs: ``constant_pad_nd`` (``pad``), depthwise
``convolution`` (``conv1d_raw``), ``embedding``, ``where`` with a scalar
branch, and scalar-tensor constants.
"""

from __future__ import annotations

from typing import Any, Callable

import torch
from torch.fx import Node

from .fx_capture import CapturedFx
from .opgraph import OpGraph, OpNode, TensorType


class UnsupportedOpError(NotImplementedError):
    """An ATen op has no OpGraph mapping."""


def _type_of(node: Node) -> TensorType:
    val = node.meta.get("val")
    if not isinstance(val, torch.Tensor):
        raise UnsupportedOpError(f"{node.name}: value is {type(val).__name__}, not a tensor")
    return TensorType(tuple(int(s) for s in val.shape), str(val.dtype).replace("torch.", ""))


def _dim(d: int, rank: int) -> int:
    return d + rank if d < 0 else d


class _Builder:
    def __init__(self, captured: CapturedFx) -> None:
        self.cap = captured
        self.ep = captured.exported
        self.g = OpGraph("model")
        self.alias: dict[str, str] = {}          # fx name -> opgraph name
        self.splits: dict[str, tuple[str, list[int], int]] = {}

    def ref(self, a: Any) -> str:
        if isinstance(a, Node):
            return self.alias[a.name]
        raise UnsupportedOpError(f"expected a tensor operand, got {a!r}")

    def emit(self, node: Node, op: str, ins: list[str], attrs: dict | None = None, kind: str = "compute") -> OpNode:
        out = self.g.add(op, ins, _type_of(node), attrs, kind=kind, name=node.name, origin=str(node.target))
        self.alias[node.name] = out.name
        return out

    def binary(self, node: Node, op: str) -> OpNode:
        a, b = node.args[0], node.args[1]
        if isinstance(a, Node) and isinstance(b, Node):
            return self.emit(node, op, [self.ref(a), self.ref(b)])
        if isinstance(a, Node):
            return self.emit(node, op, [self.ref(a)], {"scalar": float(b)})
        return self.emit(node, op, [self.ref(b)], {"scalar": float(a), "scalar_first": True})

    def run(self) -> OpGraph:
        sig = self.ep.graph_signature
        state = dict(self.ep.state_dict)
        consts = dict(getattr(self.ep, "constants", {}) or {})
        to_param = dict(sig.inputs_to_parameters)
        to_buffer = dict(sig.inputs_to_buffers)
        to_const = dict(getattr(sig, "inputs_to_lifted_tensor_constants", {}) or {})
        for node in self.cap.graph_module.graph.nodes:
            if node.op == "placeholder":
                t = _type_of(node)
                if node.name in to_param:
                    self._value(node, "param", to_param[node.name], state[to_param[node.name]], t)
                elif node.name in to_buffer:
                    key = to_buffer[node.name]
                    self._value(node, "param", key, state.get(key, consts.get(key)), t)
                elif node.name in to_const:
                    self._value(node, "const", to_const[node.name], consts[to_const[node.name]], t)
                else:
                    self._value(node, "input", node.name, None, t)
            elif node.op == "call_function":
                key = str(node.target)
                if key == "aten.split_with_sizes.default":
                    src = node.args[0]
                    rank = len(_type_of(src).shape)
                    dim = _dim(int(node.args[2]) if len(node.args) > 2 else 0, rank)
                    self.splits[node.name] = (self.ref(src), [int(v) for v in node.args[1]], dim)
                    continue
                fn = _HANDLERS.get(key)
                if fn is None:
                    raise UnsupportedOpError(f"no OpGraph mapping for {key} (node {node.name})")
                fn(self, node)
            elif node.op == "output":
                outs = node.args[0]
                outs = outs if isinstance(outs, (tuple, list)) else (outs,)
                self.g.outputs = [self.ref(o) for o in outs]
            else:
                raise UnsupportedOpError(f"unsupported fx node kind {node.op} ({node.name})")
        self.g.metadata["fx_op_histogram"] = self.cap.op_histogram()
        return self.g

    def _value(self, node: Node, kind: str, key: str, value: torch.Tensor | None, t: TensorType) -> None:
        name = key.replace(".", "_")
        v = None if value is None else value.detach().clone()
        out = self.g.add(kind, [], t, kind=kind, name=name, origin=node.name, value=v)
        self.alias[node.name] = out.name


_HANDLERS: dict[str, Callable[[_Builder, Node], Any]] = {}


def _on(*targets: str):
    def deco(fn):
        for t in targets:
            _HANDLERS[t] = fn
        return fn
    return deco


for _t, _op in {"aten.add.Tensor": "add", "aten.sub.Tensor": "sub", "aten.mul.Tensor": "mul",
                "aten.div.Tensor": "div", "aten.maximum.default": "max",
                "aten.add.Scalar": "add", "aten.mul.Scalar": "mul", "aten.sub.Scalar": "sub",
                "aten.div.Scalar": "div"}.items():
    _HANDLERS[_t] = lambda b, n, _op=_op: b.binary(n, _op)

for _t, _op in {"aten.exp.default": "exp", "aten.log.default": "log", "aten.neg.default": "neg",
                "aten.rsqrt.default": "rsqrt", "aten.sqrt.default": "sqrt", "aten.sigmoid.default": "sigmoid",
                "aten.silu.default": "silu", "aten.tanh.default": "tanh", "aten.square.default": "square",
                "aten.log1p.default": "log1p"}.items():
    _HANDLERS[_t] = lambda b, n, _op=_op: b.emit(n, _op, [b.ref(n.args[0])])


@_on("aten.pow.Tensor_Scalar")
def _pow_s(b, n):
    return b.emit(n, "powf", [b.ref(n.args[0])], {"scalar": float(n.args[1])})


@_on("aten.pow.Tensor_Tensor")
def _pow_t(b, n):
    return b.emit(n, "powf", [b.ref(n.args[0]), b.ref(n.args[1])])


@_on("aten.mean.dim", "aten.sum.dim_IntList", "aten.amax.default")
def _reduce(b, n):
    x = n.args[0]
    rank = len(_type_of(x).shape)
    dims = n.args[1] if len(n.args) > 1 else None
    dims = [dims] if isinstance(dims, int) else list(dims or [])
    keep = bool(n.args[2]) if len(n.args) > 2 else bool(n.kwargs.get("keepdim", False))
    if [_dim(d, rank) for d in dims] != [rank - 1]:
        raise UnsupportedOpError(f"{n.name}: only last-dim reductions are supported")
    op = {"aten.mean.dim": "row_mean", "aten.sum.dim_IntList": "row_sum", "aten.amax.default": "row_max"}[str(n.target)]
    return b.emit(n, op, [b.ref(x)], {"keepdim": keep})


@_on("aten._softmax.default", "aten.softmax.int")
def _softmax(b, n):
    rank = len(_type_of(n.args[0]).shape)
    if _dim(int(n.args[1]), rank) != rank - 1:
        raise UnsupportedOpError(f"{n.name}: softmax only over the last dim")
    return b.emit(n, "softmax", [b.ref(n.args[0])])


@_on("aten.mm.default")
def _mm(b, n):
    return b.emit(n, "matmul", [b.ref(n.args[0]), b.ref(n.args[1])])


@_on("aten.bmm.default")
def _bmm(b, n):
    return b.emit(n, "batch_matmul", [b.ref(n.args[0]), b.ref(n.args[1])])


@_on("aten.addmm.default")
def _addmm(b, n):
    bias, x, w = n.args[:3]
    mm = b.g.add("matmul", [b.ref(x), b.ref(w)], _type_of(n), name=n.name + "_mm", origin="aten.addmm")
    return b.emit(n, "add", [mm.name, b.ref(bias)])


@_on("aten.permute.default")
def _permute(b, n):
    return b.emit(n, "permute", [b.ref(n.args[0])], {"dims": [int(d) for d in n.args[1]]}, kind="layout")


@_on("aten.transpose.int")
def _transpose(b, n):
    rank = len(_type_of(n.args[0]).shape)
    dims = list(range(rank))
    i, j = _dim(int(n.args[1]), rank), _dim(int(n.args[2]), rank)
    dims[i], dims[j] = dims[j], dims[i]
    return b.emit(n, "permute", [b.ref(n.args[0])], {"dims": dims}, kind="layout")


@_on("aten.t.default")
def _t(b, n):
    return b.emit(n, "permute", [b.ref(n.args[0])], {"dims": [1, 0]}, kind="layout")


@_on("aten.view.default", "aten.reshape.default", "aten._unsafe_view.default", "aten.unsqueeze.default",
     "aten.squeeze.dim", "aten.squeeze.default", "aten.squeeze.dims")
def _view(b, n):
    return b.emit(n, "view", [b.ref(n.args[0])], {"shape": list(_type_of(n).shape)}, kind="layout")


@_on("aten.expand.default")
def _expand(b, n):
    return b.emit(n, "expand", [b.ref(n.args[0])], {"shape": list(_type_of(n).shape)}, kind="layout")


@_on("aten.clone.default", "aten.contiguous.default", "aten.alias.default", "aten.detach.default")
def _clone(b, n):
    return b.emit(n, "clone", [b.ref(n.args[0])], kind="layout")


@_on("aten._to_copy.default", "aten.to.dtype")
def _cast(b, n):
    return b.emit(n, "cast", [b.ref(n.args[0])], {"dtype": _type_of(n).dtype}, kind="layout")


@_on("aten.slice.Tensor")
def _slice(b, n):
    x = n.args[0]
    rank = len(_type_of(x).shape)
    dim = _dim(int(n.args[1]) if len(n.args) > 1 else 0, rank)
    size = _type_of(x).shape[dim]
    start = int(n.args[2]) if len(n.args) > 2 and n.args[2] is not None else 0
    end = int(n.args[3]) if len(n.args) > 3 and n.args[3] is not None else size
    step = int(n.args[4]) if len(n.args) > 4 else 1
    if step != 1:
        raise UnsupportedOpError(f"{n.name}: strided slices are not supported")
    start = max(0, start + size if start < 0 else start)
    end = min(size, end + size if end < 0 else end)
    return b.emit(n, "slice", [b.ref(x)], {"dim": dim, "start": start, "end": end}, kind="layout")


@_on("<built-in function getitem>")
def _getitem(b, n):
    src, idx = n.args[0], int(n.args[1])
    if not isinstance(src, Node) or src.name not in b.splits:
        raise UnsupportedOpError(f"{n.name}: getitem on something other than a tensor split")
    base, sizes, dim = b.splits[src.name]
    start = sum(sizes[:idx])
    return b.emit(n, "slice", [base], {"dim": dim, "start": start, "end": start + sizes[idx]}, kind="layout")


@_on("aten.cumsum.default")
def _cumsum(b, n):
    rank = len(_type_of(n.args[0]).shape)
    if _dim(int(n.args[1]) if len(n.args) > 1 else -1, rank) != rank - 1:
        raise UnsupportedOpError(f"{n.name}: only last-dim cumsum is supported")
    return b.emit(n, "row_cumsum", [b.ref(n.args[0])])


@_on("aten.gt.Scalar")
def _gt(b, n):
    return b.emit(n, "cmp_gt", [b.ref(n.args[0])], {"scalar": float(n.args[1])})


@_on("aten.where.self")
def _where(b, n):
    return b.emit(n, "select", [b.ref(a) for a in n.args[:3]])


@_on("aten.cat.default")
def _cat(b, n):
    rank = len(_type_of(n).shape)
    dim = _dim(int(n.args[1]) if len(n.args) > 1 else 0, rank)
    return b.emit(n, "cat", [b.ref(p) for p in n.args[0]], {"dim": dim}, kind="layout")


@_on("aten.constant_pad_nd.default")
def _pad(b, n):
    pads = [int(p) for p in n.args[1]]
    value = float(n.args[2]) if len(n.args) > 2 else 0.0
    return b.emit(n, "pad", [b.ref(n.args[0])], {"pad": pads, "value": value})


@_on("aten.convolution.default")
def _conv(b, n):
    x, w, bias, stride, padding, dilation, transposed, _outpad, groups = n.args[:9]
    if transposed or list(stride) != [1] or list(dilation) != [1]:
        raise UnsupportedOpError(f"{n.name}: only stride-1, undilated, non-transposed 1-D convolutions are supported")
    ins = [b.ref(x), b.ref(w)] + ([b.ref(bias)] if isinstance(bias, Node) else [])
    return b.emit(n, "conv1d_raw", ins, {"groups": int(groups), "padding": [int(p) for p in padding]})


@_on("aten.embedding.default")
def _embedding(b, n):
    return b.emit(n, "embedding", [b.ref(n.args[0]), b.ref(n.args[1])])


@_on("aten.linear.default")
def _linear(b, n):
    x, w = n.args[0], n.args[1]
    wt_t = _type_of(w)
    wt = b.g.add("permute", [b.ref(w)], TensorType(tuple(reversed(wt_t.shape)), wt_t.dtype), {"dims": [1, 0]},
                 kind="layout", name=n.name + "_wT", origin="aten.linear")
    if len(_type_of(x).shape) != 2:
        raise UnsupportedOpError(f"{n.name}: linear on a rank-{len(_type_of(x).shape)} input")
    if len(n.args) > 2 and n.args[2] is not None:
        mm = b.g.add("matmul", [b.ref(x), wt.name], _type_of(n), name=n.name + "_mm", origin="aten.linear")
        return b.emit(n, "add", [mm.name, b.ref(n.args[2])])
    return b.emit(n, "matmul", [b.ref(x), wt.name])


def fx_to_opgraph(captured: CapturedFx) -> OpGraph:
    return _Builder(captured).run()


def supported_aten_ops() -> list[str]:
    return sorted(_HANDLERS)
