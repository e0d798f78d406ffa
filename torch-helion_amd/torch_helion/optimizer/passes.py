"""Canonicalisation: raw (ATen-shaped) OpGraph -> kernel-ready OpGraph.

Same rewrite pipeline as the reference (optimizer/passes.py:899-944): fold
parameter-only sub-graphs, recognise RoPE / RMSNorm / attention / the SSD
scan, commute the RMS row scale into the consuming GEMMs, push feature slices
into GEMM weights, flatten to token-major 2-D, rewrite unregistered ops into
registered ones and make broadcasts explicit. Each pass is ``fn(g) -> int``
(number of rewrites) and works in place; :func:`canonicalize` runs them in
order and, given inputs, re-evaluates the graph after each pass.

Additive extensions for the MI355X configs:
* ``match_attention`` also accepts a constant causal additive bias on the
  scores (``attrs["causal"] = True``) and grouped K/V heads broadcast with
  unsqueeze/expand/reshape (``attrs["kv_heads"]``);
* ``match_conv`` turns ``pad -> depthwise convolution (-> silu)`` over the
  sequence into one ``conv1d`` op on token-major tensors;
* ``match_ssd`` emits ``ssd_chunked`` with the raw ``dt`` [T, H] and per-head
  ``A`` and ``D`` vectors instead of the reference's [T, T] decay GEMM and
  padded operands, so the scan can run in linear time with difference-form
  exponents (no overflow at any sequence length).
"""

from __future__ import annotations

import math
from typing import Callable

import torch

from ..capture.opgraph import OpGraph, OpNode, TensorType
from ..capture.ops import BINARY_OPS
from . import param_transforms as pt
from .evaluate import eval_op, graph_outputs, max_rel_err
from .layout import is_head_merge, match_head_split, trace_layout


class PassError(RuntimeError):
    """The graph holds a construct the lowering cannot express."""


# ------------------------------------------------------------------ helpers
def _convert(node: OpNode, op: str, inputs: list[str], attrs: dict | None = None, kind: str = "compute",
             type: TensorType | None = None) -> None:
    node.op, node.inputs, node.attrs, node.kind = op, list(inputs), dict(attrs or {}), kind
    if type is not None:
        node.type = type


def _is_const(g: OpGraph, name: str) -> bool:
    return g[name].kind in ("param", "const")


def _twod(shape: tuple[int, ...]) -> tuple[int, int]:
    if len(shape) == 0:
        return (1, 1)
    if len(shape) == 1:
        return (1, shape[0])
    return (math.prod(shape[:-1]), shape[-1])


def _ensure_2d(g: OpGraph, name: str) -> str:
    node = g[name]
    if node.type.rank == 2:
        return name
    shape = _twod(node.type.shape)
    return g.add("view", [name], TensorType(shape, node.type.dtype), {"shape": list(shape)}, kind="layout",
                 origin=f"ensure_2d({name})").name


def _skip_casts(g: OpGraph, node: OpNode) -> OpNode:
    while node.op == "cast" and len(node.inputs) == 1:
        node = g[node.inputs[0]]
    return node


def _through_layout(g: OpGraph, name: str) -> OpNode:
    node = g[name]
    while node.kind == "layout" and len(node.inputs) == 1:
        node = g[node.inputs[0]]
    return node


def _effective_users(g: OpGraph, name: str) -> list[tuple[OpNode, OpNode | None]]:
    """Users of ``name`` seen through identity reshapes: (consumer, via-layout)."""
    out: list[tuple[OpNode, OpNode | None]] = []
    for u in g.users(name):
        if u.kind == "layout" and u.op in ("view", "clone", "expand", "cast") and trace_layout(g, u.name).is_identity_reshape():
            out.extend((uu, u) for uu, _ in _effective_users(g, u.name))
        else:
            out.append((u, None))
    if name in g.outputs:
        out.append((OpNode("<output>", "output", [name], g[name].type), None))
    return out


def _rebuild_chain(g: OpGraph, chain: list[str], new_base: str, target: OpNode) -> None:
    """Replay the layout chain ``chain`` on ``new_base``; the last op is written
    into ``target`` so its users stay valid."""
    prev = new_base
    base_shape = g[g[chain[0]].inputs[0]].type.shape if chain else target.type.shape
    if g[prev].type.shape != base_shape:
        prev = g.add("view", [prev], TensorType(base_shape, g[prev].type.dtype), {"shape": list(base_shape)},
                     kind="layout").name
    if not chain:
        _convert(target, "view", [prev], {"shape": list(target.type.shape)}, kind="layout")
        return
    for lname in chain[:-1]:
        ln = g[lname]
        prev = g.add(ln.op, [prev], ln.type, dict(ln.attrs), kind="layout").name
    last = g[chain[-1]]
    _convert(target, last.op, [prev], dict(last.attrs), kind="layout", type=last.type)


def _binary_operands(g: OpGraph, node: OpNode, op: str) -> tuple[OpNode, OpNode] | None:
    if node.op != op or len(node.inputs) != 2 or "scalar" in node.attrs:
        return None
    return g[node.inputs[0]], g[node.inputs[1]]


def _mul_factors(g: OpGraph, node: OpNode, out: list[OpNode] | None = None) -> list[OpNode]:
    """Factors of a tree of two-operand ``mul`` nodes (layout nodes transparent)."""
    out = [] if out is None else out
    if node.kind == "layout":
        node = _through_layout(g, node.name)
    if node.op == "mul" and len(node.inputs) == 2 and "scalar" not in node.attrs:
        for i in node.inputs:
            _mul_factors(g, g[i], out)
    else:
        out.append(node)
    return out


def _per_head_vector(g: OpGraph, node: OpNode, heads: int) -> torch.Tensor | None:
    """A constant varying only along an axis of length ``heads``, as [heads]."""
    if not _is_const(g, node.name):
        return None
    v = g.value(node.name).float()
    if v.numel() == heads:
        return v.reshape(-1)
    for axis, size in enumerate(v.shape):
        if size != heads:
            continue
        moved = v.movedim(axis, 0).reshape(heads, -1)
        if torch.equal(moved, moved[:, :1].expand_as(moved)):
            return moved[:, 0].clone()
    return None


# ------------------------------------------------------------------- passes
def fold_constants(g: OpGraph) -> int:
    """Nodes whose inputs are all constants become constants."""
    n = 0
    for node in list(g):
        if node.kind in ("input", "param", "const") or not node.inputs:
            continue
        if all(_is_const(g, i) for i in node.inputs):
            val = eval_op(node.op, [g.value(i) for i in node.inputs], node.attrs)
            val = val.reshape(node.type.shape).to(node.type.torch_dtype).contiguous()
            _convert(node, "const", [], {}, kind="const")
            g.params[node.name] = val
            n += 1
    return n


def match_softplus(g: OpGraph) -> int:
    """``where(x > t, x, log1p(exp(x)))`` -> ``softplus(x)`` (the threshold guard
    is dropped, as in the reference; activations sit far below it)."""
    n = 0
    for node in list(g):
        if node.op != "select" or len(node.inputs) != 3:
            continue
        cond, big, small = (g[i] for i in node.inputs)
        if cond.op != "cmp_gt" or "scalar" not in cond.attrs:
            continue
        x = cond.inputs[0]
        if big.name != x or small.op != "log1p":
            continue
        e = g[small.inputs[0]]
        if e.op != "exp" or e.inputs[0] != x:
            continue
        _convert(node, "softplus", [x], {"threshold": float(cond.attrs["scalar"])})
        n += 1
    return n


def match_rotate_half(g: OpGraph) -> int:
    n = 0
    for node in list(g):
        if node.op != "cat" or len(node.inputs) != 2 or node.attrs["dim"] != node.type.rank - 1:
            continue
        a, b = g[node.inputs[0]], g[node.inputs[1]]
        if a.op != "neg" or b.op != "slice":
            continue
        sa = g[a.inputs[0]]
        if sa.op != "slice" or sa.inputs[0] != b.inputs[0]:
            continue
        d = g[sa.inputs[0]].type.shape[-1]
        if (sa.attrs["start"], sa.attrs["end"], b.attrs["start"], b.attrs["end"]) != (d // 2, d, 0, d // 2):
            continue
        if sa.attrs["dim"] != node.type.rank - 1 or b.attrs["dim"] != node.type.rank - 1:
            continue
        _convert(node, "rotate_half", [sa.inputs[0]], {})
        n += 1
    return n


def match_rope(g: OpGraph) -> int:
    n = 0
    for node in list(g):
        ops = _binary_operands(g, node, "add")
        if ops is None:
            continue
        found = None
        for plain, rot in (ops, ops[::-1]):
            if plain.op != "mul" or rot.op != "mul" or "scalar" in plain.attrs or "scalar" in rot.attrs:
                continue
            for xi in (0, 1):
                x, cos = plain.inputs[xi], plain.inputs[1 - xi]
                for ri in (0, 1):
                    r, sin = g[rot.inputs[ri]], rot.inputs[1 - ri]
                    if r.op == "rotate_half" and r.inputs[0] == x and _is_const(g, cos) and _is_const(g, sin):
                        found = (x, cos, sin)
        if found is None:
            continue
        x, cos, sin = found
        _convert(node, "rope", [x, cos, sin], {"head_dim": g[x].type.shape[-1]})
        n += 1
    return n


def lower_rope(g: OpGraph) -> int:
    """rope on a head-split GEMM output -> token-major ``y = a*cos + (x@(W R))*sin``
    with the rotation folded into a sibling GEMM weight (reference:
    optimizer/passes.py:186-219). The backend re-fuses the sibling."""
    n = 0
    for node in list(g):
        if node.op != "rope":
            continue
        x4, cos, sin = node.inputs
        prov = trace_layout(g, x4)
        dims = match_head_split(prov)
        if dims is None:
            raise PassError(f"rope {node.name}: input is not a head-split view of a token-major tensor")
        b, s, h, d = dims["batch"], dims["seq"], dims["heads"], dims["head_dim"]
        base = g[prov.base]
        base2d = _ensure_2d(g, base.name)
        t2 = g[base2d].type
        cos_full = pt.expand_rope_table(g.value(cos).reshape(s, d), b, h).to(t2.torch_dtype)
        sin_full = pt.expand_rope_table(g.value(sin).reshape(s, d), b, h).to(t2.torch_dtype)
        cos_c = g.add_const(cos_full, name=g.fresh_name("rope_cos"))
        sin_c = g.add_const(sin_full, name=g.fresh_name("rope_sin"))
        if base.op == "matmul" and _is_const(g, base.inputs[1]):
            wr = pt.rotate_columns(g.value(base.inputs[1]), h, d)
            wr_c = g.add_const(wr, name=g.fresh_name(base.inputs[1] + "_rot"))
            rot = g.add("matmul", [base.inputs[0], wr_c.name], base.type, origin=f"lower_rope({node.name})")
            rot2d = _ensure_2d(g, rot.name)
        else:
            r_c = g.add_const(pt.rotate_half_heads_matrix(h, d).to(t2.torch_dtype), name=g.fresh_name("rope_R"))
            rot2d = g.add("matmul", [base2d, r_c.name], t2, origin=f"lower_rope({node.name})").name
        m1 = g.add("mul", [base2d, cos_c.name], t2)
        m2 = g.add("mul", [rot2d, sin_c.name], t2)
        y = g.add("add", [m1.name, m2.name], t2, origin=f"lower_rope({node.name})")
        _rebuild_chain(g, prov.chain, y.name, node)
        n += 1
    g.toposort()
    return n


def match_rmsnorm(g: OpGraph) -> int:
    """``x * rsqrt(mean(x^2) + eps) * g`` -> ``rmsnorm(x, g)``."""
    n = 0
    for node in list(g):
        ops = _binary_operands(g, node, "mul")
        if ops is None:
            continue
        done = False
        for inner, gain in (ops, ops[::-1]):
            if done or not _is_const(g, gain.name) or inner.op != "mul" or len(inner.inputs) != 2:
                continue
            for x, r in ((g[inner.inputs[0]], g[inner.inputs[1]]), (g[inner.inputs[1]], g[inner.inputs[0]])):
                if r.op != "rsqrt":
                    continue
                add = g[r.inputs[0]]
                if add.op != "add" or "scalar" not in add.attrs:
                    continue
                mean = g[add.inputs[0]]
                if mean.op != "row_mean":
                    continue
                sq = g[mean.inputs[0]]
                ok = ((sq.op == "powf" and sq.attrs.get("scalar") == 2 and sq.inputs[0] == x.name)
                      or (sq.op == "square" and sq.inputs[0] == x.name)
                      or (sq.op == "mul" and sq.inputs == [x.name, x.name]))
                if not ok:
                    continue
                _convert(node, "rmsnorm", [x.name, gain.name], {"eps": float(add.attrs["scalar"])})
                n += 1
                done = True
                break
    return n


def _gemm_through_reshapes(g: OpGraph, name: str) -> OpNode | None:
    node = g[name]
    last = node.type.shape[-1]
    while node.kind == "layout" and node.op in ("view", "clone", "cast") and len(node.inputs) == 1:
        if node.type.shape[-1] != last or not trace_layout(g, node.name).is_identity_reshape():
            return None
        node = g[node.inputs[0]]
    if node.op == "matmul" and node.type.shape[-1] == last and _is_const(g, node.inputs[1]):
        return node
    return None


def push_slice_into_gemm(g: OpGraph) -> int:
    """``slice(a @ W, cols)`` -> ``a @ W[:, cols]``: a split projection becomes
    sibling GEMMs sharing the LHS (reference: optimizer/passes.py:389-416)."""
    n = 0
    progressed = True
    while progressed:
        progressed = False
        for node in list(g):
            if node.op != "slice" or node.attrs.get("dim") != g[node.inputs[0]].type.rank - 1:
                continue
            src = _gemm_through_reshapes(g, node.inputs[0])
            if src is None:
                continue
            lo, hi = node.attrs["start"], node.attrs["end"]
            wc = g.add_const(g.value(src.inputs[1])[:, lo:hi].contiguous(), name=g.fresh_name(src.inputs[1] + "_cols"))
            _convert(node, "matmul", [src.inputs[0], wc.name], {}, type=node.type)
            n += 1
            progressed = True
    g.toposort()
    return n


def _row_scale(g: OpGraph, x2d: str, eps: float, origin: str) -> str:
    """``(row_sumsq(x) / K + eps) ** -0.5`` as a [T, 1] column."""
    t, k = g[x2d].type.shape
    col = TensorType((t, 1), g[x2d].type.dtype)
    ss = g.add("row_sumsq", [x2d], col, origin=origin)
    m = g.add("mul", [ss.name], col, {"scalar": 1.0 / k})
    a = g.add("add", [m.name], col, {"scalar": eps})
    return g.add("powf", [a.name], col, {"scalar": -0.5}, origin=origin).name


def _lower_standalone_rmsnorm(g: OpGraph, node: OpNode) -> None:
    x, gain = node.inputs
    x2d = _ensure_2d(g, x)
    t, k = g[x2d].type.shape
    typ = g[x2d].type
    r = _row_scale(g, x2d, float(node.attrs["eps"]), f"rmsnorm({node.name})")
    bc = g.add("broadcast", [r], typ, {"dim": 1, "shape": [t, k]})
    scaled = g.add("mul", [x2d, bc.name], typ)
    gfull = g.add_const(torch.broadcast_to(g.value(gain).reshape(1, -1), (t, k)).contiguous(),
                        name=g.fresh_name(gain + "_full"))
    out = g.add("mul", [scaled.name, gfull.name], typ, origin=f"rmsnorm({node.name})")
    _rebuild_chain(g, [], out.name, node)


def lower_rmsnorm(g: OpGraph) -> int:
    """Commute the row scale through consuming GEMMs: gain folded into W, the
    [T, 1] scale applied to the accumulator (reference: optimizer/passes.py:252-285)."""
    n = 0
    for node in list(g):
        if node.op != "rmsnorm":
            continue
        x, gain = node.inputs
        eps = node.attrs["eps"]
        users = _effective_users(g, node.name)
        bad = [u for u, via in users
               if not (u.op == "matmul" and _is_const(g, u.inputs[1]) and u.inputs[0] == (via.name if via else node.name))]
        if bad:
            _lower_standalone_rmsnorm(g, node)
            n += 1
            continue
        x2d = _ensure_2d(g, x)
        r = _row_scale(g, x2d, eps, f"lower_rmsnorm({node.name})")
        gval = g.value(gain).reshape(-1)
        for mm, _via in users:
            w = mm.inputs[1]
            wg = g.add_const(pt.fold_gain_into_weight(gval, g.value(w)), name=g.fresh_name(w + "_norm"))
            g.fold_sources[wg.name] = (gval, g.value(w))
            flat = TensorType(_twod(mm.type.shape), mm.type.dtype)
            new_mm = g.add("matmul", [x2d, wg.name], flat, origin=f"lower_rmsnorm({mm.name})")
            bc = g.add("broadcast", [r], flat, {"dim": 1, "shape": list(flat.shape)})
            scaled = g.add("mul", [new_mm.name, bc.name], flat)
            _convert(mm, "view", [scaled.name], {"shape": list(mm.type.shape)}, kind="layout")
        n += 1
    g.toposort()
    return n


def _is_causal_bias(v: torch.Tensor, sq: int, skv: int) -> bool:
    """A constant [.., sq, skv] additive bias: 0 where key <= query, -inf (or
    below -1e4) strictly above the diagonal, identical across leading axes."""
    if v.dim() < 2 or tuple(v.shape[-2:]) != (sq, skv):
        return False
    m = v.reshape(-1, sq, skv).float()
    if not torch.equal(m, m[:1].expand_as(m)):
        return False
    m = m[0]
    qi = torch.arange(sq).unsqueeze(1) + (skv - sq)
    above = torch.arange(skv).unsqueeze(0) > qi
    return bool((m[~above] == 0).all() and (m[above] <= -1e4).all())


def match_attention(g: OpGraph) -> int:
    """bmm -> (scale) -> (+causal bias) -> softmax -> bmm with head-split
    operands -> one ``attention`` node on token-major tensors."""
    n = 0
    for sm in list(g):
        if sm.op != "softmax":
            continue
        s = _skip_casts(g, g[sm.inputs[0]])
        causal = False
        if s.op == "add" and len(s.inputs) == 2 and "scalar" not in s.attrs:
            a, b = g[s.inputs[0]], g[s.inputs[1]]
            bias, other = (b, a) if _is_const(g, b.name) else (a, b)
            if not _is_const(g, bias.name):
                continue
            bval = g.value(bias.name)
            if not _is_causal_bias(bval, s.type.shape[-2], s.type.shape[-1]):
                continue
            causal = True
            s = _skip_casts(g, other)
        scale = 1.0
        if s.op == "mul" and "scalar" in s.attrs:
            scale = float(s.attrs["scalar"])
            s = _skip_casts(g, g[s.inputs[0]])
        prov_s = trace_layout(g, s.name)
        bmm1 = g[prov_s.base]
        if bmm1.op != "batch_matmul" or not prov_s.is_identity_reshape():
            continue
        prov_q = trace_layout(g, bmm1.inputs[0])
        prov_k = trace_layout(g, bmm1.inputs[1])
        dq = match_head_split(prov_q)
        dk = match_head_split(prov_k, transpose_last=True, allow_grouped=True)
        if dq is None or dk is None:
            continue
        core = lambda d: (d["batch"], d["seq"], d["heads"], d["head_dim"])
        if core(dq) != core(dk):
            continue
        cons = [u for u, _ in _effective_users(g, sm.name)]
        if len(cons) != 1 or cons[0].op != "batch_matmul":
            continue
        bmm2 = cons[0]
        prov_p = trace_layout(g, bmm2.inputs[0])
        if prov_p.base != sm.name or not prov_p.is_identity_reshape():
            continue
        prov_v = trace_layout(g, bmm2.inputs[1])
        dv = match_head_split(prov_v, allow_grouped=True)
        if dv is None or core(dv) != core(dq) or dv.get("kv_heads") != dk.get("kv_heads"):
            continue
        b, sq, h, d = core(dq)
        # the last layout node of bmm2's single-user chain that reads it in token-major
        # [T, H*d] order (with S = 1 an earlier view of the chain already does, and
        # converting that one would leave the rest of the chain reading a 2-D tensor)
        final = None
        cur = bmm2
        while True:
            users = g.users(cur.name)
            if len(users) != 1 or users[0].kind != "layout":
                break
            cur = users[0]
            prov = trace_layout(g, cur.name)
            if prov.base == bmm2.name and is_head_merge(prov, b, sq, h, d):
                final = cur
        if final is None:
            continue
        attrs = {"batch": b, "seq": sq, "heads": h, "head_dim": d, "scale": scale}
        if causal:
            attrs["causal"] = True
        if "kv_heads" in dk:
            attrs["kv_heads"] = dk["kv_heads"]
        ins = [_ensure_2d(g, prov_q.base), _ensure_2d(g, prov_k.base), _ensure_2d(g, prov_v.base)]
        _convert(final, "attention", ins, attrs, type=TensorType((b * sq, h * d), final.type.dtype))
        n += 1
    g.toposort()
    return n


def match_conv(g: OpGraph) -> int:
    """``silu?(conv1d(pad(x^T, (k-1, 0)), w, groups=C))^T`` over each sequence ->
    ``conv1d(x2d, w[C, k])`` on the token-major tensor (depthwise causal conv).

    ``x`` may be a feature slice of a wider tensor (Mamba's xBC is a slice of
    the in_proj output); the slice stays in front of the conv, where
    ``push_slice_into_gemm`` later folds it into the projection weights."""
    n = 0
    for node in list(g):
        if node.op != "conv1d_raw":
            continue
        x, w = node.inputs[0], node.inputs[1]
        if len(node.inputs) > 2 or list(node.attrs.get("padding", [0])) != [0]:
            continue
        wv = g.value(w) if _is_const(g, w) else None
        pad = g[x]
        if wv is None or pad.op != "pad" or pad.attrs.get("value", 0.0) != 0.0:
            continue
        bs, ch, s_pad = pad.type.shape
        kk = wv.shape[-1]
        if node.attrs["groups"] != ch or tuple(wv.shape) != (ch, 1, kk) or list(pad.attrs["pad"]) != [kk - 1, 0]:
            continue
        seq = s_pad - (kk - 1)
        # the token-major source: the latest node of the chain holding [B, S, C] in row-major order
        src = None
        full = trace_layout(g, pad.inputs[0])
        for cand in reversed([full.base] + full.chain):
            if math.prod(g[cand].type.shape) != bs * seq * ch or g[cand].type.shape[-1] != ch:
                continue
            prov = trace_layout(g, pad.inputs[0], until=cand)
            if prov.base == cand and prov.shape == (bs, ch, seq) and prov.matches(
                    lambda p: (p[:, 0] * seq + p[:, 2]) * ch + p[:, 1]):
                src = cand
                break
        if src is None:
            continue
        act, y = None, node
        users = g.users(y.name)
        if len(users) == 1 and users[0].op == "silu":
            act, y = "silu", users[0]
            users = g.users(y.name)
        final = None
        for u in users:
            if u.kind != "layout":
                continue
            pu = trace_layout(g, u.name)
            if pu.base == y.name and pu.numel == bs * seq * ch and pu.matches(
                    lambda p, shp=pu.shape: (lambda f: ((f // ch) // seq * ch + f % ch) * seq + (f // ch) % seq)(
                        _flat(p, shp))):
                final = u
                break
        if final is None:
            continue
        if act is None and final.name not in g.outputs:
            # silu applied after the transpose back (the reference's _conv does this),
            # as one op or in its decomposed form x * sigmoid(x)
            act_node = _silu_of(g, final.name)
            if act_node is not None:
                act, final = "silu", act_node
        wc = g.add_const(wv.reshape(ch, kk).contiguous(), name=g.fresh_name(w + "_dw"))
        attrs = {"batch": bs, "seq": seq, "width": ch, "kernel": kk}
        if act:
            attrs["activation"] = act
        x2d = _ensure_2d(g, src)
        conv = g.add("conv1d", [x2d, wc.name], TensorType((bs * seq, ch), final.type.dtype), attrs,
                     origin=f"match_conv({node.name})")
        _rebuild_chain(g, [], conv.name, final)
        n += 1
    g.toposort()
    return n


def _silu_of(g: OpGraph, name: str) -> OpNode | None:
    """The node computing silu(name) if that is ``name``'s only consumer chain,
    as one ``silu`` op or decomposed ``x * sigmoid(x)``, optionally wrapped in
    the up/down casts a low-precision decomposition adds."""
    users = g.users(name)
    cast_in = None
    if len(users) == 1 and users[0].op == "cast":
        cast_in = users[0]
        name, users = cast_in.name, g.users(cast_in.name)
    act = None
    if len(users) == 1 and users[0].op == "silu":
        act = users[0]
    else:
        sig = [u for u in users if u.op == "sigmoid"]
        mul = [u for u in users if u.op == "mul" and "scalar" not in u.attrs]
        if (len(users) == 2 and len(sig) == 1 and len(mul) == 1 and sorted(mul[0].inputs) == sorted([name, sig[0].name])
                and g.users(sig[0].name) == [mul[0]]):
            act = mul[0]
    if act is None:
        return None
    after = g.users(act.name)
    if cast_in is not None and len(after) == 1 and after[0].op == "cast":
        return after[0]
    return act


def _flat(p: torch.Tensor, shape: tuple[int, ...]) -> torch.Tensor:
    f = torch.zeros(p.shape[0], dtype=torch.long)
    for k, s in enumerate(shape):
        f = f * s + p[:, k]
    return f


def push_slice_through_conv(g: OpGraph) -> int:
    """``slice(conv1d(x, w), cols)`` -> ``conv1d(slice(x, cols), w[cols])``: a
    depthwise conv is per channel, so the split of Mamba's conv output into x,
    B, C moves onto its input, where ``push_slice_into_gemm`` folds it into the
    in_proj weights."""
    n = 0
    for node in list(g):
        if node.op != "slice" or node.attrs.get("dim") != node.type.rank - 1:
            continue
        src = g[node.inputs[0]]
        while src.kind == "layout" and src.op in ("view", "clone") and trace_layout(g, src.name).is_identity_reshape():
            if src.type.shape[-1] != g[src.inputs[0]].type.shape[-1]:
                break
            src = g[src.inputs[0]]
        if src.op != "conv1d":
            continue
        lo, hi = node.attrs["start"], node.attrs["end"]
        x2d, w = src.inputs
        xt = g[x2d].type
        xs = g.add("slice", [x2d], TensorType((xt.shape[0], hi - lo), xt.dtype), {"dim": 1, "start": lo, "end": hi},
                   kind="layout")
        wc = g.add_const(g.value(w)[lo:hi].contiguous(), name=g.fresh_name(w + "_ch"))
        attrs = dict(src.attrs)
        attrs["width"] = hi - lo
        conv = g.add("conv1d", [xs.name, wc.name], TensorType((xt.shape[0], hi - lo), src.type.dtype), attrs,
                     origin=f"push_slice_through_conv({node.name})")
        _convert(node, "view", [conv.name], {"shape": list(node.type.shape)}, kind="layout")
        n += 1
    g.toposort()
    return n


def _ssd_head_scale(g: OpGraph, exp_node: OpNode, heads: int) -> torch.Tensor:
    """Per-head ``A``: the constant scaling ``dt`` inside the cumsum feeding exp."""
    seen: set[str] = set()
    stack = [exp_node.inputs[0]]
    while stack:
        name = stack.pop()
        if name in seen:
            continue
        seen.add(name)
        node = g[name]
        if node.op == "row_cumsum":
            for f in _mul_factors(g, _through_layout(g, node.inputs[0])):
                vec = _per_head_vector(g, f, heads)
                if vec is not None:
                    return vec
        stack.extend(node.inputs)
    raise PassError(f"ssd: no per-head A scale found under {exp_node.name}")


def _ssd_skip(g: OpGraph, start: OpNode, x_base: str, dims: dict) -> tuple[OpNode, torch.Tensor | None]:
    """Walk from the scan to its token-major result, absorbing ``y + D*x``."""
    b, sq, h, p = dims["batch"], dims["seq"], dims["heads"], dims["head_dim"]
    head_major, dvec = start, None
    frontier, seen = [start], {start.name}
    while frontier:
        node = frontier.pop()
        for u in g.users(node.name):
            if u.name in seen:
                continue
            seen.add(u.name)
            if u.kind == "layout":
                frontier.append(u)
                continue
            if u.op != "add" or len(u.inputs) != 2:
                continue
            other = next((i for i in u.inputs if i not in seen), None)
            if other is None:
                continue
            prod = _through_layout(g, other)
            if prod.op != "mul" or len(prod.inputs) != 2:
                continue
            for a, c in ((0, 1), (1, 0)):
                vec = _per_head_vector(g, _through_layout(g, prod.inputs[c]), h)
                if vec is None or trace_layout(g, prod.inputs[a]).base != x_base:
                    continue
                dvec, head_major = vec, u
                break
            if dvec is not None:
                frontier = []
                break
    cur = head_major
    while True:
        users = g.users(cur.name)
        if len(users) != 1 or users[0].kind != "layout":
            return head_major, dvec
        cur = users[0]
        prov = trace_layout(g, cur.name)
        if prov.base == head_major.name and is_head_merge(prov, b, sq, h, p):
            return cur, dvec


def match_ssd(g: OpGraph, chunk: int = 0) -> int:
    """The Mamba-2 scan in quadratic form -> one ``ssd_chunked`` node.

    Recognises ``(C B^T * exp(cumA_i - cumA_j) * causal * dt_j) X`` over
    head-major views of token-major tensors (the pattern of the reference's
    match_ssd, optimizer/passes.py:528-610), with B/C shared by ``ngroups``
    groups. Emits raw ``dt`` [T, H], ``A`` [H] and ``D`` [H]; the kernel forms
    the running decay per chunk itself.
    """
    n = 0
    for y in list(g):
        if y.op != "batch_matmul":
            continue
        prov_x = trace_layout(g, y.inputs[1])
        dims = match_head_split(prov_x)
        if dims is None:
            continue
        factors = _mul_factors(g, _through_layout(g, y.inputs[0]))
        cbs = [f for f in factors if f.op == "batch_matmul"]
        exps = [f for f in factors if f.op == "exp"]
        if len(cbs) != 1 or len(exps) != 1:
            continue
        cb = cbs[0]
        prov_c, prov_b = trace_layout(g, cb.inputs[0]), trace_layout(g, cb.inputs[1])
        dc = match_head_split(prov_c, allow_grouped=True)
        db = match_head_split(prov_b, transpose_last=True, allow_grouped=True)
        key = lambda d: None if d is None else (d["batch"], d["seq"], d["heads"])
        if key(dc) != key(dims) or key(db) != key(dims) or dc != db:
            continue
        rest = [f for f in factors if f not in (cb, exps[0])]
        dt_bases = [trace_layout(g, f.name).base for f in rest if not _is_const(g, f.name)]
        dt_tm = next((bb for bb in dt_bases if g[bb].type.shape[-1] == dims["heads"]), None)
        if dt_tm is None:
            continue
        b, sq, h, p = dims["batch"], dims["seq"], dims["heads"], dims["head_dim"]
        groups = dc.get("kv_heads", h)
        state = dc["head_dim"]
        a_vec = _ssd_head_scale(g, exps[0], h)
        final, dvec = _ssd_skip(g, y, prov_x.base, dims)
        if dvec is None:
            dvec = torch.zeros(h)
        q = chunk if chunk > 0 else (64 if sq <= 1024 else 256)
        q = min(q, sq)
        a_c = g.add_const(a_vec.float().contiguous(), name=g.fresh_name("ssd_A"))
        d_c = g.add_const(dvec.float().contiguous(), name=g.fresh_name("ssd_Dh"))
        dtype = g[prov_x.base].type.dtype
        node = g.add("ssd_chunked",
                     [_ensure_2d(g, prov_c.base), _ensure_2d(g, prov_b.base), _ensure_2d(g, prov_x.base),
                      _ensure_2d(g, dt_tm), a_c.name, d_c.name],
                     TensorType((b * sq, h * p), dtype),
                     {"batch": b, "seq": sq, "heads": h, "head_dim": p, "state_dim": state, "ngroups": groups,
                      "chunk": q},
                     origin=f"match_ssd({y.name})")
        _rebuild_chain(g, [], node.name, final)
        n += 1
    g.toposort()
    return n


def lower_cumsum(g: OpGraph) -> int:
    """A leftover ``row_cumsum(x)`` -> ``x @ P`` with an upper-triangular ones matrix."""
    n = 0
    for node in list(g):
        if node.op != "row_cumsum":
            continue
        x = g[node.inputs[0]]
        k = x.type.shape[-1]
        idx = torch.arange(k)
        pc = g.add_const((idx.unsqueeze(1) <= idx.unsqueeze(0)).to(x.type.torch_dtype), name=g.fresh_name("cumsum_prefix"))
        x2d = _ensure_2d(g, x.name)
        mm = g.add("matmul", [x2d, pc.name], g[x2d].type, origin=f"lower_cumsum({node.name})")
        _convert(node, "view", [mm.name], {"shape": list(node.type.shape)}, kind="layout")
        n += 1
    g.toposort()
    return n


def flatten_to_2d(g: OpGraph) -> int:
    """Drop identity reshapes; every activation becomes token-major 2-D in the
    model's activation dtype (reference: optimizer/passes.py:719-762)."""
    n = 0
    identity: list[tuple[str, str]] = []
    for node in list(g):
        if node.kind != "layout":
            continue
        prov = trace_layout(g, node.name)
        if node.op in ("view", "clone", "expand", "cast", "permute", "slice") and len(node.inputs) == 1 and prov.is_identity_reshape():
            identity.append((node.name, prov.base))
            continue
        raise PassError(f"layout op {node.name} ({node.op}) survived canonicalisation: {node.type} is a view of "
                        f"{prov.base} {g[prov.base].type} via {prov.chain}; only the head split of a kernel "
                        f"template can be absorbed")
    for name, base in identity:
        g.replace_all_uses(name, base)
        n += 1
    g.dce()
    input_shapes = {}
    for node in g:
        if node.kind in ("param", "const"):
            continue
        if node.kind == "input":
            input_shapes[node.name] = list(node.type.shape)
            if node.type.dtype in ("int64", "int32"):
                node.type = TensorType(_twod(node.type.shape), node.type.dtype)
                continue
        if node.op == "broadcast":
            node.attrs["shape"] = list(_twod(tuple(node.attrs["shape"])))
        node.type = TensorType(_twod(node.type.shape), node.type.dtype)
    float_inputs = [i for i in g.inputs if g[i].type.dtype not in ("int64", "int32")]
    # a model fed token ids computes in its embedding table's dtype
    tables = [g[n.inputs[0]].type.dtype for n in g if n.op == "embedding"]
    act = g.metadata.get("act_dtype") or (g[float_inputs[0]].type.dtype if float_inputs else
                                          tables[0] if tables else "float16")
    for node in g:
        if node.kind in ("param", "const", "input"):
            continue
        node.type = TensorType(node.type.shape, act)
    g.metadata.setdefault("input_shapes", input_shapes)
    g.metadata.setdefault("output_shapes", g.metadata.get("output_shapes_raw", {}))
    g.metadata["dtype"] = act
    return n


def materialize_const_operands(g: OpGraph) -> int:
    """A rank-1 / broadcast constant operand of a binary op -> full 2-D constant."""
    n = 0
    for node in list(g):
        if node.op not in BINARY_OPS or "scalar" in node.attrs or len(node.inputs) != 2:
            continue
        for idx in (0, 1):
            c, other = g[node.inputs[idx]], g[node.inputs[1 - idx]]
            if c.kind not in ("param", "const") or c.type.shape == other.type.shape or other.kind in ("param", "const"):
                continue
            rows, cols = other.type.shape
            v = g.value(c.name).float()
            if v.numel() == cols:
                full = v.reshape(1, cols).expand(rows, cols)
            elif v.numel() == rows:
                full = v.reshape(rows, 1).expand(rows, cols)
            elif v.numel() == 1:
                full = v.reshape(1, 1).expand(rows, cols)
            else:
                continue
            new = g.add_const(full.contiguous().to(other.type.torch_dtype), name=g.fresh_name(c.name + "_full"))
            node.inputs[idx] = new.name
            n += 1
    g.toposort()
    return n


def rewrite_unregistered(g: OpGraph) -> int:
    """neg/rsqrt/sqrt/square/sigmoid/silu/tanh/log1p/softplus/row_mean ->
    registered ops (reference: optimizer/passes.py:765-825)."""
    n = 0
    for node in list(g):
        if node.kind != "compute":
            continue
        t = node.type
        x = node.inputs[0] if node.inputs else None
        op = node.op
        if op == "neg":
            _convert(node, "mul", [x], {"scalar": -1.0})
        elif op == "rsqrt":
            _convert(node, "powf", [x], {"scalar": -0.5})
        elif op == "sqrt":
            _convert(node, "powf", [x], {"scalar": 0.5})
        elif op == "square":
            _convert(node, "mul", [x, x], {})
        elif op in ("sigmoid", "silu", "tanh"):
            src = g.add("mul", [x], t, {"scalar": 2.0}).name if op == "tanh" else x
            neg = g.add("mul", [src], t, {"scalar": -1.0})
            e = g.add("exp", [neg.name], t)
            den = g.add("add", [e.name], t, {"scalar": 1.0})
            if op == "sigmoid":
                _convert(node, "div", [den.name], {"scalar": 1.0, "scalar_first": True})
            elif op == "silu":
                sig = g.add("div", [den.name], t, {"scalar": 1.0, "scalar_first": True})
                _convert(node, "mul", [x, sig.name], {})
            else:
                sig = g.add("div", [den.name], t, {"scalar": 1.0, "scalar_first": True})
                two = g.add("mul", [sig.name], t, {"scalar": 2.0})
                _convert(node, "add", [two.name], {"scalar": -1.0})
        elif op == "log1p":
            _convert(node, "log", [g.add("add", [x], t, {"scalar": 1.0}).name], {})
        elif op == "softplus":
            e = g.add("exp", [x], t)
            one = g.add("add", [e.name], t, {"scalar": 1.0})
            _convert(node, "log", [one.name], {})
        elif op == "row_mean":
            k = g[x].type.shape[-1]
            s = g.add("row_sum", [x], t)
            _convert(node, "mul", [s.name], {"scalar": 1.0 / k})
        elif op in ("softmax", "rmsnorm", "rope", "rotate_half", "row_cumsum", "cmp_gt", "select", "pad", "conv1d_raw"):
            raise PassError(f"{node.name}: '{op}' could not be lowered to a kernel template")
        else:
            continue
        n += 1
    for node in g:
        if node.op in BINARY_OPS and "scalar" not in node.attrs:
            for i in node.inputs:
                if g[i].kind in ("param", "const") and g[i].type.rank < 2:
                    raise PassError(f"{node.name}: rank-{g[i].type.rank} operand {i} must be folded")
    g.toposort()
    return n


def insert_broadcasts(g: OpGraph) -> int:
    n = 0
    for node in list(g):
        if node.op not in BINARY_OPS or "scalar" in node.attrs or len(node.inputs) != 2:
            continue
        a, b = g[node.inputs[0]], g[node.inputs[1]]
        if a.type.shape == b.type.shape:
            continue
        for idx, (src, other) in enumerate(((a, b), (b, a))):
            if (src.type.rank == 2 and other.type.rank == 2 and src.type.shape[1] == 1
                    and src.type.shape[0] == other.type.shape[0] and other.type.shape[1] > 1):
                bc = g.add("broadcast", [src.name], other.type, {"dim": 1, "shape": list(other.type.shape)})
                node.inputs[idx] = bc.name
                n += 1
                break
        else:
            raise PassError(f"{node.name}: cannot broadcast {a.type} with {b.type}")
    g.toposort()
    return n


def dedupe_constants(g: OpGraph) -> int:
    """Merge constants holding identical tensors (e.g. RoPE tables)."""
    seen: dict[tuple, str] = {}
    n = 0
    for node in list(g):
        if node.kind != "const":
            continue
        v = g.value(node.name).contiguous()
        key = (node.type.shape, node.type.dtype, v.numel(), float(v.float().sum()) if v.numel() else 0.0)
        prev = seen.get(key)
        if prev is not None and torch.equal(g.value(prev), v):
            g.replace_all_uses(node.name, prev)
            n += 1
        elif prev is None:
            seen[key] = node.name
    return n


def cleanup(g: OpGraph) -> int:
    n = g.dce()
    g.toposort()
    return n


PASSES: list[tuple[str, Callable[[OpGraph], int]]] = [
    ("fold_constants", fold_constants),
    ("match_softplus", match_softplus),
    ("match_rotate_half", match_rotate_half),
    ("match_rope", match_rope),
    ("lower_rope", lower_rope),
    ("match_rmsnorm", match_rmsnorm),
    ("match_conv", match_conv),
    ("push_slice_through_conv", push_slice_through_conv),
    ("push_slice_into_gemm", push_slice_into_gemm),
    ("lower_rmsnorm", lower_rmsnorm),
    ("match_attention", match_attention),
    ("match_ssd", match_ssd),
    ("lower_cumsum", lower_cumsum),
    ("fold_constants_2", fold_constants),
    ("cleanup_1", cleanup),
    ("flatten_to_2d", flatten_to_2d),
    ("materialize_const_operands", materialize_const_operands),
    ("rewrite_unregistered", rewrite_unregistered),
    ("insert_broadcasts", insert_broadcasts),
    ("fold_constants_3", fold_constants),
    ("dedupe_constants", dedupe_constants),
    ("cleanup_2", cleanup),
]


def canonicalize(graph: OpGraph, verify_inputs: list[torch.Tensor] | None = None, tolerance: float = 2e-2,
                 ssd_chunk: int = 0) -> tuple[OpGraph, list[dict]]:
    """Run every pass on a copy of ``graph``; returns ``(graph, log)``. With
    ``verify_inputs`` the outputs are re-evaluated after each pass and compared
    with the raw graph's (max relative error <= ``tolerance``)."""
    g = graph.copy()
    g.metadata["output_shapes_raw"] = {o: list(g[o].type.shape) for o in g.outputs}
    raw_shapes = [list(g[o].type.shape) for o in g.outputs]
    ref = graph_outputs(g, verify_inputs) if verify_inputs is not None else None
    log: list[dict] = []
    for name, fn in PASSES:
        count = match_ssd(g, ssd_chunk) if fn is match_ssd else fn(g)
        entry = {"pass": name, "rewrites": count, "nodes": len(g)}
        if ref is not None:
            outs = graph_outputs(g, verify_inputs)
            err = max(max_rel_err(o.reshape(-1), r.reshape(-1)) for o, r in zip(outs, ref))
            entry["max_rel_err"] = err
            if err > tolerance:
                raise PassError(f"pass {name} changed the numerics (max rel err {err:.3e})")
        log.append(entry)
    # passes may rename an output node (an identity reshape folded into its base):
    # record the caller-visible shape under the final names, by position
    g.metadata["output_shapes"] = {o: shp for o, shp in zip(g.outputs, raw_shapes)}
    return g, log
