"""CPU semantics of every OpGraph op (reference: optimizer/evaluate.py:36-147).

Used at compile time for constant folding and for the per-pass numeric
check of the canonicalisation pipeline; never on the device path. Math runs
in fp32; the new kinds (causal / grouped-KV attention, ``ssd_chunked``,
``conv1d``, ``embedding``) are defined here by their plain formulas.
"""

from __future__ import annotations

from typing import Any, Callable

import torch
import torch.nn.functional as F

from ..capture.opgraph import OpGraph


def _binary(fn: Callable[[torch.Tensor, torch.Tensor], torch.Tensor], op: str):
    def run(xs: list[torch.Tensor], attrs: dict[str, Any]) -> torch.Tensor:
        if "scalar" in attrs:
            s = float(attrs["scalar"])
            a = xs[0]
            if op == "max":
                return torch.maximum(a, torch.full_like(a, s))
            if op == "powf" and attrs.get("scalar_first"):
                return torch.pow(torch.full_like(a, s), a)
            return fn(s, a) if attrs.get("scalar_first") else fn(a, s)
        return fn(xs[0], xs[1])
    return run


def rotate_half_last(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), -1)


def attention_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attrs: dict[str, Any]) -> torch.Tensor:
    b, s, h, d = attrs["batch"], attrs["seq"], attrs["heads"], attrs["head_dim"]
    hk = attrs.get("kv_heads", h)
    skv = attrs.get("seq_kv", s)
    q4 = q.reshape(b, s, h, d).transpose(1, 2)
    k4 = k.reshape(b, skv, hk, d).transpose(1, 2).repeat_interleave(h // hk, dim=1)
    v4 = v.reshape(b, skv, hk, d).transpose(1, 2).repeat_interleave(h // hk, dim=1)
    sc = torch.matmul(q4, k4.transpose(-1, -2)) * attrs["scale"]
    if attrs.get("causal"):
        qi = torch.arange(s).unsqueeze(1) + (skv - s)
        kj = torch.arange(skv).unsqueeze(0)
        sc = sc.masked_fill(kj > qi, float("-inf"))
    p = torch.softmax(sc, -1)
    return torch.matmul(p, v4).transpose(1, 2).reshape(b * s, h * d)


def ssd_quadratic_ref(xs: list[torch.Tensor], attrs: dict[str, Any]) -> torch.Tensor:
    """The reference's ``ssd`` kind: padded cum/dt operands, [S,S] mask, D skip."""
    cm, bm, xm, cum_pad, dt_pad, mask, d_full = xs
    bs, h, s = attrs["batch"], attrs["heads"], attrs["seq"]
    p, n, pad = attrs["head_dim"], attrs["state_dim"], attrs["pad"]
    c4 = cm.reshape(bs, s, h, n).transpose(1, 2)
    b4 = bm.reshape(bs, s, h, n).transpose(1, 2)
    x4 = xm.reshape(bs, s, h, p).transpose(1, 2)
    cum = cum_pad.reshape(bs, s, h, pad)[..., 0].transpose(1, 2)
    dt = dt_pad.reshape(bs, s, h, pad)[..., 0].transpose(1, 2)
    w = torch.matmul(c4, b4.transpose(-1, -2)) * mask
    v = x4 * (torch.exp(-cum) * dt).unsqueeze(-1)
    y = torch.matmul(w, v) * torch.exp(cum).unsqueeze(-1)
    return y.transpose(1, 2).reshape(bs * s, h * p) + xm * d_full


def ssd_chunked_ref(c: torch.Tensor, b: torch.Tensor, x: torch.Tensor, dt: torch.Tensor, a: torch.Tensor,
                    dvec: torch.Tensor, attrs: dict[str, Any]) -> torch.Tensor:
    """``ssd_chunked``: y_t = sum_{s<=t} (C_t.B_s) exp(cum_t - cum_s) dt_s x_s + D x_t,
    cum = running sum of dt*A, per (batch, head); B/C shared by ngroups groups.
    Evaluated chunk by chunk with difference-form exponents (no overflow)."""
    bs, s, h = attrs["batch"], attrs["seq"], attrs["heads"]
    p, n, g = attrs["head_dim"], attrs["state_dim"], attrs.get("ngroups", attrs["heads"])
    q = min(int(attrs.get("chunk", 64)), s)
    x4 = x.reshape(bs, s, h, p)
    c4 = c.reshape(bs, s, g, n).repeat_interleave(h // g, dim=2)
    b4 = b.reshape(bs, s, g, n).repeat_interleave(h // g, dim=2)
    dt3 = dt.reshape(bs, s, h)
    da = dt3 * a.reshape(1, 1, h)
    state = torch.zeros(bs, h, p, n, dtype=x.dtype)
    out = torch.empty(bs, s, h, p, dtype=x.dtype)
    for c0 in range(0, s, q):
        c1 = min(c0 + q, s)
        cum = torch.cumsum(da[:, c0:c1], 1)                             # [bs, l, h]
        cb = torch.einsum("bihn,bjhn->bhij", c4[:, c0:c1], b4[:, c0:c1])
        diff = cum.permute(0, 2, 1).unsqueeze(-1) - cum.permute(0, 2, 1).unsqueeze(-2)
        ll = c1 - c0
        tri = torch.ones(ll, ll, dtype=torch.bool).tril()
        decay = torch.where(tri, torch.exp(torch.where(tri, diff, torch.zeros_like(diff))), torch.zeros_like(diff))
        m = cb * decay * dt3[:, c0:c1].permute(0, 2, 1).unsqueeze(-2)
        y = torch.einsum("bhij,bjhp->bihp", m, x4[:, c0:c1])
        y = y + torch.einsum("bihn,bhpn->bihp", c4[:, c0:c1], state) * torch.exp(cum).unsqueeze(-1)
        out[:, c0:c1] = y
        last = cum[:, -1]                                                # [bs, h]
        w = dt3[:, c0:c1] * torch.exp(last.unsqueeze(1) - cum)         # [bs, l, h]
        state = state * torch.exp(last).reshape(bs, h, 1, 1) + torch.einsum(
            "blhp,blhn->bhpn", x4[:, c0:c1] * w.unsqueeze(-1), b4[:, c0:c1])
    out = out + x4 * dvec.reshape(1, 1, h, 1)
    return out.reshape(bs * s, h * p)


def conv1d_ref(x: torch.Tensor, w: torch.Tensor, attrs: dict[str, Any]) -> torch.Tensor:
    """Depthwise causal conv over each sequence of a token-major [B*S, W] tensor."""
    bs, s = attrs["batch"], attrs["seq"]
    width, kk = w.shape
    xb = x.reshape(bs, s, width).transpose(1, 2)
    y = F.conv1d(F.pad(xb, (kk - 1, 0)), w.unsqueeze(1), groups=width).transpose(1, 2).reshape(bs * s, width)
    if attrs.get("activation") == "silu":
        y = F.silu(y)
    return y


def _ssd(xs, attrs):
    return ssd_quadratic_ref(xs, attrs)


def _ssd_chunked(xs, attrs):
    return ssd_chunked_ref(*xs[:6], attrs)


def _rope(xs, attrs):
    x, cos, sin = xs
    return x * cos + rotate_half_last(x) * sin


def _rmsnorm(xs, attrs):
    x, g = xs
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + attrs["eps"]) * g


def _rotate_half_heads(xs, attrs):
    x, d = xs[0], attrs["head_dim"]
    return rotate_half_last(x.reshape(*x.shape[:-1], x.shape[-1] // d, d)).reshape(x.shape)


def _conv1d_raw(xs, attrs):
    x, w = xs[0], xs[1]
    y = F.conv1d(x, w, xs[2] if len(xs) > 2 else None, padding=attrs.get("padding", [0]), groups=attrs["groups"])
    return y


def _pad(xs, attrs):
    return F.pad(xs[0], attrs["pad"], value=attrs.get("value", 0.0))


_OPS: dict[str, Callable[[list[torch.Tensor], dict[str, Any]], torch.Tensor]] = {
    "add": _binary(lambda a, b: a + b, "add"),
    "sub": _binary(lambda a, b: a - b, "sub"),
    "mul": _binary(lambda a, b: a * b, "mul"),
    "div": _binary(lambda a, b: a / b, "div"),
    "max": _binary(torch.maximum, "max"),
    "powf": _binary(torch.pow, "powf"),
    "exp": lambda xs, a: torch.exp(xs[0]),
    "log": lambda xs, a: torch.log(xs[0]),
    "neg": lambda xs, a: -xs[0],
    "rsqrt": lambda xs, a: torch.rsqrt(xs[0]),
    "sqrt": lambda xs, a: torch.sqrt(xs[0]),
    "sigmoid": lambda xs, a: torch.sigmoid(xs[0]),
    "silu": lambda xs, a: F.silu(xs[0]),
    "tanh": lambda xs, a: torch.tanh(xs[0]),
    "square": lambda xs, a: xs[0] * xs[0],
    "log1p": lambda xs, a: torch.log1p(xs[0]),
    "softplus": lambda xs, a: F.softplus(xs[0]),
    "row_cumsum": lambda xs, a: torch.cumsum(xs[0], -1),
    "cmp_gt": lambda xs, a: (xs[0] > float(a["scalar"])) if "scalar" in a else (xs[0] > xs[1]),
    "row_sum": lambda xs, a: xs[0].sum(-1, keepdim=a.get("keepdim", True)),
    "row_max": lambda xs, a: xs[0].amax(-1, keepdim=a.get("keepdim", True)),
    "row_mean": lambda xs, a: xs[0].mean(-1, keepdim=a.get("keepdim", True)),
    "row_sumsq": lambda xs, a: (xs[0] * xs[0]).sum(-1, keepdim=True),
    "softmax": lambda xs, a: torch.softmax(xs[0], -1),
    "matmul": lambda xs, a: xs[0] @ xs[1],
    "batch_matmul": lambda xs, a: torch.bmm(xs[0], xs[1]),
    "broadcast": lambda xs, a: xs[0].expand(a["shape"]),
    "view": lambda xs, a: xs[0].reshape(a["shape"]),
    "permute": lambda xs, a: xs[0].permute(a["dims"]),
    "expand": lambda xs, a: xs[0].expand(a["shape"]),
    "clone": lambda xs, a: xs[0].clone(),
    "cast": lambda xs, a: xs[0].clone(),
    "slice": lambda xs, a: xs[0].narrow(a["dim"], a["start"], a["end"] - a["start"]),
    "cat": lambda xs, a: torch.cat(xs, a["dim"]),
    "rotate_half": lambda xs, a: rotate_half_last(xs[0]),
    "rotate_half_heads": _rotate_half_heads,
    "rope": _rope,
    "rmsnorm": _rmsnorm,
    "ssd": _ssd,
    "ssd_chunked": _ssd_chunked,
    "attention": lambda xs, a: attention_ref(xs[0], xs[1], xs[2], a),
    "attention_decode": lambda xs, a: attention_decode_ref(*xs, a),
    "conv1d": lambda xs, a: conv1d_ref(xs[0], xs[1], a),
    "conv1d_raw": _conv1d_raw,
    "pad": _pad,
    "embedding": lambda xs, a: F.embedding(xs[1].long(), xs[0]),
}


def attention_decode_ref(q, k_cache, v_cache, k_new, v_new, a: dict[str, Any]) -> torch.Tensor:
    """One query per sequence against the cache's first ``pos`` keys plus the new one:
    q [B, H*d]; caches [B*L, Hkv*d] (token-major, L = max_len); k_new, v_new [B, Hkv*d]."""
    b, h, hk, d, pos = a["batch"], a["heads"], a["kv_heads"], a["head_dim"], a["pos"]
    kc = k_cache.reshape(b, a["max_len"], hk * d)[:, :pos]
    vc = v_cache.reshape(b, a["max_len"], hk * d)[:, :pos]
    keys = torch.cat([kc, k_new.reshape(b, 1, hk * d)], 1)
    vals = torch.cat([vc, v_new.reshape(b, 1, hk * d)], 1)
    attrs = {"batch": b, "seq": 1, "seq_kv": pos + 1, "heads": h, "kv_heads": hk, "head_dim": d,
             "scale": a["scale"], "causal": False}
    qs = q.reshape(b, 1, h * d)
    outs = [attention_ref(qs[i], keys[i], vals[i], {**attrs, "batch": 1}) for i in range(b)]
    return torch.cat(outs, 0)


def eval_op(op: str, args: list[torch.Tensor], attrs: dict[str, Any]) -> torch.Tensor:
    """Evaluate one op on concrete tensors; floating operands are taken as fp32."""
    if op == "select":
        return torch.where(args[0].bool(), args[1].float(), args[2].float())
    xs = [a.float() if a.is_floating_point() else a for a in args]
    fn = _OPS.get(op)
    if fn is None:
        raise NotImplementedError(f"eval_op: {op}")
    return fn(xs, attrs)


def evaluate_graph(graph: OpGraph, inputs: dict[str, torch.Tensor] | list[torch.Tensor]) -> dict[str, torch.Tensor]:
    if isinstance(inputs, (list, tuple)):
        inputs = dict(zip(graph.inputs, inputs))
    env: dict[str, torch.Tensor] = {}
    for node in graph:
        if node.kind == "input":
            env[node.name] = inputs[node.name].reshape(node.type.shape)
        elif node.kind in ("param", "const"):
            env[node.name] = graph.value(node.name)
        else:
            out = eval_op(node.op, [env[i] for i in node.inputs], node.attrs)
            if tuple(out.shape) != node.type.shape:
                out = out.reshape(node.type.shape)
            env[node.name] = out
    return env


def graph_outputs(graph: OpGraph, inputs) -> list[torch.Tensor]:
    env = evaluate_graph(graph, inputs)
    return [env[o] for o in graph.outputs]


def max_rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max|a-b| / (max|b| + 1e-6): the reference's normalised error
    (reference: optimizer/evaluate.py:174-176)."""
    a, b = a.float(), b.float()
    return float((a - b).abs().max() / (b.abs().max() + 1e-6))
