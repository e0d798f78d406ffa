"""OpIR interpreter (oracle; test infrastructure only).

Restates the reference's codegen/interpret.py:18-77 (accumulators
``lhs @ rhs_i``, the row sum of squares, the epilogue SSA in order, the
attention and scan kinds) with the op semantics of optimizer/evaluate.py:36-147,
written independently of the product's interpreter and computing in float64
by default. New kinds follow their defining formulas: causal / grouped-KV
attention, ``ssd_chunked`` (the O(S) recurrence of oracle.mamba),
``conv1d`` (a direct sum over the kernel taps), ``embedding`` (row
indexing of the table: ``out[t] = table[ids[t]]``, what torch.nn.Embedding
defines) and ``attention_decode`` (one query per sequence against a cache's
first ``pos`` rows plus the new key/value); gemm weights may be e4m3 with
per-column scales and an activation-side norm gain.

``storage="declared"`` rounds every kernel output to the dtype the Program
declares for it, i.e. what a device that stores intermediates in their
declared dtype computes; ``storage=None`` keeps every value in ``dtype`` as
the reference interpreter does.
"""

from __future__ import annotations

import math
from typing import Any

import torch

_DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16, "float64": torch.float64}


def _scalar_op(op: str, x: torch.Tensor, s: float, first: bool) -> torch.Tensor:
    a, b = (s, x) if first else (x, s)
    if op == "add":
        return a + b
    if op == "sub":
        return a - b
    if op == "mul":
        return a * b
    if op == "div":
        return a / b
    if op == "max":
        return torch.clamp(x, min=s)
    if op == "powf":
        return torch.pow(torch.full_like(x, s), x) if first else torch.pow(x, s)
    raise ValueError(op)


def apply_op(op: str, xs: list[torch.Tensor], attrs: dict[str, Any]) -> torch.Tensor:
    """Registered epilogue ops (capture/ops.py:34-37 of the reference)."""
    if op in ("add", "sub", "mul", "div", "max", "powf"):
        if "scalar" in attrs:
            return _scalar_op(op, xs[0], float(attrs["scalar"]), bool(attrs.get("scalar_first", False)))
        a, b = xs
        if op == "add":
            return a + b
        if op == "sub":
            return a - b
        if op == "mul":
            return a * b
        if op == "div":
            return a / b
        if op == "max":
            return torch.maximum(a, b)
        return torch.pow(a, b)
    if op == "exp":
        return torch.exp(xs[0])
    if op == "log":
        return torch.log(xs[0])
    if op == "row_sum":
        return xs[0].sum(-1, keepdim=True)
    if op == "row_max":
        return xs[0].amax(-1, keepdim=True)
    if op == "broadcast":
        return xs[0].expand(attrs["shape"])
    raise NotImplementedError(f"oracle: epilogue op {op}")


def attention(q, k, v, a: dict[str, Any]) -> torch.Tensor:
    b, s, h, d = a["batch"], a["seq"], a["heads"], a["head_dim"]
    hk = a.get("kv_heads", h)
    skv = a.get("seq_kv", s)
    q4 = q.reshape(b, s, h, d).permute(0, 2, 1, 3)
    k4 = k.reshape(b, skv, hk, d).permute(0, 2, 1, 3)
    v4 = v.reshape(b, skv, hk, d).permute(0, 2, 1, 3)
    idx = torch.arange(h) // (h // hk)
    k4, v4 = k4[:, idx], v4[:, idx]
    sc = torch.einsum("bhid,bhjd->bhij", q4, k4) * a["scale"]
    if a.get("causal"):
        allowed = torch.arange(skv)[None, :] <= torch.arange(s)[:, None] + (skv - s)
        sc = sc.masked_fill(~allowed, float("-inf"))
    p = torch.softmax(sc, dim=-1)
    return torch.einsum("bhij,bhjd->bihd", p, v4).reshape(b * s, h * d)


def ssd_quadratic(c, bm, x, cum_pad, dt_pad, mask, d_full, a: dict[str, Any]) -> torch.Tensor:
    """The reference's ``ssd`` kind: sum_j (C_i.B_j) mask_ij exp(cum_i - cum_j) dt_j x_j + D x_i,
    cum/dt read from column 0 of each head's padded group (optimizer/evaluate.py:123-138)."""
    bs, s, h, p, n, pad = a["batch"], a["seq"], a["heads"], a["head_dim"], a["state_dim"], a["pad"]
    c4 = c.reshape(bs, s, h, n)
    b4 = bm.reshape(bs, s, h, n)
    x4 = x.reshape(bs, s, h, p)
    cum = cum_pad.reshape(bs, s, h, pad)[..., 0]
    dt = dt_pad.reshape(bs, s, h, pad)[..., 0]
    cb = torch.einsum("bihn,bjhn->bhij", c4, b4) * mask
    decay = torch.exp(cum.permute(0, 2, 1)[..., :, None] - cum.permute(0, 2, 1)[..., None, :])
    m = cb * decay * dt.permute(0, 2, 1)[..., None, :]
    y = torch.einsum("bhij,bjhp->bihp", m, x4).reshape(bs * s, h * p)
    return y + x * d_full


def conv1d(x, w, a: dict[str, Any]) -> torch.Tensor:
    """y[b, t, c] = sum_j w[c, j] x[b, t - (k-1) + j, c] (zero before t = 0), then SiLU."""
    bs, s = a["batch"], a["seq"]
    width, kk = w.shape
    xb = x.reshape(bs, s, width)
    y = torch.zeros_like(xb)
    for j in range(kk):
        shift = kk - 1 - j
        if shift == 0:
            y = y + w[:, j] * xb
        else:
            y[:, shift:] = y[:, shift:] + w[:, j] * xb[:, :-shift]
    if a.get("activation") == "silu":
        y = y * torch.sigmoid(y)
    return y.reshape(bs * s, width)


def run_kernel(spec, env: dict[str, torch.Tensor], dtype=torch.float64) -> dict[str, torch.Tensor]:
    from .mamba import ssd_chunked_program

    args = {a.name: env[a.tensor] for a in spec.args}
    vals: dict[str, torch.Tensor] = {}
    if spec.kind == "gemm":
        lhs = args["lhs"]
        # e4m3 weights: W = q * s per output column ("<rhs>_scale"); an activation-side norm
        # gain (role "gain") scales the lhs columns of the products only, not the sum of squares
        a_lhs = lhs * args["gain"] if "gain" in args else lhs
        for g in spec.gemms:
            w = args[g.rhs]
            if g.rhs + "_scale" in args:
                w = w * args[g.rhs + "_scale"]
            vals[g.acc] = a_lhs @ w
        if spec.sumsq:
            vals["sumsq"] = (lhs * lhs).sum(-1, keepdim=True)
    elif spec.kind == "attention":
        return {spec.outputs[0].tensor: attention(args["q"], args["k"], args["v"], spec.attrs)}
    elif spec.kind == "attention_decode":
        # keys/values: the cache's first pos rows of each sequence, then the new token's
        a = spec.attrs
        b, L, pos = a["batch"], a["max_len"], a["pos"]
        kw = a["kv_heads"] * a["head_dim"]
        keys = torch.cat([args["k_cache"].reshape(b, L, kw)[:, :pos], args["k_new"].reshape(b, 1, kw)], 1)
        vals_ = torch.cat([args["v_cache"].reshape(b, L, kw)[:, :pos], args["v_new"].reshape(b, 1, kw)], 1)
        out = [attention(args["q"].reshape(b, -1)[i:i + 1], keys[i], vals_[i],
                         {**a, "batch": 1, "seq": 1, "seq_kv": pos + 1, "causal": False}) for i in range(b)]
        return {spec.outputs[0].tensor: torch.cat(out, 0)}
    elif spec.kind == "ssd":
        vals["acc"] = ssd_quadratic(*(args[r] for r in ("c", "b", "x", "cum", "dt", "mask", "dskip")), spec.attrs)
    elif spec.kind == "ssd_chunked":
        vals["acc"] = ssd_chunked_program(*(args[r] for r in ("c", "b", "x", "dt", "A", "D")), spec.attrs)
    elif spec.kind == "conv1d":
        vals["acc"] = conv1d(args["x"], args["w"], spec.attrs)
    elif spec.kind == "embedding":
        ids = args["ids"].reshape(-1)
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= args["table"].shape[0]):
            raise IndexError("token id outside the embedding table")
        vals["out"] = args["table"][ids]
    else:
        raise ValueError(spec.kind)
    for a in spec.args:
        if a.role == "extra":
            vals[a.name] = args[a.name]
    for op in spec.epilogue:
        vals[op.name] = apply_op(op.op, [vals[i] for i in op.inputs], op.attrs)
    return {o.tensor: vals[o.value] for o in spec.outputs}


def run_program(program, params: dict[str, torch.Tensor], inputs, dtype=torch.float64,
                storage: str | None = None) -> dict[str, torch.Tensor]:
    if isinstance(inputs, (list, tuple)):
        inputs = dict(zip(program.inputs, inputs))
    conv = lambda t: t.to(dtype) if t.is_floating_point() else t
    env = {n: conv(inputs[n].reshape(program.tensors[n].shape)) for n in program.inputs}
    env.update({n: conv(params[n]) for n in program.params})
    for spec in program.kernels:
        outs = run_kernel(spec, env, dtype)
        if storage == "declared":
            outs = {t: v.to(_DT.get(program.tensors[t].dtype, dtype)).to(dtype) for t, v in outs.items()}
        env.update(outs)
    return env


def program_outputs(program, params, inputs, dtype=torch.float64, storage: str | None = None) -> list[torch.Tensor]:
    env = run_program(program, params, inputs, dtype, storage)
    shapes = program.metadata.get("output_shapes", {})
    return [env[o].reshape(shapes[o]) if o in shapes else env[o] for o in program.outputs]


def max_rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max|a-b| / (max|b| + 1e-6) (reference optimizer/evaluate.py:174-176)."""
    a, b = a.double(), b.double()
    return float((a - b).abs().max() / (b.abs().max() + 1e-6))
