"""Layout provenance: which base element does each element of a view read?

The reference answers this by replaying the chain of view/permute/expand/
slice nodes on a full ``arange`` index tensor (reference:
optimizer/layout.py:61-72). At the MI355X shapes that tensor is hundreds of
MiB, so here a chain is instead applied *backwards* to view coordinates:
each layout op maps an output coordinate to the input coordinate it reads,
and composing them maps any view coordinate to a flat base index. Checks
evaluate the map on every coordinate of a small view, or on a seeded sample
plus all corner coordinates of a large one.

``match_head_split`` recognises ``[T, H*d] -> [B, H, S, d]`` views and, new
here, their grouped-KV form where view head ``h`` reads base head
``h // (H / H_kv)`` (the unsqueeze/expand/reshape broadcast of K and V).
"""

from __future__ import annotations

import itertools
import math
from dataclasses import dataclass

import torch

from ..capture.opgraph import OpGraph, OpNode

TRACEABLE = ("view", "permute", "expand", "clone", "slice", "cast")
EXACT_LIMIT = 1 << 16
SAMPLES = 1 << 14


def _unravel(flat: torch.Tensor, shape: tuple[int, ...]) -> torch.Tensor:
    out = torch.empty(flat.shape[0], len(shape), dtype=torch.long)
    rem = flat.clone()
    for k in range(len(shape) - 1, -1, -1):
        out[:, k] = rem % shape[k]
        rem = rem // shape[k]
    return out


def _ravel(idx: torch.Tensor, shape: tuple[int, ...]) -> torch.Tensor:
    flat = torch.zeros(idx.shape[0], dtype=torch.long)
    for k, s in enumerate(shape):
        flat = flat * s + idx[:, k]
    return flat


def _out_shape(node: OpNode, in_shape: tuple[int, ...]) -> tuple[int, ...]:
    """Shape a layout op produces from ``in_shape`` (clone/cast pass it through,
    so a node whose input was rewritten to a new shape is still traced right)."""
    if node.op in ("view", "expand"):
        return tuple(int(s) for s in node.attrs["shape"])
    if node.op == "permute":
        return tuple(in_shape[d] for d in node.attrs["dims"])
    if node.op == "slice":
        shp = list(in_shape)
        shp[node.attrs["dim"]] = node.attrs["end"] - node.attrs["start"]
        return tuple(shp)
    return tuple(in_shape)


def _step_back(node: OpNode, idx: torch.Tensor, in_shape: tuple[int, ...], out_shape: tuple[int, ...]) -> torch.Tensor:
    """Coordinates in the input of ``node`` read by output coordinates ``idx``."""
    if node.op == "view":
        return _unravel(_ravel(idx, out_shape), in_shape)
    if node.op == "permute":
        res = torch.empty(idx.shape[0], len(in_shape), dtype=torch.long)
        res[:, node.attrs["dims"]] = idx
        return res
    if node.op == "expand":
        off = len(out_shape) - len(in_shape)
        res = idx[:, off:].clone()
        for k, s in enumerate(in_shape):
            if s == 1:
                res[:, k] = 0
        return res
    if node.op in ("clone", "cast"):
        return idx
    if node.op == "slice":
        res = idx.clone()
        res[:, node.attrs["dim"]] += node.attrs["start"]
        return res
    raise ValueError(f"{node.op} is not a traceable layout op")


@dataclass
class Provenance:
    base: str
    base_shape: tuple[int, ...]
    shape: tuple[int, ...]
    nodes: list[OpNode]          # base-first
    in_shapes: list[tuple[int, ...]]
    out_shapes: list[tuple[int, ...]]

    @property
    def chain(self) -> list[str]:
        return [n.name for n in self.nodes]

    @property
    def numel(self) -> int:
        return math.prod(self.shape) if self.shape else 1

    def points(self) -> torch.Tensor:
        """All view coordinates of a small view, else a seeded sample plus corners."""
        n = self.numel
        if n <= EXACT_LIMIT:
            return _unravel(torch.arange(n), self.shape)
        g = torch.Generator().manual_seed(1234)
        cols = [torch.randint(0, s, (SAMPLES,), generator=g) for s in self.shape]
        rnd = torch.stack(cols, 1) if cols else torch.zeros(SAMPLES, 0, dtype=torch.long)
        corners = torch.tensor(list(itertools.product(*[(0, s - 1) for s in self.shape])), dtype=torch.long)
        return torch.cat([rnd, corners.reshape(-1, len(self.shape))], 0)

    def base_index(self, idx: torch.Tensor) -> torch.Tensor:
        cur = idx
        for node, ish, osh in zip(reversed(self.nodes), reversed(self.in_shapes), reversed(self.out_shapes)):
            cur = _step_back(node, cur, ish, osh)
        return _ravel(cur, self.base_shape)

    def matches(self, fn) -> bool:
        """True when ``base_index == fn(coords)`` on the checked coordinates."""
        pts = self.points()
        return bool(torch.equal(self.base_index(pts), fn(pts)))

    def is_identity_reshape(self) -> bool:
        base_n = math.prod(self.base_shape) if self.base_shape else 1
        if self.numel != base_n:
            return False
        return self.matches(lambda p: _ravel(p, self.shape))

    def index_tensor(self) -> torch.Tensor:
        """Full base-index tensor of the view (small views only)."""
        return self.base_index(_unravel(torch.arange(self.numel), self.shape)).reshape(self.shape)


def trace_layout(graph: OpGraph, name: str, until: str | None = None) -> Provenance:
    """Provenance of ``name`` back to its first non-layout producer, or to the
    node ``until`` if the chain reaches it first."""
    chain: list[OpNode] = []
    cur = graph[name]
    while cur.kind == "layout" and cur.op in TRACEABLE and len(cur.inputs) == 1 and cur.name != until:
        chain.append(cur)
        cur = graph[cur.inputs[0]]
    chain.reverse()
    in_shapes, out_shapes = [], []
    shape = cur.type.shape
    for n in chain:
        in_shapes.append(shape)
        shape = _out_shape(n, shape)
        out_shapes.append(shape)
    return Provenance(cur.name, cur.type.shape, shape, chain, in_shapes, out_shapes)


def head_split_fn(batch: int, seq: int, heads: int, head_dim: int, kv_heads: int | None = None,
                  transpose_last: bool = False, merged: bool = False):
    """Base index of view coordinate for ``[T, Hkv*d]`` viewed as ``[B, H, S, d]``
    (``[B, H, d, S]`` when transposed, ``B*H`` merged when ``merged``)."""
    hk = heads if kv_heads is None else kv_heads
    grp = heads // hk

    def fn(p: torch.Tensor) -> torch.Tensor:
        if merged:
            bh = p[:, 0]
            b, h = bh // heads, bh % heads
            rest = p[:, 1:]
        else:
            b, h = p[:, 0], p[:, 1]
            rest = p[:, 2:]
        s, d = (rest[:, 1], rest[:, 0]) if transpose_last else (rest[:, 0], rest[:, 1])
        return ((b * seq + s) * hk + h // grp) * head_dim + d

    return fn


def head_merge_fn(batch: int, seq: int, heads: int, head_dim: int, view_shape: tuple[int, ...]):
    """Base index read by a view whose row-major order is token-major ``[T, H*d]``
    while its base is head-major ``[B, H, S, d]`` (or ``[B*H, S, d]``)."""

    def fn(p: torch.Tensor) -> torch.Tensor:
        flat = _ravel(p, view_shape)
        t, c = flat // (heads * head_dim), flat % (heads * head_dim)
        b, s = t // seq, t % seq
        h, d = c // head_dim, c % head_dim
        return ((b * heads + h) * seq + s) * head_dim + d

    return fn


def match_head_split(prov: Provenance, transpose_last: bool = False, allow_grouped: bool = False) -> dict | None:
    """``{batch, seq, heads, head_dim[, kv_heads]}`` if ``prov`` is a head-split
    view of a token-major base, else None."""
    shape = prov.shape
    base_n = math.prod(prov.base_shape) if prov.base_shape else 1
    if len(shape) == 4:
        b, h = shape[0], shape[1]
        s, d = (shape[3], shape[2]) if transpose_last else (shape[2], shape[3])
        cands = [(b, h, False)]
    elif len(shape) == 3:
        bh = shape[0]
        s, d = (shape[2], shape[1]) if transpose_last else (shape[1], shape[2])
        cands = [(bb, bh // bb, True) for bb in range(1, bh + 1) if bh % bb == 0]
    else:
        return None
    # a token-major base has B*S rows ([B*S, N], or [B, S, N]): with S = 1 a merged
    # [B*H, 1, d] view reads the same flat offsets for every split of B*H, so the
    # base's own row structure decides between them
    if len(prov.base_shape) >= 2:
        rows = math.prod(prov.base_shape[:-1])
        lead = prov.base_shape[0] if len(prov.base_shape) == 3 else None
        cands = [c for c in cands if c[0] * s == rows and (lead is None or c[0] == lead)] or cands
    for b, h, merged in cands:
        kv_opts = [h]
        if allow_grouped:
            kv_opts += [k for k in range(1, h) if h % k == 0]
        for hk in kv_opts:
            if b * s * hk * d != base_n:
                continue
            if prov.matches(head_split_fn(b, s, h, d, hk, transpose_last, merged)):
                out = {"batch": b, "seq": s, "heads": h, "head_dim": d}
                if hk != h:
                    out["kv_heads"] = hk
                return out
    return None


def is_head_merge(prov: Provenance, batch: int, seq: int, heads: int, head_dim: int) -> bool:
    """True when ``prov`` reads a head-major base in token-major ``[T, H*d]`` order."""
    n = batch * seq * heads * head_dim
    if prov.numel != n or math.prod(prov.base_shape) != n:
        return False
    return prov.matches(head_merge_fn(batch, seq, heads, head_dim, prov.shape))
