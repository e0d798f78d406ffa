"""Execute an OpIR Program on one MI355X through libth_hip.so.

The device twin of the reference's interpreter loop (codegen/interpret.py:54-77):
parameters are uploaded once (GEMM weights pre-packed into th_gemm's layout,
RoPE tables compressed back to [S, head_dim] after checking their structure),
intermediates get device buffers from a liveness-based pool (a buffer is
reused once the last kernel reading its tensor has run; memplan.py), and each
KernelSpec becomes one or two C-ABI launches on the current stream, in
program order. There is no host fallback: a kernel the library cannot run
raises :class:`HipBackendError` naming it.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Callable

import torch

from ..optimizer.opir import KernelSpec, Program
from . import abi, ops
from .epilogue import (EpiloguePlan, build_trees, is_rotated_copy, match_epilogue, match_rscale, periodic_table,
                       rope_geometry)

_TORCH_DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16,
             "int64": torch.int64, "int32": torch.int32, "float8_e4m3fn": torch.float8_e4m3fn}
_FP8 = torch.float8_e4m3fn


def _err(kernel: str, msg: str) -> abi.HipBackendError:
    return abi.HipBackendError("lower", abi.TH_ERR_UNSUPPORTED, msg, kernel)


@dataclass
class Launch:
    """One kernel of the program, bound to device buffers."""

    kernel: str
    kind: str
    run: Callable[[], None]
    entry: str
    info: dict[str, Any] = field(default_factory=dict)


def conv_merge_groups(program: Program, excluded: set[str] = frozenset()) -> list[list[str]]:
    """Groups (kernel names, program order) of depthwise conv1d kernels that feed one
    SSD kernel with the same (batch, seq, kernel, activation, dtypes): a Mamba-2
    layer's x, B and C convolutions (the reference convolves them as one xBC
    tensor, models/mamba.py:278-283; its partition splits them). A group runs as
    one th_conv1d_causal launch over the members' channels side by side: the
    GEMMs that produce the inputs write them as column windows of one
    [tokens, sum of widths] buffer and the SSD reads the outputs as column windows
    of another (GEMM outputs, the convolution and the SSD all take row strides).
    A member's input is a GEMM output read by nothing else, its output is read
    only by the SSD, neither is a program output nor in ``excluded`` (tensors
    with fp32 copies or cache slots), and its width is a multiple of 8 (every
    window starts 16-byte aligned); the SSD runs after the group's last member."""
    producer = {o.tensor: k for k in program.kernels for o in k.outputs}
    readers: dict[str, list[KernelSpec]] = {}
    for k in program.kernels:
        for a in k.args:
            readers.setdefault(a.tensor, []).append(k)
    index = {k.name: i for i, k in enumerate(program.kernels)}
    barred = set(program.outputs) | set(excluded)
    cands: dict[tuple, list[KernelSpec]] = {}
    for k in program.kernels:
        if k.kind != "conv1d" or k.epilogue or len(k.outputs) != 1 or k.outputs[0].value != "acc":
            continue
        x, y = k.arg("x").tensor, k.outputs[0].tensor
        tx, ty = program.tensors[x], program.tensors[y]
        pk, rx, ry = producer.get(x), readers.get(x, []), readers.get(y, [])
        if (pk is None or pk.kind != "gemm" or len(tx.shape) != 2 or tuple(tx.shape) != tuple(ty.shape)
                or int(tx.shape[1]) % 8 or {x, y} & barred or [r.name for r in rx] != [k.name]
                or len({r.name for r in ry}) != 1 or ry[0].kind not in ("ssd", "ssd_chunked")):
            continue
        a = k.attrs
        key = (a["batch"], a["seq"], a["kernel"], a.get("activation"), tx.dtype, ty.dtype, ry[0].name)
        cands.setdefault(key, []).append(k)
    groups = []
    for key, ms in cands.items():
        if len(ms) >= 2 and index[key[-1]] > max(index[k.name] for k in ms):
            groups.append([k.name for k in ms])
    return groups


class DeviceProgram:
    """A Program lowered and bound for execution on ``device``."""

    def __init__(self, program: Program, params: dict[str, torch.Tensor], device: int | torch.device = 0,
                 fuse_rope: bool = True, fp32_outputs: bool = True, residual_fp32: bool = True,
                 merge_siblings: bool | None = False,
                 fold_sources: dict[str, tuple[torch.Tensor, torch.Tensor]] | None = None,
                 reuse_buffers: bool = True, merge_convs: bool = True, hw=None) -> None:
        self.program = program
        # RMSNorm gains folded into weights by the front end, to be taken back
        # out (weight const -> (gain, unfolded weight)): such GEMMs read the
        # activations normalised WITH the gain by th_rmsnorm and the model's own
        # weights, so the gain never meets the weights in bf16
        self.fold_sources = fold_sources or {}
        self._normed: dict[tuple, torch.Tensor] = {}
        self.device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        if self.device.type != "cuda":
            raise abi.HipBackendError("DeviceProgram", abi.TH_ERR_INVALID, f"device {device} is not a HIP device")
        abi.init_device(self.device.index or 0)
        self.fuse_rope = fuse_rope
        self.buffers: dict[str, torch.Tensor] = {}
        self.workspaces: list[torch.Tensor] = []
        self.launches: list[Launch] = []
        self.graph: torch.cuda.CUDAGraph | None = None
        self.plans: dict[str, Any] = {}
        self._host_params = params
        for name in program.params:
            self.buffers[name] = params[name].to(self.device)
        for name in program.inputs:
            t = program.tensors[name]
            self.buffers[name] = torch.empty(t.shape, dtype=_TORCH_DT[t.dtype], device=self.device)
        # Residual operands produced inside the program get an fp32 shadow:
        # the producer also writes fp32 and every GEMM that adds it as an
        # epilogue operand reads the shadow, so the residual stream is rounded
        # to the activation dtype only where a GEMM consumes it as its LHS.
        # (The SSD's gate multiplies its output: it is read in its own dtype,
        # as the eager model does, and keeps the kernel's vector epilogue.)
        half = ("bfloat16", "float16")
        produced = {o.tensor for k in program.kernels for o in k.outputs}
        # a gathered table row is exact in the table's dtype: no shadow needed
        exact = {o.tensor for k in program.kernels if k.kind == "embedding" for o in k.outputs}
        shadowed: set[str] = set()
        for k in program.kernels:
            if k.kind != "gemm" or not residual_fp32:
                continue
            for a in k.args:
                if (a.role == "extra" and a.tensor in produced and a.tensor not in exact
                        and program.tensors[a.tensor].dtype in half):
                    shadowed.add(a.tensor)
        if fp32_outputs:
            # program outputs are also kept in fp32 (the epilogue computes them in
            # fp32; rounding to the declared dtype is only the storage step)
            shadowed |= {o for o in program.outputs
                         if o in produced and o not in exact and program.tensors[o].dtype in half}
        # decode programs: outputs the device writes straight into a cache input at
        # row ``pos`` of each sequence (the new token's key/value), kept in the cache's dtype
        self._slots = dict(program.metadata.get("cache_slots", {}))
        shadowed -= set(self._slots)
        self._shadowed = shadowed
        self.shadow: dict[str, torch.Tensor] = {}
        # depthwise convolutions feeding one SSD run as one launch (see _plan_conv_merges)
        self._conv_groups: dict[str, dict] = {}
        self._conv_member: dict[str, dict] = {}
        self._conv_window: dict[str, tuple[dict, str, int, int]] = {}
        if merge_convs:
            self._plan_conv_merges(program)
        # Intermediates (and shadows, workspaces, normalised operands) come from a
        # pool that recycles a buffer once the last kernel reading it has been
        # bound: kernels run in program order on one stream. Program outputs keep
        # buffers of their own. (A merged sibling launch writes its members'
        # outputs at the leader's position: they are bound there, each held to
        # its own last reader.)
        from .memplan import BufferPool, lifetimes

        self.reuse = reuse_buffers
        self._born, self._last = lifetimes(program)
        self._pool = BufferPool(lambda n: torch.empty(n, dtype=torch.uint8, device=self.device)) if self.reuse else None
        self._cur = 0
        if not self.reuse:
            for k in program.kernels:
                self._bind_outputs(k)
        # program inputs read as token ids, with the size of the table they index
        self._vocab: dict[str, int] = {}
        for k in program.kernels:
            if k.kind == "embedding" and k.arg("ids").tensor in program.inputs:
                ids = k.arg("ids").tensor
                self._vocab[ids] = min(self._vocab.get(ids, k.attrs["vocab"]), k.attrs["vocab"])
        # Sibling GEMM kernels (one lhs) as one launch: True merges every group that can
        # merge, False (this constructor's default) none; None (CompileConfig's default)
        # takes the planner's priced decision per group (optimizer/planner.py
        # price_launch_merges: separate launches against one launch of the concatenated
        # width, on the calibrated cost model of ``hw``, else the shipped hardware spec).
        self.launch_merges: list = []
        groups, away = self._plan_sibling_merges(program) if merge_siblings is not False else ({}, set())
        if merge_siblings is None and groups:
            from ..cost_models.hw_spec import HardwareSpec
            from ..optimizer.planner import price_launch_merges

            cand = [[(m[0].name, len(m[2])) for m in members] for members in groups.values()]
            self.launch_merges = price_launch_merges(program, cand, hw or HardwareSpec.load())
            keep = {lm.members[0] for lm in self.launch_merges if lm.merged}
            groups = {k: v for k, v in groups.items() if k in keep}
            away = {m[0].name for v in groups.values() for m in v[1:]}
        self._merge_groups, self._merged_away = groups, away
        # (e4m3 decode GEMMs: a few rows against weight streams, one launch always pays)
        self._fp8_groups = self._plan_fp8_merges(program, self._merged_away) if merge_siblings is not False else {}
        # scans whose only reader normalises them with a gain: the scan applies it (_plan_norm_folds)
        self._rs_parts: dict[tuple, torch.Tensor] = {}
        self._norm_folds = self._plan_norm_folds(program)
        # e4m3 GEMMs whose gained lhs the producing e4m3 GEMM stores (_plan_fp8_gain_folds)
        self._fp8_gain_folds = self._plan_fp8_gain_folds(program)
        self._fp8_gained: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}
        for i, k in enumerate(program.kernels):
            self._cur = i
            if self.reuse:
                self._pool.release_before(i)
                self._bind_outputs(k)
                for m in (self._merge_groups.get(k.name) or self._fp8_groups.get(k.name) or [])[1:]:
                    self._bind_outputs(m[0])
            if k.name in self._merged_away:
                continue
            if k.name in self._conv_groups:
                self.launches.append(self._lower_conv_group(self._conv_groups[k.name]))
                continue
            if k.name in self._conv_member:
                continue  # runs with its group, at the group's last member
            if k.name in self._merge_groups:
                self.launches.extend(self._lower_gemm_merged(self._merge_groups[k.name]))
            elif k.name in self._fp8_groups:
                members = [m[0] for m in self._fp8_groups[k.name]]
                merged = self._lower_fp8_merged(members)
                if merged is None:  # the parts disagree: each member at the leader's position
                    merged = [x for m in members for x in self._lower(m)]
                self.launches.extend(merged)
            else:
                self.launches.extend(self._lower(k))

    # ------------------------------------------------------------- memory
    def _device_buffer(self, shape, dtype: torch.dtype, last: int) -> torch.Tensor:
        """A tensor that nothing else uses through kernel ``last`` (pooled), or a fresh one."""
        numel = 1
        for s in shape:
            numel *= int(s)
        if self._pool is None or last >= len(self.program.kernels):
            return torch.empty(tuple(shape), dtype=dtype, device=self.device)
        nbytes = numel * torch.empty((), dtype=dtype).element_size()
        return self._pool.alloc(nbytes, last)[:nbytes].view(dtype).view(tuple(shape))

    def _bind_outputs(self, k: KernelSpec) -> None:
        """Buffers (and fp32 shadows) for the tensors kernel ``k`` produces."""
        for o in k.outputs:
            name = o.tensor
            if name in self.buffers:
                continue
            t = self.program.tensors[name]
            if name in self._conv_window:
                g, side, off, w = self._conv_window[name]
                if side not in g:  # the group's [tokens, sum of widths] buffer, for all its windows' lifetimes
                    last = g["pos"] if side == "x" else max(self._last.get(m.outputs[0].tensor, g["pos"])
                                                            for m in g["members"])
                    g[side] = self._device_buffer((g["rows"], g["width"]), _TORCH_DT[t.dtype], last)
                self.buffers[name] = g[side][:, off:off + w]
                continue
            if name in self._slots:
                self.buffers[name] = self._cache_row(name)
                continue
            last = self._last.get(name, self._cur)
            self.buffers[name] = self._device_buffer(t.shape, _TORCH_DT[t.dtype], last)
            if name in self._shadowed:
                self.shadow[name] = self._device_buffer(t.shape, torch.float32, last)

    def _plan_conv_merges(self, program: Program) -> None:
        """Bind the groups of conv_merge_groups: per group, the input and output
        tensors become column windows of two [tokens, sum of widths] buffers
        (allocated when the first window is bound)."""
        index = {k.name: i for i, k in enumerate(program.kernels)}
        kern = {k.name: k for k in program.kernels}
        for names in conv_merge_groups(program, self._shadowed | set(self._slots)):
            ms = [kern[n] for n in names]
            pos = max(index[n] for n in names)
            g = {"members": ms, "pos": pos, "rows": int(program.tensors[ms[0].arg("x").tensor].shape[0]), "width": 0}
            for k in ms:
                w = int(program.tensors[k.arg("x").tensor].shape[1])
                self._conv_window[k.arg("x").tensor] = (g, "x", g["width"], w)
                self._conv_window[k.outputs[0].tensor] = (g, "y", g["width"], w)
                self._conv_member[k.name] = g
                g["width"] += w
            self._conv_groups[program.kernels[pos].name] = g

    def _lower_conv_group(self, g: dict) -> Launch:
        """One th_conv1d_causal launch for a group of _plan_conv_merges."""
        ms = g["members"]
        ws = []
        for k in ms:
            host_w = self._host(k.arg("w").tensor)
            w = host_w if host_w is not None else self.buffers[k.arg("w").tensor]
            ws.append(w.float().reshape(int(self.program.tensors[k.arg("x").tensor].shape[1]), -1))
        w = torch.cat(ws, 0).contiguous().to(self.device)
        a = ms[0].attrs
        x, y, act = g["x"], g["y"], a.get("activation")
        name = "+".join(k.name for k in ms)

        def run() -> None:
            ops.conv1d_causal(x, w, y, batch=a["batch"], seq=a["seq"], activation=act, kernel=name)

        return Launch(name, "conv1d", run, "th_conv1d_causal",
                      {"activation": act, "merged": [k.name for k in ms], "width": g["width"]})

    def _cache_row(self, name: str) -> torch.Tensor:
        """Row ``pos`` of every sequence of the cache input a cache-slot output lives in:
        a [batch, width] view whose row stride is the cache's sequence stride."""
        slot, dec = self._slots[name], self.program.metadata["decode"]
        cache = self.buffers[slot["cache"]]
        b, L, pos = dec["batch"], dec["max_len"], slot["pos"]
        if not 0 <= pos < L or cache.shape[0] != b * L:
            raise _err(name, f"cache slot at pos {pos} outside the cache {tuple(cache.shape)} (batch {b}, max_len {L})")
        return cache.view(b, L, cache.shape[1])[:, pos]

    def memory_report(self) -> dict[str, int]:
        """Bytes of intermediate storage held, and what one buffer per tensor would hold."""
        if self._pool is None:
            return {"reuse": False}
        return {"reuse": True, "pool_bytes": self._pool.block_bytes, "without_reuse_bytes": self._pool.requested_bytes}

    # -------------------------------------------------------------- running
    def set_inputs(self, inputs: dict[str, torch.Tensor] | list[torch.Tensor] | tuple) -> None:
        if isinstance(inputs, (list, tuple)):
            inputs = dict(zip(self.program.inputs, inputs))
        for name in self.program.inputs:
            dst = self.buffers[name]
            src = inputs[name]
            if name in self._vocab and src.numel():
                lo, hi = int(src.min()), int(src.max())
                if lo < 0 or hi >= self._vocab[name]:
                    raise IndexError(f"input {name}: token id {lo if lo < 0 else hi} outside the embedding table "
                                     f"[0, {self._vocab[name]})")
            dst.copy_(src.reshape(dst.shape).to(dst.dtype), non_blocking=True)

    def launch_all(self) -> None:
        for l in self.launches:
            l.run()

    def capture(self) -> None:
        """Record the whole launch sequence into a HIP graph (torch.cuda.CUDAGraph).

        Every launch reads and writes the buffers bound at lowering time and
        allocates nothing, so the graph replays the program on whatever the
        input buffers hold at replay time (``set_inputs`` first). One eager run
        precedes the capture; nothing in the sequence records a memset."""
        with torch.cuda.device(self.device):
            torch.cuda.synchronize()
            self.launch_all()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.launch_all()
            torch.cuda.synchronize()
        self.graph = g

    def replay(self) -> None:
        """Run the captured graph on the current stream (``capture`` first)."""
        if self.graph is None:
            raise abi.HipBackendError("replay", abi.TH_ERR_INVALID, "no graph captured; call capture() first")
        self.graph.replay()

    def run(self, inputs=None) -> list[torch.Tensor]:
        """Run the program; returns the program outputs (device tensors)."""
        if inputs is not None:
            self.set_inputs(inputs)
        if self.graph is not None:
            self.replay()
        else:
            self.launch_all()
        return self.outputs()

    def outputs(self, fp32: bool = False) -> list[torch.Tensor]:
        """Program outputs in their declared dtype, or (``fp32=True``) their fp32
        copies where the producing kernel wrote one."""
        shapes = self.program.metadata.get("output_shapes", {})
        res = []
        for o in self.program.outputs:
            t = self.shadow[o] if fp32 and o in self.shadow else self.buffers[o]
            res.append(t.reshape(shapes[o]) if o in shapes else t)
        return res

    def tensor(self, name: str) -> torch.Tensor:
        return self.buffers[name]

    def operand(self, name: str) -> torch.Tensor:
        """Buffer an epilogue reads for ``name`` (its fp32 shadow if it has one)."""
        return self.shadow.get(name, self.buffers[name])

    # ------------------------------------------------------------- lowering
    def _dt(self, name: str) -> torch.dtype:
        return _TORCH_DT[self.program.tensors[name].dtype]

    def _host(self, name: str) -> torch.Tensor | None:
        return self._host_params.get(name) if name in self.program.params else None

    def _workspace(self, numel: int, dtype=torch.float32) -> torch.Tensor:
        """Scratch memory of the kernel being lowered (free again for the next kernel)."""
        w = self._device_buffer((numel,), dtype, self._cur)
        self.workspaces.append(w)
        return w

    def _lower(self, spec: KernelSpec) -> list[Launch]:
        if spec.kind == "gemm":
            return self._lower_gemm(spec)
        if spec.kind == "attention":
            return [self._lower_attention(spec)]
        if spec.kind == "attention_decode":
            return [self._lower_attention_decode(spec)]
        if spec.kind in ("ssd", "ssd_chunked"):
            from .ssd import lower_ssd
            return lower_ssd(self, spec)
        if spec.kind == "conv1d":
            from .ssd import lower_conv1d
            return lower_conv1d(self, spec)
        if spec.kind == "embedding":
            return [self._lower_embedding(spec)]
        raise _err(spec.name, f"kernel kind {spec.kind!r} has no HIP kernel")

    # embedding ------------------------------------------------------------
    def _lower_embedding(self, spec: KernelSpec) -> Launch:
        table = self.buffers[spec.arg("table").tensor]
        ids = self.buffers[spec.arg("ids").tensor]
        if table.dtype not in (torch.bfloat16, torch.float32):
            raise _err(spec.name, f"embedding table dtype {table.dtype} has no kernel")
        out = self.buffers[spec.outputs[0].tensor]
        out32 = self.shadow.get(spec.outputs[0].tensor)
        ids_flat = ids.reshape(-1)

        def run() -> None:
            ops.embedding(table, ids_flat, out, out32=out32, kernel=spec.name)

        return Launch(spec.name, "embedding", run, "th_embedding", {"vocab": table.shape[0], "dim": table.shape[1]})

    # attention ------------------------------------------------------------
    def _lower_attention(self, spec: KernelSpec) -> Launch:
        a = spec.attrs
        q, k, v = (self.buffers[spec.arg(r).tensor] for r in ("q", "k", "v"))
        out = self.buffers[spec.outputs[0].tensor]
        kw = dict(batch=a["batch"], seq_q=a["seq"], seq_kv=a.get("seq_kv", a["seq"]), heads_q=a["heads"],
                  heads_kv=a.get("kv_heads", a["heads"]), head_dim=a["head_dim"], scale=float(a["scale"]),
                  causal=bool(a.get("causal", False)))

        def run() -> None:
            ops.attention_prefill(q, k, v, out, kernel=spec.name, **kw)

        return Launch(spec.name, "attention", run, "th_attention_prefill", kw)

    def _lower_attention_decode(self, spec: KernelSpec) -> Launch:
        """Keys/values 0..pos-1 from the caches and the new token's at pos: the new key and
        value must be cache-slot outputs (written into the caches at row pos by their
        producer), so one th_attention_decode over rows 0..pos reads them all."""
        a = spec.attrs
        b, L, pos, hk, hd = a["batch"], a["max_len"], a["pos"], a["kv_heads"], a["head_dim"]
        caches = []
        for new, cache in (("k_new", "k_cache"), ("v_new", "v_cache")):
            t_new, t_cache = spec.arg(new).tensor, spec.arg(cache).tensor
            slot = self._slots.get(t_new)
            if slot is None or slot["cache"] != t_cache or slot["pos"] != pos:
                raise _err(spec.name, f"{new} ({t_new}) is not written into {t_cache} at row {pos}: "
                                      "attention_decode needs the program's cache_slots")
            caches.append(self.buffers[t_cache].view(b, L, hk, hd))
        q = self.buffers[spec.arg("q").tensor]
        out = self.buffers[spec.outputs[0].tensor]
        ws_bytes = ops.attention_decode_workspace_bytes(b, a["heads"], hk, hd, L)
        ws = self._workspace(max(ws_bytes // 4, 1))
        kw = dict(scale=float(a["scale"]), fixed_len=pos + 1)

        def run() -> None:
            ops.attention_decode(q, caches[0], caches[1], out, workspace=ws, kernel=spec.name, **kw)

        return Launch(spec.name, "attention_decode", run, "th_attention_decode",
                      {"batch": b, "heads_q": a["heads"], "heads_kv": hk, "head_dim": hd, "keys": pos + 1})

    # gemm -----------------------------------------------------------------
    def _pack(self, spec: KernelSpec, rhs_args: list[str], in_dtype: torch.dtype,
              unfold: bool = False) -> Callable[[], torch.Tensor]:
        """Packed rhs for these weight arguments: packed once if all are params,
        else re-packed into a workspace at every run. ``unfold``: the weights the
        front end folded a norm gain into, taken without the gain."""
        tens = [spec.arg(r).tensor for r in rhs_args]
        if unfold:
            srcs = [self.fold_sources[t][1].to(self.device) for t in tens]
            packed = ops.pack_rhs([x if x.dtype in (torch.float32, torch.bfloat16) else x.float() for x in srcs],
                                  in_dtype)
            return lambda: packed
        srcs = [self.buffers[t] for t in tens]
        if in_dtype == _FP8:
            if not all(t in self.program.params and s.dtype == _FP8 for t, s in zip(tens, srcs)):
                raise _err(spec.name, "e4m3 products need e4m3 parameter weights")
            packed = ops.pack_rhs(srcs, _FP8)
            return lambda: packed
        if all(t in self.program.params for t in tens):
            srcs = [s if s.dtype in (torch.float32, torch.bfloat16) else s.float() for s in srcs]
            if in_dtype == torch.float32:
                srcs = [s.float() for s in srcs]
            packed = ops.pack_rhs(srcs, in_dtype)
            return lambda: packed
        k_, n_ = srcs[0].shape
        nbytes = abi.load().th_gemm_packed_bytes(n_, k_, len(srcs), ops.th_dtype(in_dtype))
        ws = self._workspace(int(nbytes), torch.uint8)
        return lambda: ops.pack_rhs(srcs, in_dtype, out=ws)

    def _lower_gemm(self, spec: KernelSpec) -> list[Launch]:
        lhs = self.buffers[spec.arg("lhs").tensor]
        T, N, K = spec.grid["rows"], spec.grid["cols"], spec.k_extent
        if lhs.dtype not in (torch.bfloat16, torch.float32):
            raise _err(spec.name, f"lhs dtype {lhs.dtype} has no MFMA GEMM in this build")
        if not spec.gemms:
            norm = self._lower_norm(spec)
            if norm is not None:
                return [norm]
            return self._lower_gemm_vm(spec)
        plan = match_epilogue(spec)
        if plan.fused:
            launches = self._lower_gemm_fused(spec, plan)
            if launches is not None:
                return launches
        return self._lower_gemm_vm(spec)

    def _lower_norm(self, spec: KernelSpec) -> Launch | None:
        """gemms=[] + sumsq kernels of the form (x * r) * gain_full -> th_rmsnorm."""
        trees = build_trees(spec)
        if len(spec.outputs) != 1:
            return None
        e = trees[spec.outputs[0].value]
        lhs_tensor = spec.arg("lhs").tensor
        if not (len(e) == 4 and e[0] == "mul" and not dict(e[1])):
            return None
        for inner, gain in ((e[2], e[3]), (e[3], e[2])):
            if gain[0] != "extra" or not (len(inner) == 4 and inner[0] == "mul"):
                continue
            for x, r in ((inner[2], inner[3]), (inner[3], inner[2])):
                rs = match_rscale(r)
                if rs is None or x[0] != "extra" or spec.arg(x[1]).tensor != lhs_tensor:
                    continue
                gt = spec.arg(gain[1]).tensor
                host = self._host(gt)
                if host is None:
                    continue
                row = periodic_table(host.float(), 1, host.shape[1])
                if row is None:
                    continue
                gvec = row.reshape(-1).to(self.device).contiguous()
                xbuf = self.buffers[lhs_tensor]
                out = self.buffers[spec.outputs[0].tensor]
                out32 = self.shadow.get(spec.outputs[0].tensor)
                inv_k, eps = rs

                def run() -> None:
                    ops.rmsnorm(xbuf, gvec, eps, out, inv_k=inv_k, kernel=spec.name, out32=out32)

                return Launch(spec.name, "rmsnorm", run, "th_rmsnorm", {"inv_k": inv_k, "eps": eps})
        return None

    def _lower_gemm_fused(self, spec: KernelSpec, plan: EpiloguePlan, collect: list | None = None) -> list[Launch] | None:
        """The fused th_gemm launch of this kernel (None: the epilogue needs the VM).
        ``collect``: append the call's parts there instead (for a merged launch)."""
        T, N, K = spec.grid["rows"], spec.grid["cols"], spec.k_extent
        lhs_t = spec.arg("lhs").tensor
        lhs = self.buffers[lhs_t]
        rhs_of = {i: g.rhs for i, g in enumerate(spec.gemms)}
        # e4m3 weights (decode programs): bf16 lhs x e4m3 rhs with per-column scales
        fp8 = [self.program.tensors[spec.arg(g.rhs).tensor].dtype == "float8_e4m3fn" for g in spec.gemms]
        if any(fp8) and not all(fp8):
            raise _err(spec.name, "a kernel mixes e4m3 and higher-precision weights")
        fp8 = all(fp8)
        if fp8 and lhs.dtype != torch.bfloat16:
            raise _err(spec.name, "e4m3 weights need a bf16 lhs")
        in_dtype = _FP8 if fp8 else lhs.dtype
        outs = []
        rope_tables: dict[tuple[str, str], tuple[torch.Tensor, torch.Tensor, int, int]] = {}
        for o in plan.outs:
            op, a, b = o.op, o.a, o.b
            if op == abi.EPI_ROPE_PAIR:
                cos_t, sin_t = (spec.arg(x).tensor for x in o.rope)
                hc, hs = self._host(cos_t), self._host(sin_t)
                if hc is None or hs is None:
                    return None
                key = (cos_t, sin_t)
                geo = rope_geometry(hc.float(), hs.float())
                if geo is None:
                    return None
                rp, period = geo
                wa, wb = self._host(spec.arg(rhs_of[a]).tensor), self._host(spec.arg(rhs_of[b]).tensor)
                if fp8 and wa is not None and wb is not None:
                    # compare the dequantised weights: values and scales are both rotated
                    wa, wb = (self._host(spec.arg(rhs_of[i]).tensor).float()
                              * self._host(spec.arg(rhs_of[i] + "_scale").tensor).float()[None, :] for i in (a, b))
                # the tables repeat every half head (cos = cat(f, f)), so the head
                # dim is the multiple of their period for which w_b is w_a rotated
                hd, fused = period, False
                if self.fuse_rope and wa is not None and wb is not None:
                    cand = period
                    while cand <= N and N % cand == 0:
                        if is_rotated_copy(wa.float(), wb.float(), cand):
                            hd, fused = cand, True
                            break
                        cand *= 2
                if key in rope_tables and rope_tables[key][3] != hd:
                    return None
                if key not in rope_tables:
                    ct = periodic_table(hc.float(), rp, hd).to(self.device)
                    st = periodic_table(hs.float(), rp, hd).to(self.device)
                    rope_tables[key] = (ct, st, rp, hd)
                outs.append((o, abi.EPI_ROPE, a, -1, key) if fused else (o, abi.EPI_ROPE_PAIR, a, b, key))
            else:
                outs.append((o, op, a, b, None))
        if len(rope_tables) > 1:
            return None
        used: list[int] = []
        for _, op, a, b, _ in outs:
            for i in (a, b):
                if i >= 0 and i not in used:
                    used.append(i)
        used.sort()
        if any(op == abi.EPI_ROPE for _, op, *_ in outs) and not fp8:
            # (e4m3 products rotate in the split reduction, which reads any column)
            bn = abi.load().th_gemm_acc_tile(N, min(len(used), abi.MAX_ACC), ops.th_dtype(in_dtype))
            hd = next(iter(rope_tables.values()))[3]
            if bn % hd:
                # the column tile cannot hold whole heads: keep the rotated accumulators
                outs = [(o, abi.EPI_ROPE_PAIR if op == abi.EPI_ROPE else op, a, o.b if op == abi.EPI_ROPE else b, key)
                        for (o, op, a, b, key) in outs]
                used = sorted({i for _, _, a, b, _ in outs for i in (a, b) if i >= 0})
        if len(used) > abi.MAX_ACC:
            return None
        slot = {i: s for s, i in enumerate(used)}
        extras: list[str] = []
        for o, *_ in outs:
            if o.extra is not None and o.extra not in extras:
                extras.append(o.extra)
        if len(extras) > abi.MAX_EXTRA:
            return None
        norm_launch, normed, rs_parts = None, None, None
        gain = self._unfold_gain(spec, plan, used)
        if gain is not None:
            # (collect mode only asks: the shared buffer is registered when a launch is made)
            norm_launch, normed = self._normed_lhs(spec, lhs_t, gain, plan.rscale, register=collect is None)
            lhs = normed
            # (the producing scan applied the gain and left the row sums: _plan_norm_folds)
            rs_parts = self._rs_parts.get(self._norm_key(lhs_t, gain, plan.rscale))
        # (a merged launch packs its own concatenated weights)
        get_packed = self._pack(spec, [rhs_of[i] for i in used], in_dtype, unfold=gain is not None) \
            if collect is None else None
        extra_bufs = [self.operand(spec.arg(x).tensor) for x in extras]
        epi = []
        for o, op, a, b, key in outs:
            dsts = [self.buffers[o.tensor]] + ([self.shadow[o.tensor]] if o.tensor in self.shadow else [])
            for out_buf in dsts:
                epi.append(ops.EpiSpec(op, out_buf, a=slot[a], b=slot[b] if b >= 0 else -1,
                                       e=extras.index(o.extra) if o.extra is not None else -1))
        gain_out = None
        fold = self._fp8_gain_folds.get(spec.name) if fp8 and collect is None else None
        if fold is not None:
            # the consumer's operand: this output again, times its norm gain, with the row sums
            g = next(k for k in self.program.kernels if k.name == fold["consumer"])
            o, op, a, b, _ = next(x for x in outs if x[0].tensor == fold["tensor"])
            last = self._last.get(fold["tensor"], self._cur)
            xg = self._device_buffer((T, N), torch.bfloat16, last)
            parts = self._device_buffer((T, N // 256), torch.float32, last)
            gvec = self.buffers[g.arg("gain").tensor].float().reshape(-1).contiguous()
            epi.append(ops.EpiSpec(op, xg, a=slot[a], b=slot[b] if b >= 0 else -1,
                                   e=extras.index(o.extra) if o.extra is not None else -1))
            gain_out = (len(epi) - 1, gvec, parts)
            self._fp8_gained[fold["consumer"]] = (xg, parts)
        if len(epi) > abi.MAX_OUT:
            return None
        mask = 0
        for i in used:
            if plan.scaled.get(i, False):
                mask |= 1 << slot[i]
        inv_k, eps = plan.rscale if plan.rscale else (0.0, 0.0)
        sumsq = plan.rscale is not None
        if normed is not None and rs_parts is None:   # the row scale is inside the normalised lhs
            mask, sumsq = 0, False
        rope = next(iter(rope_tables.values())) if rope_tables else None
        info = {"n_acc": len(used), "ops": [op for _, op, *_ in outs], "rscale": plan.rscale is not None,
                "rope_fused": any(op == abi.EPI_ROPE for _, op, *_ in outs), "gain_on_activation": normed is not None}
        if rs_parts is not None:
            info["row_sums_from_producer"] = True
        fp8_kw: dict[str, Any] = {}
        if in_dtype == torch.float32 and collect is None:
            # small fp32 grids split K over workgroups through a workspace (0 bytes otherwise)
            nb = ops.gemm_workspace_bytes(T, N, K, len(used), torch.float32)
            if nb > 0:
                fp8_kw["workspace"] = self._workspace(nb, torch.uint8)
        if fp8:
            scale_t = [rhs_of[i] + "_scale" for i in used]
            names = {x.name for x in spec.args}
            if any(x not in names for x in scale_t):
                raise _err(spec.name, "e4m3 weights without their <rhs>_scale arguments")
            scale = torch.stack([self.buffers[spec.arg(x).tensor].float().reshape(-1) for x in scale_t]).contiguous()
            ws = self._workspace(max(ops.gemm_workspace_bytes(T, N, K, len(used), _FP8), 16), torch.uint8) \
                if collect is None else None
            fp8_kw = dict(in_dtype=_FP8, rhs_scale=scale, workspace=ws)
            gained = self._fp8_gained.get(spec.name) if collect is None else None
            if gained is not None:
                # the producer stored lhs * g and the rows' sums of squares (_plan_fp8_gain_folds)
                lhs, rs_parts = gained
                info["row_sums_from_producer"] = True
            elif "gain" in names:
                # activation-side norm gain: the products see lhs * g, the sum of squares lhs
                fp8_kw["lhs_gain"] = self.buffers[spec.arg("gain").tensor].float().reshape(-1).contiguous()
            if gain_out is not None:
                fp8_kw["gain_out"] = gain_out
                info["gain_out_for"] = self._fp8_gain_folds[spec.name]["consumer"]
            info.update({"weights": "float8_e4m3fn", "lhs_gain": "gain" in names and gained is None})

        if collect is not None:
            collect.append(dict(T=T, N=N, K=K, lhs=lhs, fp8=fp8, rhs=[spec.arg(rhs_of[i]).tensor for i in used],
                                scales=[spec.arg(rhs_of[i] + "_scale").tensor for i in used] if fp8 else [],
                                epi=epi, mask=mask, n_used=len(used), sumsq=sumsq, inv_k=inv_k, eps=eps, rope=rope,
                                extras=extra_bufs, lhs_gain=fp8_kw.get("lhs_gain"), norm=norm_launch, info=info))
            return []

        def run() -> None:
            call = ops.GemmCall(T, N, K, len(used), lhs, get_packed(), epi, sumsq=sumsq,
                                rscale_mask=mask, inv_k=inv_k, eps=eps, extras=extra_bufs, rs_parts=rs_parts, **fp8_kw)
            if rope is not None:
                call.rope_cos, call.rope_sin, call.rope_period, call.rope_head_dim = rope[0], rope[1], rope[2], rope[3]
            ops.gemm(call, kernel=spec.name)

        self.plans[spec.name] = info
        launches = [Launch(spec.name, "gemm", run, "th_gemm", info)]
        return [norm_launch] + launches if norm_launch is not None else launches

    def _unfold_gain(self, spec: KernelSpec, plan: EpiloguePlan, used: list[int]) -> torch.Tensor | None:
        """The norm gain to take back out of this kernel's weights: every used weight is
        a fold of the same gain, every used accumulator carries the row scale, and the
        lhs is bf16. None otherwise (the kernel then runs as folded)."""
        if not self.fold_sources or plan.rscale is None or not used:
            return None
        # (the declared dtype: the merge planner asks before buffers are bound)
        if self.program.tensors[spec.arg("lhs").tensor].dtype != "bfloat16":
            return None
        tens = [spec.arg(spec.gemms[i].rhs).tensor for i in used]
        # e4m3 weights are quantised from the model's own weights and carry their gain
        # as a ``gain`` argument: there is nothing to take back out of them
        if any(self.program.tensors[t].dtype == "float8_e4m3fn" for t in tens):
            return None
        if any(t not in self.fold_sources for t in tens) or not all(plan.scaled.get(i, False) for i in used):
            return None
        g0 = self.fold_sources[tens[0]][0]
        if any(not torch.equal(self.fold_sources[t][0], g0) for t in tens[1:]):
            return None
        return g0

    @staticmethod
    def _norm_key(lhs_t: str, gain: torch.Tensor, rscale) -> tuple:
        """The normalised operand of ``lhs_t`` with this gain and row scale (shared by the
        kernels that read it)."""
        return (lhs_t, gain.data_ptr(), float(rscale[0]), float(rscale[1]))

    def _plan_norm_folds(self, program: Program) -> dict[str, dict]:
        """SSD scans whose output is read by exactly one GEMM, as its lhs, normalised with
        an RMSNorm gain taken back out of that GEMM's weights (norm_gain='activation': the
        gated norm before Mamba's out-projection). Such a scan stores y times the gain and
        the sums of squares of y per token and 32 columns (th_ssd_chunked's y_gain and
        rs_parts); the GEMM applies the row scale from those sums (th_gemm's rs_parts), and
        the th_rmsnorm launch between them goes away. Only where the scan runs its MFMA
        path with the vector epilogue (bf16 operands and output, no fp32 copy of the
        output, which no other kernel and no program output reads). Returns
        {scan kernel: {"gemm", "gain", "key", "tensor"}}."""
        from .ssd import _gate_of

        folds: dict[str, dict] = {}
        if not self.fold_sources:
            return folds
        readers: dict[str, list] = {}
        for k in program.kernels:
            for a in k.args:
                readers.setdefault(a.tensor, []).append((k, a))
        for k in program.kernels:
            if k.kind != "ssd_chunked" or len(k.outputs) != 1 or not _gate_of(k)[1]:
                continue
            t, at = k.outputs[0].tensor, k.attrs
            H, P, N = at["heads"], at["head_dim"], at["state_dim"]
            bf16 = all(program.tensors[k.arg(r).tensor].dtype == "bfloat16" for r in ("x", "b", "c", "dt"))
            if (t in program.outputs or t in self._shadowed or program.tensors[t].dtype != "bfloat16" or not bf16
                    or P not in (32, 64, 128) or N not in (32, 64, 128) or int(at.get("chunk", 64)) % 32
                    or (H * P) % 128):
                continue
            rd = readers.get(t, [])
            if len(rd) != 1 or rd[0][0].kind != "gemm" or rd[0][1].role != "lhs" or not rd[0][0].gemms:
                continue
            g = rd[0][0]
            if g.name in self._merge_groups or g.name in self._merged_away or g.name in self._fp8_groups:
                continue
            plan = match_epilogue(g)
            if not plan.fused or plan.rscale is None or any(o.rope is not None for o in plan.outs):
                continue
            used = sorted({i for o in plan.outs for i in (o.a, o.b) if i >= 0})
            gain = self._unfold_gain(g, plan, used)
            if gain is None or gain.numel() != H * P:
                continue
            folds[k.name] = {"gemm": g.name, "gain": gain, "key": self._norm_key(t, gain, plan.rscale), "tensor": t}
        return folds

    def _plan_fp8_gain_folds(self, program: Program) -> dict[str, dict]:
        """e4m3 GEMMs with an activation-side norm gain (a ``gain`` argument) whose lhs is a
        bf16 output, over all its columns, of another e4m3 GEMM: the decode step's gate/up
        reading the o-projection's x1. The producer's finishing pass also stores x1 with the
        gain applied and its rows' sums of squares (th_gemm's gain_out), and the consumer
        multiplies that copy, taking the sums as its rs_parts, instead of scaling x1 in a
        pre-pass of its own. Neither kernel may be part of a merged launch; the producer's
        width must be a multiple of 1024 and it must run through its split reduction with
        4-column outputs (whole 128-column packed tiles, K a multiple of 128).
        Returns {producer kernel: {"consumer", "tensor"}}."""
        folds: dict[str, dict] = {}
        writer: dict[str, KernelSpec] = {}
        for k in program.kernels:
            for o in k.outputs:
                writer[o.tensor] = k

        def e4m3(k: KernelSpec) -> bool:
            return k.kind == "gemm" and bool(k.gemms) and all(
                program.tensors[k.arg(g.rhs).tensor].dtype == "float8_e4m3fn" for g in k.gemms)

        def alone(k: KernelSpec) -> bool:
            return k.name not in self._merge_groups and k.name not in self._merged_away and not any(
                k.name == m[0].name for v in self._fp8_groups.values() for m in v)

        taken: set[str] = set()
        for g in program.kernels:
            if not e4m3(g) or "gain" not in {a.name for a in g.args} or not alone(g):
                continue
            t = g.arg("lhs").tensor
            pk = writer.get(t)
            if pk is None or pk.name in taken or not e4m3(pk) or not alone(pk) or program.tensors[t].dtype != "bfloat16":
                continue
            N, K = pk.grid["cols"], pk.k_extent
            if N % 1024 or K % 128 or g.grid["cols"] <= 0:
                continue
            pp, pg = match_epilogue(pk), match_epilogue(g)
            if not pp.fused or not pg.fused or pg.rscale is None or any(o.rope is not None for o in pp.outs):
                continue
            if sum(1 for o in pp.outs if o.tensor == t) != 1:
                continue
            folds[pk.name] = {"consumer": g.name, "tensor": t}
            taken.add(pk.name)
        return folds

    def _normed_lhs(self, spec: KernelSpec, lhs_t: str, gain: torch.Tensor, rscale,
                    register: bool = True) -> tuple[Launch | None, torch.Tensor]:
        """bf16 ``x * r * g`` of this lhs (x read from its fp32 shadow when it has one),
        made by one th_rmsnorm launch before the first kernel that needs it and shared
        by the later ones (sibling projections of the same normalised input).
        ``register=False``: a probe (collect mode) whose launch may never be emitted,
        so later kernels must not take the buffer as already written."""
        inv_k, eps = rscale
        key = self._norm_key(lhs_t, gain, rscale)
        if key in self._normed:
            return None, self._normed[key]
        x = self.operand(lhs_t)
        # read only by kernels that read the lhs: the lhs's lifetime bounds it
        out = self._device_buffer(x.shape, torch.bfloat16, self._last.get(lhs_t, self._cur))
        gvec = gain.float().reshape(-1).to(self.device).contiguous()
        if register:
            self._normed[key] = out

        def run() -> None:
            ops.rmsnorm(x, gvec, eps, out, inv_k=inv_k, kernel=f"{spec.name} (normalised lhs)")

        # (a launch of the kernel that first needs it: its time counts with that kernel's)
        return Launch(spec.name, "gemm", run, "th_rmsnorm", {"inv_k": inv_k, "eps": eps, "normalised_lhs": True}), out

    # sibling merge --------------------------------------------------------
    # GEMM kernels that multiply the same lhs by weights (projections of one
    # input that the partition kept apart because their widths or epilogue ops
    # differ) run as ONE th_gemm: the used weight columns of every kernel are
    # concatenated into one accumulator, and each output keeps its op on its own
    # column window. One launch reads the lhs once and fills the GPU with the
    # sum of the widths instead of several small grids.
    _MERGE_OPS = (abi.EPI_ACC, abi.EPI_SILU, abi.EPI_ADD, abi.EPI_SOFTPLUS_ADD, abi.EPI_MUL)

    def _merge_key(self, k: KernelSpec):
        if k.kind != "gemm" or not k.gemms:
            return None
        lhs_t = k.arg("lhs").tensor
        if self.program.tensors[lhs_t].dtype != "bfloat16" or k.grid["cols"] % 8:
            return None
        plan = match_epilogue(k)
        if not plan.fused or not plan.outs:
            return None
        if any(o.op not in self._MERGE_OPS or o.rope is not None or o.b >= 0 for o in plan.outs):
            return None
        used = sorted({o.a for o in plan.outs})
        if any(k.arg(k.gemms[a].rhs).tensor not in self.program.params for a in used):
            return None
        # A weight with its norm gain folded in runs on the normalised activations
        # and the unfolded weight (_lower_gemm_fused): such kernels merge only with
        # kernels that unfold the same gain, and the merged launch does the same.
        unfold = None
        if any(k.arg(k.gemms[a].rhs).tensor in self.fold_sources for a in used):
            g = self._unfold_gain(k, plan, used)
            if g is None:
                return None
            unfold = g.data_ptr()
        flags = {bool(plan.scaled.get(a, False)) for a in used}
        if len(flags) != 1:
            return None
        return (lhs_t, k.k_extent, plan.rscale, flags.pop(), unfold), plan, used

    def _plan_sibling_merges(self, program: Program):
        """Leader kernel name -> [(spec, plan, used accumulators)] in launch
        order; the other members launch with their leader (they read only the
        shared lhs, parameters and tensors ready before the leader)."""
        produced_at = {o.tensor: i for i, k in enumerate(program.kernels) for o in k.outputs}
        keyed = [(i, k, self._merge_key(k)) for i, k in enumerate(program.kernels)]
        groups: dict[str, list] = {}
        away: set[str] = set()
        for i, k, m in keyed:
            if m is None or k.name in away:
                continue
            key, plan, used = m
            members = [(k, plan, used)]
            n_out = sum(1 + (o.tensor in self._shadowed) for o in plan.outs)
            extras = {k.arg(o.extra).tensor for o in plan.outs if o.extra is not None}
            for j, k2, m2 in keyed[i + 1:]:
                if m2 is None or k2.name in away or m2[0] != key:
                    continue
                _, plan2, used2 = m2
                ext2 = {k2.arg(o.extra).tensor for o in plan2.outs if o.extra is not None}
                ready = all(t in program.params or produced_at.get(t, len(program.kernels)) < i for t in ext2)
                n2 = n_out + sum(1 + (o.tensor in self._shadowed) for o in plan2.outs)
                if not ready or n2 > abi.MAX_OUT or len(extras | ext2) > abi.MAX_EXTRA:
                    continue
                members.append((k2, plan2, used2))
                n_out, extras = n2, extras | ext2
            if len(members) > 1:
                groups[k.name] = members
                away.update(m[0].name for m in members[1:])
        return groups, away

    def _lower_gemm_merged(self, members) -> list[Launch]:
        lead = members[0][0]
        lhs_t = lead.arg("lhs").tensor
        lhs = self.buffers[lhs_t]
        T, K = lead.grid["rows"], lead.k_extent
        plan0 = members[0][1]
        # (every member unfolds the same gain, or none does: it is part of the merge key)
        gain = self._unfold_gain(lead, plan0, members[0][2])
        norm_launch = None
        if gain is not None:
            norm_launch, lhs = self._normed_lhs(lead, lhs_t, gain, plan0.rscale)
        cols: dict[tuple[str, int], tuple[int, int]] = {}
        weights: list[torch.Tensor] = []
        n_tot = 0
        for spec, plan, used in members:
            n = spec.grid["cols"]
            for a in used:
                t = spec.arg(spec.gemms[a].rhs).tensor
                w = self.fold_sources[t][1].to(self.device) if gain is not None else self.buffers[t]
                weights.append(w if w.dtype in (torch.float32, torch.bfloat16) else w.float())
                cols[(spec.name, a)] = (n_tot, n_tot + n)
                n_tot += n
        packed = ops.pack_rhs([torch.cat([w.float() for w in weights], dim=1).contiguous()], torch.bfloat16)
        extras: list[str] = []
        epi = []
        for spec, plan, _ in members:
            for o in plan.outs:
                e = -1
                if o.extra is not None:
                    t = spec.arg(o.extra).tensor
                    if t not in extras:
                        extras.append(t)
                    e = extras.index(t)
                for buf in [self.buffers[o.tensor]] + ([self.shadow[o.tensor]] if o.tensor in self.shadow else []):
                    epi.append(ops.EpiSpec(o.op, buf, a=0, e=e, cols=cols[(spec.name, o.a)]))
        extra_bufs = [self.operand(t) for t in extras]
        scaled = bool(plan0.scaled.get(members[0][2][0], False))
        inv_k, eps = plan0.rscale if plan0.rscale else (0.0, 0.0)
        sumsq = plan0.rscale is not None
        if gain is not None:  # the row scale is inside the normalised lhs
            scaled, sumsq = False, False
        names = [m[0].name for m in members]
        info = {"n_acc": 1, "merged": names, "cols": n_tot, "ops": [x.op for x in epi], "rscale": plan0.rscale is not None,
                "rope_fused": False, "gain_on_activation": gain is not None}

        def run() -> None:
            ops.gemm(ops.GemmCall(T, n_tot, K, 1, lhs, packed, epi, sumsq=sumsq,
                                  rscale_mask=1 if scaled else 0, inv_k=inv_k, eps=eps, extras=extra_bufs),
                     kernel="+".join(names))

        for n in names:
            self.plans[n] = info
        launch = Launch("+".join(names), "gemm", run, "th_gemm", info)
        return [norm_launch, launch] if norm_launch is not None else [launch]

    # e4m3 sibling merge (decode programs): GEMM kernels with e4m3 weights that
    # read the same lhs (q and k|v of the decode step) run as ONE th_gemm over
    # the concatenated weights and scales, each output on its own column window
    # (fused RoPE included: a head never straddles two windows), with one
    # activation-gain pre-pass and one reduce pass instead of one per kernel.
    def _plan_fp8_merges(self, program: Program, away: set[str]):
        produced_at = {o.tensor: i for i, k in enumerate(program.kernels) for o in k.outputs}

        def key(k: KernelSpec):
            if k.kind != "gemm" or not k.gemms:
                return None
            if any(self.program.tensors[k.arg(g.rhs).tensor].dtype != "float8_e4m3fn" for g in k.gemms):
                return None
            return (k.arg("lhs").tensor, k.k_extent, k.grid["rows"])

        groups: dict[str, list] = {}
        for i, k in enumerate(program.kernels):
            ki = key(k)
            if ki is None or k.name in away:
                continue
            members = [k]
            for j in range(i + 1, len(program.kernels)):
                k2 = program.kernels[j]
                if k2.name in away or key(k2) != ki:
                    continue
                # every other operand exists before the leader runs (params, program
                # inputs and constants, or an earlier kernel's output)
                ins = {a.tensor for a in k2.args if a.name != "lhs"}
                if all(produced_at.get(t, -1) < i for t in ins):
                    members.append(k2)
            if len(members) > 1:
                groups[k.name] = [(m, None, None) for m in members]
                away.update(m.name for m in members[1:])
        return groups

    def _lower_fp8_merged(self, members: list[KernelSpec]) -> list[Launch] | None:
        """One th_gemm for these e4m3 kernels, or None when their parts disagree
        (lhs, row scale, gain, RoPE tables) or an output needs a second accumulator
        or an extra operand."""
        parts = []
        for spec in members:
            plan = match_epilogue(spec)
            col: list = []
            if not plan.fused or self._lower_gemm_fused(spec, plan, collect=col) is None or not col:
                return None
            parts.append((spec, col[0]))
        p0 = parts[0][1]
        rope = next((pt["rope"] for _, pt in parts if pt["rope"] is not None), None)
        for spec, pt in parts:
            if not pt["fp8"] or pt["lhs"] is not p0["lhs"] or pt["extras"] or pt["norm"] is not None:
                return None
            if (pt["T"], pt["K"], pt["sumsq"], pt["inv_k"], pt["eps"]) != (p0["T"], p0["K"], p0["sumsq"], p0["inv_k"], p0["eps"]):
                return None
            if pt["mask"] not in (0, (1 << pt["n_used"]) - 1) or bool(pt["mask"]) != bool(p0["mask"]):
                return None
            if (pt["lhs_gain"] is None) != (p0["lhs_gain"] is None) or \
                    (pt["lhs_gain"] is not None and not torch.equal(pt["lhs_gain"], p0["lhs_gain"])):
                return None
            # every member's RoPE tables must equal the first ones met (one pair per launch)
            r = pt["rope"]
            if r is not None and (r[2:] != rope[2:] or not torch.equal(r[0], rope[0]) or not torch.equal(r[1], rope[1])):
                return None
            if any(e.b >= 0 or e.e >= 0 or e.cols is not None for e in pt["epi"]):
                return None
        T, K = p0["T"], p0["K"]
        ws_: list[torch.Tensor] = []
        scales: list[torch.Tensor] = []
        epi = []
        n_tot = 0
        for spec, pt in parts:
            win = {}
            for slot, (t, st) in enumerate(zip(pt["rhs"], pt["scales"])):
                ws_.append(self.buffers[t].view(torch.uint8))
                scales.append(self.buffers[st].float().reshape(-1))
                win[slot] = (n_tot, n_tot + pt["N"])
                n_tot += pt["N"]
            for e in pt["epi"]:
                if e.op in (abi.EPI_ROPE, abi.EPI_ROPE_PAIR) and rope is not None:
                    # a rotated window must hold whole heads (th_gemm would refuse it at run time)
                    hd = rope[3]
                    if win[e.a][0] % hd or (win[e.a][1] - win[e.a][0]) % hd:
                        return None
                epi.append(ops.EpiSpec(e.op, e.out, a=0, cols=win[e.a]))
        if len(epi) > abi.MAX_OUT:
            return None
        if rope is not None and n_tot % rope[3]:
            return None
        packed = ops.pack_rhs([torch.cat(ws_, dim=1).view(_FP8).contiguous()], _FP8)
        scale = torch.cat(scales).reshape(1, -1).contiguous()
        ws = self._workspace(max(ops.gemm_workspace_bytes(T, n_tot, K, 1, _FP8), 16), torch.uint8)
        names = [spec.name for spec, _ in parts]
        info = {"n_acc": 1, "merged": names, "cols": n_tot, "ops": [x.op for x in epi], "rscale": p0["sumsq"],
                "rope_fused": rope is not None, "weights": "float8_e4m3fn", "lhs_gain": p0["lhs_gain"] is not None}
        lhs, gain = p0["lhs"], p0["lhs_gain"]
        kw = dict(sumsq=p0["sumsq"], rscale_mask=1 if p0["mask"] else 0, inv_k=p0["inv_k"], eps=p0["eps"],
                  in_dtype=_FP8, rhs_scale=scale, workspace=ws)
        if gain is not None:
            kw["lhs_gain"] = gain

        def run() -> None:
            call = ops.GemmCall(T, n_tot, K, 1, lhs, packed, epi, **kw)
            if rope is not None:
                call.rope_cos, call.rope_sin, call.rope_period, call.rope_head_dim = rope[0], rope[1], rope[2], rope[3]
            ops.gemm(call, kernel="+".join(names))

        for n in names:
            self.plans[n] = info
        return [Launch("+".join(names), "gemm", run, "th_gemm", info)]

    # generic path ---------------------------------------------------------
    def _lower_gemm_vm(self, spec: KernelSpec) -> list[Launch]:
        """Raw fp32 accumulators (+ sum of squares) then th_epilogue_vm."""
        T, N, K = spec.grid["rows"], spec.grid["cols"], spec.k_extent
        lhs = self.buffers[spec.arg("lhs").tensor]
        launches: list[Launch] = []
        acc_bufs: dict[str, torch.Tensor] = {}
        sumsq = self._workspace(T) if spec.sumsq else None
        if spec.gemms:
            for start in range(0, len(spec.gemms), abi.MAX_ACC):
                group = list(range(start, min(start + abi.MAX_ACC, len(spec.gemms))))
                get_packed = self._pack(spec, [spec.gemms[i].rhs for i in group], lhs.dtype)
                bufs = [self._workspace(T * N).view(T, N) for _ in group]
                for i, b in zip(group, bufs):
                    acc_bufs[spec.gemms[i].acc] = b
                epi = [ops.EpiSpec(abi.EPI_ACC, b, a=s) for s, b in enumerate(bufs)]
                first = start == 0

                def run(group=group, get_packed=get_packed, epi=epi, first=first) -> None:
                    ops.gemm(ops.GemmCall(T, N, K, len(group), lhs, get_packed(), epi, sumsq=bool(first and sumsq is not None),
                                          sumsq_out=sumsq if first else None), kernel=spec.name)

                launches.append(Launch(spec.name, "gemm", run, "th_gemm", {"n_acc": len(group), "vm": True}))
        launches.append(self._vm_launch(spec, acc_bufs, sumsq, lhs))
        return launches

    def _vm_launch(self, spec: KernelSpec, acc_bufs: dict[str, torch.Tensor], sumsq: torch.Tensor | None,
                   lhs: torch.Tensor | None) -> Launch:
        from .vm import compile_vm

        M, N = (spec.grid["rows"], spec.grid["cols"]) if spec.kind == "gemm" else next(
            iter(acc_bufs.values())).shape
        prog = compile_vm(self, spec, acc_bufs, sumsq, lhs, M, N)
        ws = self._workspace(prog.n_slots * M * N)

        def run() -> None:
            ops.epilogue_vm(M, N, prog.operands, prog.ops, prog.outs, prog.n_slots, ws, kernel=spec.name)

        return Launch(spec.name, "epilogue_vm", run, "th_epilogue_vm", {"slots": prog.n_slots, "ops": len(prog.ops)})


def run_program(program: Program, params: dict[str, torch.Tensor], inputs, device: int = 0) -> dict[str, torch.Tensor]:
    """Device twin of the reference's interpreter ``run_program``: every produced
    tensor, on the device (each in a buffer of its own)."""
    dp = DeviceProgram(program, params, device, reuse_buffers=False)
    dp.run(inputs)
    return dict(dp.buffers)


def program_outputs(program: Program, params: dict[str, torch.Tensor], inputs, device: int = 0) -> list[torch.Tensor]:
    return DeviceProgram(program, params, device).run(inputs)
