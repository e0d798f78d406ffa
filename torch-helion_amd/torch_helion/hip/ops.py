"""Python entry points over the C ABI, taking torch device tensors.

Each function fills one descriptor of ``include/th_hip.h`` and launches on the
current torch stream. No function here computes anything on the host: if the
library is missing or the device is not gfx950 they raise
:class:`~torch_helion.hip.abi.HipBackendError`.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Sequence

import torch

from . import abi

_DT = {torch.float32: abi.TH_F32, torch.bfloat16: abi.TH_BF16, torch.float16: abi.TH_F16,
       torch.float8_e4m3fn: abi.TH_F8E4M3, torch.int32: abi.TH_I32, torch.int64: abi.TH_I64}


def th_dtype(t: torch.Tensor | torch.dtype) -> int:
    dt = t if isinstance(t, torch.dtype) else t.dtype
    if dt not in _DT:
        raise abi.HipBackendError("dtype", abi.TH_ERR_UNSUPPORTED, f"{dt} has no kernel")
    return _DT[dt]


def _lib(t: torch.Tensor) -> C.CDLL:
    if t.device.type != "cuda":
        raise abi.HipBackendError("device", abi.TH_ERR_INVALID, f"tensor on {t.device}, expected a HIP device")
    return abi.init_device(t.device.index or 0)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _row_major(t: torch.Tensor, name: str) -> int:
    """Row stride of a 2-D tensor whose last dim is contiguous."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise abi.HipBackendError(name, abi.TH_ERR_INVALID, f"expected a 2-D row-major tensor, got {tuple(t.shape)} strides {t.stride()}")
    return t.stride(0)


# ------------------------------------------------------------------ gemm
def acc_tile(n: int, n_acc: int, dtype: torch.dtype) -> int:
    return int(abi.load().th_gemm_acc_tile(n, n_acc, th_dtype(dtype)))


def pack_rhs(ws: Sequence[torch.Tensor], dtype: torch.dtype, out: torch.Tensor | None = None) -> torch.Tensor:
    """Pack [K, N] operands into th_gemm's K-contiguous interleaved layout."""
    lib = _lib(ws[0])
    k, n = ws[0].shape
    for w in ws:
        if tuple(w.shape) != (k, n) or w.dtype != ws[0].dtype:
            raise abi.HipBackendError("th_gemm_pack_rhs", abi.TH_ERR_INVALID, "operands differ in shape/dtype")
    nbytes = lib.th_gemm_packed_bytes(n, k, len(ws), th_dtype(dtype))
    if nbytes <= 0:
        raise abi.HipBackendError("th_gemm_packed_bytes", abi.TH_ERR_INVALID, f"N={n} K={k} n_acc={len(ws)}")
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=ws[0].device)
    elif out.numel() * out.element_size() < nbytes:
        raise abi.HipBackendError("th_gemm_pack_rhs", abi.TH_ERR_INVALID, "packed buffer too small")
    ptrs = (C.c_void_p * len(ws))(*[w.data_ptr() for w in ws])
    lds = (C.c_int64 * len(ws))(*[_row_major(w, "pack_rhs") for w in ws])
    abi.check(lib.th_gemm_pack_rhs(ptrs, lds, th_dtype(ws[0]), n, k, len(ws), th_dtype(dtype), out.data_ptr(),
                                   _stream(ws[0])), "th_gemm_pack_rhs")
    return out


@dataclass
class EpiSpec:
    """One fused output of th_gemm (see th_epi_op in include/th_hip.h). ``cols``: the
    accumulator column window [begin, end) the output holds (None: all N columns)."""

    op: int
    out: torch.Tensor
    a: int = 0
    b: int = -1
    e: int = -1
    cols: tuple[int, int] | None = None


@dataclass
class GemmCall:
    M: int
    N: int
    K: int
    n_acc: int
    lhs: torch.Tensor
    packed: torch.Tensor
    outs: list[EpiSpec]
    sumsq: bool = False
    rscale_mask: int = 0
    inv_k: float = 0.0
    eps: float = 0.0
    extras: list[torch.Tensor] = field(default_factory=list)
    rope_cos: torch.Tensor | None = None
    rope_sin: torch.Tensor | None = None
    rope_head_dim: int = 0
    rope_period: int = 0
    sumsq_out: torch.Tensor | None = None
    in_dtype: torch.dtype | None = None        # torch.float8_e4m3fn: bf16 lhs x e4m3 packed rhs
    rhs_scale: torch.Tensor | None = None      # fp8: [n_acc, N] fp32 per-column scales
    workspace: torch.Tensor | None = None      # gemm_workspace_bytes(...) bytes (fp8: required; fp32: optional)
    lhs_gain: torch.Tensor | None = None       # fp8: [K] fp32, products use lhs * gain (RMSNorm gain)
    rs_parts: torch.Tensor | None = None       # bf16 (fp8 without lhs_gain), with sumsq: [M, parts] fp32, the
                                               # rows' sums of squares as partial sums (the lhs producer's),
                                               # used instead of sum lhs^2
    gain_out: tuple[int, torch.Tensor, torch.Tensor] | None = None
    # fp8: (output index, gain [N] fp32, ss_parts_out [M, N/256] fp32): that bf16 output is stored as
    # bf16(bf16(v) * gain) and its rows' sums of bf16(v)^2 go to ss_parts_out, 256 columns per part
    # (the next GEMM's lhs with its RMSNorm gain applied, and that GEMM's rs_parts)

    def descriptor(self) -> abi.GemmDesc:
        d = abi.GemmDesc()
        d.M, d.N, d.K, d.n_acc = self.M, self.N, self.K, self.n_acc
        d.in_dtype = th_dtype(self.in_dtype if self.in_dtype is not None else self.lhs)
        if self.rhs_scale is not None:
            if self.rhs_scale.dtype != torch.float32 or not self.rhs_scale.is_contiguous() \
                    or self.rhs_scale.numel() != self.n_acc * self.N:
                raise abi.HipBackendError("th_gemm", abi.TH_ERR_INVALID, "rhs_scale must be contiguous fp32 [n_acc, N]")
            d.rhs_scale = self.rhs_scale.data_ptr()
        if self.workspace is not None:
            d.workspace = self.workspace.data_ptr()
            d.workspace_bytes = self.workspace.numel() * self.workspace.element_size()
        d.lhs = self.lhs.data_ptr()
        d.ld_lhs = _row_major(self.lhs, "th_gemm lhs")
        d.rhs_packed = self.packed.data_ptr()
        d.sumsq = 1 if self.sumsq else 0
        d.rscale_mask = self.rscale_mask
        d.inv_k, d.eps = self.inv_k, self.eps
        d.n_extra = len(self.extras)
        for i, x in enumerate(self.extras):
            d.extra[i] = x.data_ptr()
            d.ld_extra[i] = _row_major(x, "th_gemm extra")
            d.extra_dtype[i] = th_dtype(x)
        if self.rope_cos is not None:
            d.rope_cos, d.rope_sin = self.rope_cos.data_ptr(), self.rope_sin.data_ptr()
            d.rope_head_dim, d.rope_period = self.rope_head_dim, self.rope_period
        d.n_out = len(self.outs)
        for i, o in enumerate(self.outs):
            e = d.out[i]
            e.op, e.a, e.b, e.e = o.op, o.a, o.b, o.e
            e.ptr = o.out.data_ptr()
            e.ld = _row_major(o.out, "th_gemm out")
            e.dtype = th_dtype(o.out)
            if o.cols is not None:
                e.col_begin, e.col_end = o.cols
        if self.sumsq_out is not None:
            d.sumsq_out = self.sumsq_out.data_ptr()
        if self.lhs_gain is not None:
            if self.lhs_gain.dtype != torch.float32 or not self.lhs_gain.is_contiguous() or self.lhs_gain.numel() != self.K:
                raise abi.HipBackendError("th_gemm", abi.TH_ERR_INVALID, "lhs_gain must be contiguous fp32 [K]")
            d.lhs_gain = self.lhs_gain.data_ptr()
        if self.rs_parts is not None:
            if self.rs_parts.dtype != torch.float32 or self.rs_parts.dim() != 2 or self.rs_parts.shape[0] != self.M:
                raise abi.HipBackendError("th_gemm", abi.TH_ERR_INVALID, "rs_parts must be fp32 [M, parts]")
            d.rs_parts, d.ld_rs_parts = self.rs_parts.data_ptr(), _row_major(self.rs_parts, "th_gemm rs_parts")
            d.n_rs_parts = self.rs_parts.shape[1]
        if self.gain_out is not None:
            idx, g, parts = self.gain_out
            if g.dtype != torch.float32 or not g.is_contiguous() or g.numel() != self.N:
                raise abi.HipBackendError("th_gemm", abi.TH_ERR_INVALID, "gain_out gain must be contiguous fp32 [N]")
            if parts.dtype != torch.float32 or parts.dim() != 2 or parts.shape[0] != self.M \
                    or parts.shape[1] < self.N // 256:
                raise abi.HipBackendError("th_gemm", abi.TH_ERR_INVALID, "ss_parts_out must be fp32 [M, N/256]")
            d.gain_out, d.gain_out_index = g.data_ptr(), idx
            d.ss_parts_out, d.ld_ss_parts_out = parts.data_ptr(), _row_major(parts, "th_gemm ss_parts_out")
        return d


def gemm_workspace_bytes(M: int, N: int, K: int, n_acc: int, in_dtype: torch.dtype) -> int:
    n = abi.load().th_gemm_workspace_bytes(M, N, K, n_acc, th_dtype(in_dtype))
    if n < 0:
        raise abi.HipBackendError("th_gemm_workspace_bytes", abi.TH_ERR_INVALID, f"M={M} N={N} K={K} n_acc={n_acc}")
    return int(n)


def gemm(call: GemmCall, kernel: str | None = None) -> None:
    lib = _lib(call.lhs)
    d = call.descriptor()
    abi.check(lib.th_gemm(C.byref(d), _stream(call.lhs)), "th_gemm", kernel)


def gemm_noalloc(call: GemmCall, kernel: str | None = None) -> None:
    """th_gemm_noalloc: the same GEMM with the library's fixed per-GPU scratch in place of a
    workspace (``call.workspace`` is ignored); allocates nothing."""
    lib = _lib(call.lhs)
    d = call.descriptor()
    abi.check(lib.th_gemm_noalloc(C.byref(d), _stream(call.lhs)), "th_gemm_noalloc", kernel)


# --------------------------------------------------------------- RMSNorm
def rmsnorm(x: torch.Tensor, gain: torch.Tensor, eps: float, out: torch.Tensor, inv_k: float | None = None,
            kernel: str | None = None, out32: torch.Tensor | None = None) -> torch.Tensor:
    lib = _lib(x)
    d = abi.RmsNormDesc()
    d.M, d.K = x.shape
    d.x, d.ld_x, d.x_dtype = x.data_ptr(), _row_major(x, "th_rmsnorm x"), th_dtype(x)
    d.out, d.ld_out, d.out_dtype = out.data_ptr(), _row_major(out, "th_rmsnorm out"), th_dtype(out)
    if gain.dtype != torch.float32 or not gain.is_contiguous() or gain.numel() != x.shape[1]:
        raise abi.HipBackendError("th_rmsnorm", abi.TH_ERR_INVALID, "gain must be a contiguous fp32 [K] tensor")
    d.gain = gain.data_ptr()
    d.inv_k = 1.0 / x.shape[1] if inv_k is None else inv_k
    d.eps = eps
    if out32 is not None:
        d.out32, d.ld_out32 = out32.data_ptr(), _row_major(out32, "th_rmsnorm out32")
    abi.check(lib.th_rmsnorm(C.byref(d), _stream(x)), "th_rmsnorm", kernel)
    return out


# ------------------------------------------------------------- attention
def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, *, batch: int,
                      seq_q: int, seq_kv: int, heads_q: int, heads_kv: int, head_dim: int, scale: float,
                      causal: bool, kernel: str | None = None) -> torch.Tensor:
    lib = _lib(q)
    d = abi.AttnDesc()
    d.batch, d.seq_q, d.seq_kv, d.heads_q, d.heads_kv, d.head_dim = batch, seq_q, seq_kv, heads_q, heads_kv, head_dim
    d.scale, d.causal, d.dtype = scale, 1 if causal else 0, th_dtype(q)
    for t in (k, v, out):
        if t.dtype != q.dtype:
            raise abi.HipBackendError("th_attention_prefill", abi.TH_ERR_INVALID, "q/k/v/o dtypes differ")
    d.q, d.ld_q = q.data_ptr(), _row_major(q, "attention q")
    d.k, d.ld_k = k.data_ptr(), _row_major(k, "attention k")
    d.v, d.ld_v = v.data_ptr(), _row_major(v, "attention v")
    d.o, d.ld_o = out.data_ptr(), _row_major(out, "attention o")
    abi.check(lib.th_attention_prefill(C.byref(d), _stream(q)), "th_attention_prefill", kernel)
    return out


def attention_decode_workspace_bytes(batch: int, heads_q: int, heads_kv: int, head_dim: int, max_len: int,
                                     n_split: int = 0) -> int:
    n = abi.load().th_attention_decode_workspace_bytes(batch, heads_q, heads_kv, head_dim, max_len, n_split)
    if n < 0:
        raise abi.HipBackendError("th_attention_decode_workspace_bytes", abi.TH_ERR_INVALID, "bad sizes")
    return int(n)


def attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, out: torch.Tensor, *,
                     scale: float, lengths: torch.Tensor | None = None, fixed_len: int = 0, n_split: int = 0,
                     workspace: torch.Tensor | None = None, kernel: str | None = None) -> torch.Tensor:
    """One query token per sequence against a [batch, max_len, heads_kv, head_dim] KV cache.

    ``q``/``out``: [batch, heads_q*head_dim]; ``lengths``: optional int32 [batch] on the device."""
    lib = _lib(q)
    B, max_len, hkv, hd = k_cache.shape
    if v_cache.shape != k_cache.shape:
        raise abi.HipBackendError("th_attention_decode", abi.TH_ERR_INVALID, "k and v caches differ in shape")
    for t in (k_cache, v_cache):
        if t.stride(3) != 1 or t.stride(2) != hd:
            raise abi.HipBackendError("th_attention_decode", abi.TH_ERR_INVALID, "cache rows must be [heads_kv][head_dim] contiguous")
    d = abi.DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.head_dim = B, q.shape[1] // hd, hkv, hd
    d.max_len, d.n_split, d.fixed_len, d.dtype, d.scale = max_len, n_split, fixed_len, th_dtype(q), scale
    if lengths is not None:
        if lengths.dtype != torch.int32 or lengths.device != q.device:
            raise abi.HipBackendError("th_attention_decode", abi.TH_ERR_INVALID, "lengths must be int32 on the device")
        d.lengths = lengths.data_ptr()
    d.q, d.ld_q = q.data_ptr(), _row_major(q, "decode q")
    d.k_cache, d.k_stride_b, d.k_stride_t = k_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1)
    d.v_cache, d.v_stride_b, d.v_stride_t = v_cache.data_ptr(), v_cache.stride(0), v_cache.stride(1)
    d.o, d.ld_o = out.data_ptr(), _row_major(out, "decode o")
    if workspace is not None:
        d.workspace, d.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    abi.check(lib.th_attention_decode(C.byref(d), _stream(q)), "th_attention_decode", kernel)
    return out


# ----------------------------------------------------------- epilogue VM
def epilogue_vm(M: int, N: int, operands: list[tuple[torch.Tensor, bool]], ops: list[tuple], outs: list[tuple[torch.Tensor, int]],
                n_slots: int, workspace: torch.Tensor, kernel: str | None = None) -> None:
    """``operands``: (tensor, is_column); ``ops``: (code, dst, a, b, scalar, mode);
    ``outs``: (tensor, slot)."""
    ref = workspace
    lib = _lib(ref)
    if len(operands) > abi.VM_MAX_IN or len(ops) > abi.VM_MAX_OPS or len(outs) > abi.VM_MAX_OUT:
        raise abi.HipBackendError("th_epilogue_vm", abi.TH_ERR_UNSUPPORTED, "epilogue program too large")
    if workspace.dtype != torch.float32 or workspace.numel() < n_slots * M * N:
        raise abi.HipBackendError("th_epilogue_vm", abi.TH_ERR_INVALID, "workspace too small")
    d = abi.VmDesc()
    d.M, d.N = M, N
    d.n_in, d.n_ops, d.n_out, d.n_slots = len(operands), len(ops), len(outs), n_slots
    for i, (t, col) in enumerate(operands):
        d.in_[i].ptr, d.in_[i].ld, d.in_[i].dtype, d.in_[i].column = t.data_ptr(), t.stride(0), th_dtype(t), 1 if col else 0
    for i, (code, dst, a, b, scalar, mode) in enumerate(ops):
        o = d.ops[i]
        o.code, o.dst, o.a, o.b, o.scalar, o.mode = code, dst, a, b, scalar, mode
    for i, (t, slot) in enumerate(outs):
        d.out[i].ptr, d.out[i].ld, d.out[i].dtype, d.out[i].slot = t.data_ptr(), _row_major(t, "vm out"), th_dtype(t), slot
    d.workspace = workspace.data_ptr()
    abi.check(lib.th_epilogue_vm(C.byref(d), _stream(ref)), "th_epilogue_vm", kernel)


# ------------------------------------------------------------------- SSD
def ssd_workspace_bytes(batch: int, seq: int, heads: int, head_dim: int, state_dim: int, chunk: int,
                        ngroups: int | None = None) -> int:
    """Workspace of th_ssd_chunked: the minimum, or with ``ngroups`` the size that also holds
    the chunks' shared G^T tiles (formed once per B/C group instead of once per head)."""
    if ngroups is None:
        return int(abi.load().th_ssd_workspace_bytes(batch, seq, heads, head_dim, state_dim, chunk))
    return int(abi.load().th_ssd_gtile_workspace_bytes(batch, seq, heads, head_dim, state_dim, chunk, ngroups))


def ssd_chunked(*, x, b, c, dt, out, workspace, batch, seq, heads, head_dim, state_dim, ngroups, chunk, A=None, D=None,
                cum=None, dt_stride=1, dskip=None, gate=None, out32=None, y_gain=None, rs_parts=None,
                kernel: str | None = None) -> None:
    """One th_ssd_chunked launch. ``y_gain`` (fp32 [heads * head_dim]) stores y times that
    per-column gain and writes, into ``rs_parts`` (fp32 [batch * seq, heads * head_dim / 32]),
    the sums of squares of y before it per token and 32 columns: an RMSNorm whose row scale
    the consuming th_gemm applies (its ``rs_parts``)."""
    lib = _lib(x)
    d = abi.SsdDesc()
    d.batch, d.seq, d.heads, d.head_dim, d.state_dim, d.ngroups, d.chunk = batch, seq, heads, head_dim, state_dim, ngroups, chunk
    d.dtype = th_dtype(x)
    for t in (b, c, dt) + ((cum,) if cum is not None else ()) + ((dskip,) if dskip is not None else ()):
        if t.dtype != x.dtype:
            raise abi.HipBackendError("th_ssd_chunked", abi.TH_ERR_INVALID, "scan operands must share one dtype", kernel)
    d.x, d.ld_x = x.data_ptr(), _row_major(x, "ssd x")
    d.b, d.ld_b = b.data_ptr(), _row_major(b, "ssd b")
    d.c, d.ld_c = c.data_ptr(), _row_major(c, "ssd c")
    d.dt, d.ld_dt, d.dt_stride = dt.data_ptr(), _row_major(dt, "ssd dt"), dt_stride
    if cum is not None:
        d.cum, d.ld_cum = cum.data_ptr(), _row_major(cum, "ssd cum")
    if A is not None:
        d.A = A.data_ptr()
    if D is not None:
        d.D = D.data_ptr()
    if dskip is not None:
        d.dskip, d.ld_dskip = dskip.data_ptr(), _row_major(dskip, "ssd dskip")
    if gate is not None:
        d.gate, d.ld_gate, d.gate_dtype = gate.data_ptr(), _row_major(gate, "ssd gate"), th_dtype(gate)
    d.y, d.ld_y, d.y_dtype = out.data_ptr(), _row_major(out, "ssd y"), th_dtype(out)
    if out32 is not None:
        d.y32, d.ld_y32 = out32.data_ptr(), _row_major(out32, "ssd y32")
    if y_gain is not None:
        if y_gain.dtype != torch.float32 or not y_gain.is_contiguous() or y_gain.numel() != heads * head_dim:
            raise abi.HipBackendError("th_ssd_chunked", abi.TH_ERR_INVALID, "y_gain must be contiguous fp32 [H*P]", kernel)
        if rs_parts is None or rs_parts.dtype != torch.float32:
            raise abi.HipBackendError("th_ssd_chunked", abi.TH_ERR_INVALID, "y_gain needs fp32 rs_parts", kernel)
        d.y_gain = y_gain.data_ptr()
        d.rs_parts, d.ld_rs_parts = rs_parts.data_ptr(), _row_major(rs_parts, "ssd rs_parts")
    d.workspace, d.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    abi.check(lib.th_ssd_chunked(C.byref(d), _stream(x)), "th_ssd_chunked", kernel)


def conv1d_causal(x, w, out, *, batch: int, seq: int, activation: str | None, out32=None, kernel: str | None = None) -> None:
    lib = _lib(x)
    if w.dtype != torch.float32 or not w.is_contiguous():
        raise abi.HipBackendError("th_conv1d_causal", abi.TH_ERR_INVALID, "weights must be contiguous fp32 [C, K]", kernel)
    d = abi.ConvDesc()
    d.batch, d.seq, d.width, d.kernel = batch, seq, w.shape[0], w.shape[1]
    d.activation = 1 if activation == "silu" else 0
    d.x_dtype, d.y_dtype = th_dtype(x), th_dtype(out)
    d.x, d.ld_x = x.data_ptr(), _row_major(x, "conv x")
    d.w = w.data_ptr()
    d.y, d.ld_y = out.data_ptr(), _row_major(out, "conv y")
    if out32 is not None:
        d.y32, d.ld_y32 = out32.data_ptr(), _row_major(out32, "conv y32")
    abi.check(lib.th_conv1d_causal(C.byref(d), _stream(x)), "th_conv1d_causal", kernel)


def embedding(table: torch.Tensor, ids: torch.Tensor, out: torch.Tensor, *, out32: torch.Tensor | None = None,
              n_invalid: torch.Tensor | None = None, kernel: str | None = None) -> None:
    """out[t] = table[ids[t]] (th_embedding). Rows of ids outside [0, vocab) are
    written as zeros and counted in ``n_invalid`` (an int32 device scalar) if given."""
    lib = _lib(table)
    if ids.dtype not in (torch.int64, torch.int32) or not ids.is_contiguous():
        raise abi.HipBackendError("th_embedding", abi.TH_ERR_INVALID, "ids must be contiguous int64 or int32", kernel)
    if out.dtype != table.dtype or out.shape[-1] != table.shape[1] or out.numel() != ids.numel() * table.shape[1]:
        raise abi.HipBackendError("th_embedding", abi.TH_ERR_INVALID,
                                  f"out {tuple(out.shape)} {out.dtype} does not match ids {tuple(ids.shape)} "
                                  f"x table {tuple(table.shape)} {table.dtype}", kernel)
    if n_invalid is not None and (n_invalid.dtype != torch.int32 or n_invalid.device != table.device):
        raise abi.HipBackendError("th_embedding", abi.TH_ERR_INVALID, "n_invalid must be an int32 device tensor", kernel)
    out2 = out.reshape(-1, table.shape[1]) if out.dim() != 2 else out
    d = abi.EmbeddingDesc()
    d.tokens, d.dim, d.vocab = ids.numel(), table.shape[1], table.shape[0]
    d.dtype, d.ids_dtype = th_dtype(table), th_dtype(ids)
    d.table, d.ld_table = table.data_ptr(), _row_major(table, "embedding table")
    d.ids = ids.data_ptr()
    d.out, d.ld_out = out2.data_ptr(), _row_major(out2, "embedding out")
    if out32 is not None:
        o32 = out32.reshape(-1, table.shape[1]) if out32.dim() != 2 else out32
        d.out32, d.ld_out32 = o32.data_ptr(), _row_major(o32, "embedding out32")
    if n_invalid is not None:
        d.n_invalid = n_invalid.data_ptr()
    abi.check(lib.th_embedding(C.byref(d), _stream(table)), "th_embedding", kernel)
