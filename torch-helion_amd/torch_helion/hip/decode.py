"""Decode step of a Llama block on the HIP backend: one new token per sequence,
e4m3 weights with per-output-channel scales, a bf16 KV cache.

The reference has no decode path (its models/llama_block.py:82-105 has no KV
cache and its OpGraph no fp8 type); this runner is the decode configuration of
the BASELINE (Llama-3-8B-shaped block, batch 64, cache 4096) built from the same
kernel library. A step is five library calls:

  k0  th_gemm e4m3   [q | k | v] = r (x g1) [Wq | Wk | Wv],  r = RMS row scale of x;
                     three column-window outputs: q = rope_pos(.), k = rope_pos(.)
                     and v written straight into the caches at position ``pos``
                     (the output row stride is the cache's sequence stride)
  k1  th_attention_decode over keys 0..pos
  k2  th_gemm e4m3   x1 = x + attn Wo
  k3  th_gemm e4m3   act = silu(r2 (x1 g2) Wg) * (r2 (x1 g2) Wu)
  k4  th_gemm e4m3   out = x1 + act Wd

With ``fold_gain`` (the default; hidden a multiple of 1024) k2's finishing pass
also applies the post-attention norm's gain: it stores bf16(bf16(x1) g2), the
operand k3 multiplies, and each row's sums of bf16(x1)^2 in parts of 256
columns, which k3 adds up for r2 (``gain_out`` / ``rs_parts``); k3 then needs no
pass of its own to scale its rows. The values are the same either way; the
row sums add the same squares in another order.

Every weight is the model's own ``W`` quantised per output channel,
``q = e4m3(W / s_n)`` with ``s_n = max_k |W[k, n]| / 448``. The RMSNorm gains
stay on the activation side (``lhs_gain``: the GEMM multiplies x by g as it
stages it, after taking the row's sum of squares), so the step computes the
block whose weights are the dequantised ``q s_n`` and whose norm gains are the
model's: ``effective_weights()``. (Folding the gain into the weights before
quantising, as the prefill pipeline folds it into bf16 weights, would quantise
a different matrix.)
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import abi, ops

_FP8 = torch.float8_e4m3fn
_E4M3_MAX = 448.0


def quantize_e4m3(w_kn: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel e4m3 quantisation of a [K, N] weight:
    s[n] = max_k |w[k, n]| / 448, q = e4m3(w / s)."""
    w = w_kn.float()
    s = (w.abs().amax(0).clamp_min(1e-30) / _E4M3_MAX).float()
    return (w / s).to(_FP8), s


@dataclass
class _Proj:
    packed: torch.Tensor
    scale: torch.Tensor   # [n_acc, N] fp32
    n: int
    k: int
    n_acc: int


class DecodeBlock:
    """A Llama block's weights in e4m3 on the device, its KV cache and the step launches."""

    def __init__(self, state_dict: dict[str, torch.Tensor], *, hidden: int, heads: int, kv_heads: int,
                 intermediate: int, eps: float, rope_theta: float, batch: int, max_len: int,
                 device: int | torch.device = 0, fold_gain: bool = True) -> None:
        self.device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        if self.device.type != "cuda":
            raise abi.HipBackendError("DecodeBlock", abi.TH_ERR_INVALID, f"device {device} is not a HIP device")
        abi.init_device(self.device.index or 0)
        self.D, self.H, self.Hkv, self.F = hidden, heads, kv_heads, intermediate
        self.hd = hidden // heads
        self.eps, self.theta = eps, rope_theta
        self.B, self.max_len = batch, max_len
        sd = {k: v.detach().float().cpu() for k, v in state_dict.items()}
        g1, g2 = sd["input_norm.weight"], sd["post_norm.weight"]
        self._eff: dict[str, torch.Tensor] = {"input_norm.weight": g1.clone(), "post_norm.weight": g2.clone()}

        def proj(names: list[str], concat: bool = False) -> _Proj:
            """One accumulator per weight, or (concat) one accumulator over the weights'
            columns side by side; per-output-channel scales either way."""
            qs = [quantize_e4m3(sd[n].T.contiguous()) for n in names]   # nn.Linear [out, in] -> [K, N]
            for n, (q, s) in zip(names, qs):
                self._eff[n] = (q.float() * s[None, :]).T.contiguous()   # [out, in], what the step multiplies by
            if concat:
                qs = [(torch.cat([q.view(torch.uint8) for q, _ in qs], 1).view(_FP8), torch.cat([s for _, s in qs]))]
            k_, n_ = qs[0][0].shape
            packed = ops.pack_rhs([q.to(self.device) for q, _ in qs], _FP8)
            scale = torch.stack([s for _, s in qs]).to(self.device).contiguous()
            return _Proj(packed, scale, n_, k_, len(qs))

        self.wqkv = proj(["attn.q_proj.weight", "attn.k_proj.weight", "attn.v_proj.weight"], concat=True)
        self.wo = proj(["attn.o_proj.weight"])
        self.wgu = proj(["mlp.gate_proj.weight", "mlp.up_proj.weight"])
        self.wd = proj(["mlp.down_proj.weight"])

        dev, B = self.device, batch
        self.g1 = g1.to(dev).contiguous()
        self.g2 = g2.to(dev).contiguous()
        bf = torch.bfloat16
        self.k_cache = torch.zeros(B, max_len, kv_heads, self.hd, dtype=bf, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.q = torch.empty(B, heads * self.hd, dtype=bf, device=dev)
        self.attn = torch.empty_like(self.q)
        self.x1 = torch.empty(B, hidden, dtype=bf, device=dev)  # with fold_gain: bf16(x1) g2
        self.x1_32 = torch.empty(B, hidden, device=dev)
        self.fold_gain = fold_gain and hidden % 1024 == 0
        self.x1_parts = torch.empty(B, hidden // 256, device=dev) if self.fold_gain else None
        self.act = torch.empty(B, intermediate, dtype=bf, device=dev)
        self.out = torch.empty(B, hidden, dtype=bf, device=dev)
        self.out32 = torch.empty(B, hidden, device=dev)
        inv = 1.0 / (rope_theta ** (torch.arange(0, self.hd, 2, dtype=torch.float64) / self.hd))
        ang = torch.outer(torch.arange(max_len, dtype=torch.float64), inv)
        ang = torch.cat([ang, ang], -1)
        self.cos = ang.cos().float().to(dev).contiguous()
        self.sin = ang.sin().float().to(dev).contiguous()
        ws = max(ops.gemm_workspace_bytes(B, p.n, p.k, p.n_acc, _FP8) for p in (self.wqkv, self.wo, self.wgu, self.wd))
        self.gemm_ws = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        aw = ops.attention_decode_workspace_bytes(B, heads, kv_heads, self.hd, max_len)
        self.attn_ws = torch.empty(max(aw // 4, 1), device=dev)

    # ------------------------------------------------------------------
    def effective_weights(self) -> dict[str, torch.Tensor]:
        """The weights the step multiplies by, as an fp32 state dict: the dequantised
        projections ``q s_n`` and the model's norm gains."""
        return dict(self._eff)

    def _gemm(self, p: _Proj, lhs: torch.Tensor, outs: list[ops.EpiSpec], **kw) -> None:
        ops.gemm(ops.GemmCall(lhs.shape[0], p.n, p.k, p.n_acc, lhs, p.packed, outs, in_dtype=_FP8,
                              rhs_scale=p.scale, workspace=self.gemm_ws, **kw))

    def step(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        """One token per sequence at position ``pos`` (0 <= pos < max_len); x [batch, hidden]
        bf16 on the device. Writes the new keys/values into the caches and returns the block
        output [batch, hidden] (bf16; ``self.out32`` holds it in fp32)."""
        if not 0 <= pos < self.max_len:
            raise abi.HipBackendError("DecodeBlock.step", abi.TH_ERR_INVALID, f"pos {pos} outside the cache")
        if x.dtype != torch.bfloat16 or tuple(x.shape) != (self.B, self.D):
            raise abi.HipBackendError("DecodeBlock.step", abi.TH_ERR_INVALID, "x must be bf16 [batch, hidden]")
        E = abi
        norm = dict(sumsq=True, inv_k=1.0 / self.D, eps=self.eps)
        rope = dict(rope_cos=self.cos[pos:pos + 1], rope_sin=self.sin[pos:pos + 1], rope_head_dim=self.hd,
                    rope_period=1)
        B, kvw = self.B, self.Hkv * self.hd
        kslot = self.k_cache[:, pos].view(B, kvw)
        vslot = self.v_cache[:, pos].view(B, kvw)
        qw = self.H * self.hd
        self._gemm(self.wqkv, x, [ops.EpiSpec(E.EPI_ROPE, self.q, a=0, cols=(0, qw)),
                                  ops.EpiSpec(E.EPI_ROPE, kslot, a=0, cols=(qw, qw + kvw)),
                                  ops.EpiSpec(E.EPI_ACC, vslot, a=0, cols=(qw + kvw, qw + 2 * kvw))],
                   rscale_mask=0b1, lhs_gain=self.g1, **norm, **rope)
        ops.attention_decode(self.q, self.k_cache, self.v_cache, self.attn, scale=1.0 / math.sqrt(self.hd),
                             fixed_len=pos + 1, workspace=self.attn_ws)
        o_outs = [ops.EpiSpec(E.EPI_ADD, self.x1, e=0), ops.EpiSpec(E.EPI_ADD, self.x1_32, e=0)]
        gu_outs = [ops.EpiSpec(E.EPI_SWIGLU, self.act, a=0, b=1)]
        if self.fold_gain:
            self._gemm(self.wo, self.attn, o_outs, extras=[x], gain_out=(0, self.g2, self.x1_parts))
            self._gemm(self.wgu, self.x1, gu_outs, rscale_mask=0b11, rs_parts=self.x1_parts, **norm)
        else:
            self._gemm(self.wo, self.attn, o_outs, extras=[x])
            self._gemm(self.wgu, self.x1, gu_outs, rscale_mask=0b11, lhs_gain=self.g2, **norm)
        self._gemm(self.wd, self.act, [ops.EpiSpec(E.EPI_ADD, self.out, e=0), ops.EpiSpec(E.EPI_ADD, self.out32, e=0)],
                   extras=[self.x1_32])
        return self.out

    def capture(self, x: torch.Tensor, pos: int) -> None:
        """Record ``step(x, pos)`` into a HIP graph (fixed input buffer and position);
        ``replay()`` then re-runs it without host launch overhead."""
        with torch.cuda.device(self.device):
            torch.cuda.synchronize()
            self.step(x, pos)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.step(x, pos)
            torch.cuda.synchronize()
        self.graph = g

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.out

    def bytes_per_step(self, pos: int) -> int:
        """HBM bytes a step must move: every weight byte and the cached keys/values it attends over."""
        kv = 2 * self.B * (pos + 1) * self.Hkv * self.hd * 2
        return self.weight_bytes() + kv

    def weight_bytes(self) -> int:
        return sum(p.n * p.k * p.n_acc for p in (self.wqkv, self.wo, self.wgu, self.wd))
