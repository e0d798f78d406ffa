"""The decode step of a Llama block with e4m3 weights (C5).

The reference block has no KV cache and its OpGraph no fp8 type
(models/llama_block.py:82-105, capture/opgraph.py:26); this module is the
decode configuration's eager definition: one new token per sequence at
position ``pos`` against a bf16 cache of the ``pos`` earlier keys and values,
with every projection stored as the BASELINE quantises it,

    s_n = max_k |W[n, k]| / 448,   q = e4m3(W / s_n),   W ~= q * s_n  (per output channel),

and the RMSNorm gains kept as the model's own (applied to the activations).
``forward(x, k_cache, v_cache)`` returns the block output and the new token's
key and value rows (the caller stores them at ``pos``).
"""

from __future__ import annotations

import dataclasses

import torch
from torch import nn

from .llama_block import LlamaBlock, LlamaBlockConfig, rope_tables, rotate_half

E4M3_MAX = 448.0
PROJECTIONS = {"wq": "attn.q_proj.weight", "wk": "attn.k_proj.weight", "wv": "attn.v_proj.weight",
               "wo": "attn.o_proj.weight", "wg": "mlp.gate_proj.weight", "wu": "mlp.up_proj.weight",
               "wd": "mlp.down_proj.weight"}


def quantize_per_output_channel(w_out_in: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """nn.Linear weight [out, in] -> (e4m3 [out, in], fp32 scales [out])."""
    w = w_out_in.detach().float()
    s = w.abs().amax(1).clamp_min(1e-30) / E4M3_MAX
    return (w / s[:, None]).to(torch.float8_e4m3fn), s


class LlamaDecodeBlock(nn.Module):
    """A Llama block's decode step at cache position ``pos`` (static, like the prefill's S)."""

    is_decode_step = True

    def __init__(self, block: LlamaBlock, pos: int) -> None:
        super().__init__()
        cfg = block.cfg
        if not 0 <= pos < cfg.seq:
            raise ValueError(f"pos {pos} outside the cache capacity {cfg.seq}")
        self.cfg, self.pos = cfg, pos
        sd = block.state_dict()
        for short, name in PROJECTIONS.items():
            q, s = quantize_per_output_channel(sd[name])
            self.register_buffer(f"{short}_q", q)
            self.register_buffer(f"{short}_s", s)
        self.register_buffer("g1", sd["input_norm.weight"].detach().clone())
        self.register_buffer("g2", sd["post_norm.weight"].detach().clone())
        cos, sin = rope_tables(pos + 1, cfg.head_dim, cfg.rope_theta, cfg.dtype)
        self.register_buffer("rope_cos", cos[pos:pos + 1].clone())
        self.register_buffer("rope_sin", sin[pos:pos + 1].clone())

    def weight(self, short: str) -> torch.Tensor:
        """The dequantised projection q * s_n, [out, in], in the model dtype."""
        return (getattr(self, f"{short}_q").float() * getattr(self, f"{short}_s")[:, None]).to(self.cfg.dtype)

    def dense_state_dict(self) -> dict[str, torch.Tensor]:
        """The LlamaBlock state (dequantised weights, the model's gains) this step computes with."""
        out = {name: self.weight(short) for short, name in PROJECTIONS.items()}
        out["input_norm.weight"], out["post_norm.weight"] = self.g1.clone(), self.g2.clone()
        return out

    def prefill_block(self, batch: int) -> LlamaBlock:
        """The block at S = 1 (non-causal) computing with this step's dequantised
        weights, the model's gains and the RoPE rows of ``pos``: the module whose
        capture compile_model turns into the decode program."""
        cfg1 = dataclasses.replace(self.cfg, seq=1, batch=batch, causal=False)
        blk = LlamaBlock(cfg1)
        sd = self.dense_state_dict()
        sd["rope_cos"], sd["rope_sin"] = self.rope_cos, self.rope_sin
        blk.load_state_dict(sd, strict=False)
        return blk.eval()

    def _norm(self, x: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.cfg.eps)).to(x.dtype) * g

    def forward(self, x: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor):
        """x [B, D]; k_cache, v_cache [B, L, Hkv, hd] (rows < pos hold the earlier tokens) ->
        (out [B, D], k_new [B, Hkv, hd], v_new [B, Hkv, hd])."""
        cfg, pos = self.cfg, self.pos
        b, hd, hq, hk = x.shape[0], cfg.head_dim, cfg.heads, cfg.n_kv
        h = self._norm(x, self.g1)
        q = (h @ self.weight("wq").T).view(b, hq, hd)
        k = (h @ self.weight("wk").T).view(b, hk, hd)
        v = (h @ self.weight("wv").T).view(b, hk, hd)
        q = q * self.rope_cos + rotate_half(q) * self.rope_sin
        k = k * self.rope_cos + rotate_half(k) * self.rope_sin
        keys = torch.cat([k_cache[:, :pos], k[:, None]], 1)          # [B, pos+1, Hkv, hd]
        vals = torch.cat([v_cache[:, :pos], v[:, None]], 1)
        grp = hq // hk
        keys = keys.repeat_interleave(grp, dim=2).permute(0, 2, 3, 1)  # [B, H, hd, pos+1]
        vals = vals.repeat_interleave(grp, dim=2).permute(0, 2, 1, 3)  # [B, H, pos+1, hd]
        scores = (q.unsqueeze(2) @ keys).float() * (hd ** -0.5)        # [B, H, 1, pos+1]
        a = (torch.softmax(scores, -1).to(x.dtype) @ vals).reshape(b, hq * hd)
        x1 = x + a @ self.weight("wo").T
        h2 = self._norm(x1, self.g2)
        act = torch.nn.functional.silu(h2 @ self.weight("wg").T) * (h2 @ self.weight("wu").T)
        return x1 + act @ self.weight("wd").T, k, v

    def example_inputs(self, seed: int = 0, batch: int | None = None):
        cfg = self.cfg
        b = batch or cfg.batch
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(b, cfg.hidden, generator=g).to(cfg.dtype)
        kc = torch.randn(b, cfg.seq, cfg.n_kv, cfg.head_dim, generator=g).to(cfg.dtype)
        vc = torch.randn(b, cfg.seq, cfg.n_kv, cfg.head_dim, generator=g).to(cfg.dtype)
        return x, kc, vc


def build_llama_decode_block(cfg: LlamaBlockConfig, pos: int, seed: int = 0) -> LlamaDecodeBlock:
    from .llama_block import build_llama_block

    return LlamaDecodeBlock(build_llama_block(cfg, seed=seed), pos).eval()
