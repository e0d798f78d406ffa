"""One Llama-style decoder block in plain PyTorch (the benchmark workload).

Restates the reference's models/llama_block.py:28-159 (pre-norm RMSNorm, q/k/v
projections, RoPE from registered cos/sin buffers, explicit softmax attention,
SwiGLU MLP, residuals, no biases) and extends it for the MI355X configs:

* ``kv_heads`` < ``heads`` gives grouped-query attention; K/V heads are
  broadcast to the query heads with unsqueeze/expand/reshape (pure views);
* ``causal=True`` adds a registered [S, S] additive bias (0 on and below the
  diagonal, -inf above) to the scaled scores before the softmax.

With the defaults (``kv_heads=None``, ``causal=False``) it is the reference
block exactly. Weight init follows build_llama_block (reference
models/llama_block.py:148-159): 2-D weights N(0, 0.02), 1-D norm gains
U(0.8, 1.2), all drawn from the global RNG after ``torch.manual_seed(seed)``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn


@dataclass
class LlamaBlockConfig:
    batch: int = 2
    seq: int = 256
    hidden: int = 256
    heads: int = 4
    intermediate: int = 512
    eps: float = 1e-5
    rope_theta: float = 10000.0
    dtype: torch.dtype = torch.float16
    kv_heads: int | None = None
    causal: bool = False

    @property
    def head_dim(self) -> int:
        assert self.hidden % self.heads == 0
        return self.hidden // self.heads

    @property
    def n_kv(self) -> int:
        return self.heads if self.kv_heads is None else self.kv_heads

    @property
    def tokens(self) -> int:
        return self.batch * self.seq


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float, dtype: torch.dtype) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        var = x.pow(2).mean(-1, keepdim=True)
        return x * torch.rsqrt(var + self.eps) * self.weight


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope_tables(seq: int, head_dim: int, theta: float, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [seq, head_dim] (reference models/llama_block.py:73-79)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = torch.outer(torch.arange(seq, dtype=torch.float32), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def causal_bias(seq: int, dtype: torch.dtype) -> torch.Tensor:
    """[seq, seq] additive mask: 0 where key <= query, -inf above the diagonal."""
    idx = torch.arange(seq)
    return torch.zeros(seq, seq, dtype=dtype).masked_fill(idx.unsqueeze(0) > idx.unsqueeze(1), float("-inf"))


class LlamaAttention(nn.Module):
    def __init__(self, cfg: LlamaBlockConfig) -> None:
        super().__init__()
        self.heads, self.kv, self.head_dim, self.causal = cfg.heads, cfg.n_kv, cfg.head_dim, cfg.causal
        kv_dim = cfg.n_kv * cfg.head_dim
        self.q_proj = nn.Linear(cfg.hidden, cfg.hidden, bias=False, dtype=cfg.dtype)
        self.k_proj = nn.Linear(cfg.hidden, kv_dim, bias=False, dtype=cfg.dtype)
        self.v_proj = nn.Linear(cfg.hidden, kv_dim, bias=False, dtype=cfg.dtype)
        self.o_proj = nn.Linear(cfg.hidden, cfg.hidden, bias=False, dtype=cfg.dtype)

    def _expand_kv(self, t: torch.Tensor) -> torch.Tensor:
        if self.kv == self.heads:
            return t
        b, h, s, d = t.shape
        g = self.heads // self.kv
        return t[:, :, None, :, :].expand(b, h, g, s, d).reshape(b, h * g, s, d)

    def forward(self, h: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        b, s, _ = h.shape
        q = self.q_proj(h).view(b, s, self.heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(h).view(b, s, self.kv, self.head_dim).transpose(1, 2)
        v = self.v_proj(h).view(b, s, self.kv, self.head_dim).transpose(1, 2)
        q = q * cos + rotate_half(q) * sin
        k = k * cos + rotate_half(k) * sin
        k, v = self._expand_kv(k), self._expand_kv(v)
        scores = torch.matmul(q, k.transpose(-1, -2)) * (self.head_dim ** -0.5)
        if bias is not None:
            scores = scores + bias
        probs = torch.softmax(scores, dim=-1)
        a = torch.matmul(probs, v)
        a = a.transpose(1, 2).reshape(b, s, self.heads * self.head_dim)
        return self.o_proj(a)


class LlamaMLP(nn.Module):
    def __init__(self, cfg: LlamaBlockConfig) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden, cfg.intermediate, bias=False, dtype=cfg.dtype)
        self.up_proj = nn.Linear(cfg.hidden, cfg.intermediate, bias=False, dtype=cfg.dtype)
        self.down_proj = nn.Linear(cfg.intermediate, cfg.hidden, bias=False, dtype=cfg.dtype)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(h)) * self.up_proj(h))


class LlamaBlock(nn.Module):
    """``forward(x)``, ``x: [B, S, D]``; RoPE tables and the causal bias are buffers."""

    def __init__(self, cfg: LlamaBlockConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.input_norm = RMSNorm(cfg.hidden, cfg.eps, cfg.dtype)
        self.attn = LlamaAttention(cfg)
        self.post_norm = RMSNorm(cfg.hidden, cfg.eps, cfg.dtype)
        self.mlp = LlamaMLP(cfg)
        cos, sin = rope_tables(cfg.seq, cfg.head_dim, cfg.rope_theta, cfg.dtype)
        self.register_buffer("rope_cos", cos)
        self.register_buffer("rope_sin", sin)
        if cfg.causal:
            self.register_buffer("attn_bias", causal_bias(cfg.seq, cfg.dtype))
        else:
            self.attn_bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.input_norm(x), self.rope_cos, self.rope_sin, self.attn_bias)
        x = x + self.mlp(self.post_norm(x))
        return x

    def example_inputs(self, seed: int | None = None) -> tuple[torch.Tensor]:
        cfg = self.cfg
        if seed is None:
            return (torch.randn(cfg.batch, cfg.seq, cfg.hidden, dtype=cfg.dtype),)
        g = torch.Generator().manual_seed(seed)
        return (torch.randn(cfg.batch, cfg.seq, cfg.hidden, generator=g).to(cfg.dtype),)


def build_llama_block(cfg: LlamaBlockConfig | None = None, seed: int = 0) -> LlamaBlock:
    cfg = cfg or LlamaBlockConfig()
    torch.manual_seed(seed)
    block = LlamaBlock(cfg)
    with torch.no_grad():
        for _, p in block.named_parameters():
            if p.ndim == 2:
                p.normal_(0.0, 0.02)
            else:
                p.uniform_(0.8, 1.2)
    return block.eval()


# BASELINE.json configs 0 and 2 (C1, C3)
def config_c1() -> LlamaBlockConfig:
    return LlamaBlockConfig(batch=1, seq=128, hidden=512, heads=8, intermediate=1376, eps=1e-6,
                            rope_theta=10000.0, dtype=torch.float32, causal=True)


def config_c3() -> LlamaBlockConfig:
    return LlamaBlockConfig(batch=8, seq=2048, hidden=4096, heads=32, kv_heads=8, intermediate=14336, eps=1e-5,
                            rope_theta=500000.0, dtype=torch.bfloat16, causal=True)


def config_c5() -> LlamaBlockConfig:
    """BASELINE config 4 (C5): Llama-3-8B-shaped decode step, batch 64, KV cache 4096 per
    sequence (the new token is position 4096), 32 q / 8 kv heads x 128, FFN 14336;
    ``seq`` is the cache capacity including the new token."""
    return LlamaBlockConfig(batch=64, seq=4097, hidden=4096, heads=32, kv_heads=8, intermediate=14336, eps=1e-5,
                            rope_theta=500000.0, dtype=torch.bfloat16, causal=True)
