"""Functional Llama decoder block (oracle; test infrastructure only).

Restates reference models/llama_block.py:28-159: pre-norm RMSNorm
(``x * rsqrt(mean(x^2) + eps) * g``, :55-63), q/k/v projections, RoPE with
``rotate_half`` (:66-79, :99-100), softmax(q k^T / sqrt(d)) v (:101-103),
o-projection + residual, RMSNorm, SwiGLU MLP + residual (:108-117, :137-139).
Extensions used by the BASELINE configs: a causal mask (key j visible to
query i iff j <= i) and grouped KV heads (query head h reads kv head
h // (H / H_kv)).

``weights`` uses the nn.Linear convention [out, in] and the state-dict names
of ``targets.llama_block.LlamaBlock``.
"""

from __future__ import annotations

import math

import torch


def rms_norm(x: torch.Tensor, g: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * g


def rope_tables(seq: int, head_dim: int, theta: float, dtype=torch.float64):
    """cos/sin [seq, head_dim]: angle(pos, i) = pos * theta^(-2(i mod d/2)/d)."""
    half = head_dim // 2
    inv = theta ** (-torch.arange(half, dtype=torch.float64) * 2.0 / head_dim)
    ang = torch.arange(seq, dtype=torch.float64)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=1)
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def attention(q, k, v, causal: bool) -> torch.Tensor:
    """q [b, h, s, d]; k, v [b, hk, s, d] with h a multiple of hk."""
    h, hk = q.shape[1], k.shape[1]
    if hk != h:
        k = k.repeat_interleave(h // hk, dim=1)
        v = v.repeat_interleave(h // hk, dim=1)
    d = q.shape[-1]
    scores = q @ k.transpose(-1, -2) / math.sqrt(d)
    if causal:
        s = q.shape[2]
        scores = scores.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    return torch.softmax(scores, dim=-1) @ v


def block_forward(x: torch.Tensor, w: dict[str, torch.Tensor], *, heads: int, kv_heads: int, eps: float,
                  theta: float, causal: bool, rope: tuple[torch.Tensor, torch.Tensor] | None = None,
                  dtype=torch.float64, storage: torch.dtype | None = None,
                  round_residual: bool = False) -> torch.Tensor:
    """x [b, s, D] -> [b, s, D], computed in ``dtype``.

    ``rope`` overrides the cos/sin tables (e.g. with the model's own buffers,
    which the reference rounds to the model dtype, models/llama_block.py:79).

    ``storage`` (e.g. torch.bfloat16) rounds the values a bf16 program keeps
    in memory between kernels -- q, k, v after RoPE, the attention output,
    the residual stream where the MLP reads it as a GEMM operand and the
    SwiGLU product -- while the residual additions and the output stay in
    ``dtype``. This is the arithmetic of a bf16 block whose kernels
    accumulate in fp32, the bar a device result is compared against.
    ``round_residual`` (with ``storage``) also rounds the residual stream after
    the attention's residual addition and the block output: a program that
    keeps no fp32 copy of the residual stream and returns the model dtype."""
    w = {k: v.to(dtype) for k, v in w.items()}
    x = x.to(dtype)
    b, s, dm = x.shape
    hd = dm // heads
    cos, sin = rope if rope is not None else rope_tables(s, hd, theta, dtype)
    cos, sin = cos.to(dtype)[:s], sin.to(dtype)[:s]
    h = rms_norm(x, w["input_norm.weight"], eps)
    q = (h @ w["attn.q_proj.weight"].T).view(b, s, heads, hd).transpose(1, 2)
    k = (h @ w["attn.k_proj.weight"].T).view(b, s, kv_heads, hd).transpose(1, 2)
    v = (h @ w["attn.v_proj.weight"].T).view(b, s, kv_heads, hd).transpose(1, 2)
    rnd = (lambda t: t.to(storage).to(dtype)) if storage is not None else (lambda t: t)
    q = rnd(q * cos + rotate_half(q) * sin)
    k = rnd(k * cos + rotate_half(k) * sin)
    v = rnd(v)
    a = rnd(attention(q, k, v, causal).transpose(1, 2).reshape(b, s, heads * hd))
    x = x + a @ w["attn.o_proj.weight"].T
    if round_residual:
        x = rnd(x)
    h2 = rms_norm(rnd(x), w["post_norm.weight"], eps)
    gate = h2 @ w["mlp.gate_proj.weight"].T
    up = h2 @ w["mlp.up_proj.weight"].T
    mlp = rnd(gate * torch.sigmoid(gate) * up) @ w["mlp.down_proj.weight"].T
    return rnd(x + mlp) if round_residual else x + mlp


def decode_step(x: torch.Tensor, w: dict[str, torch.Tensor], k_cache: torch.Tensor, v_cache: torch.Tensor, pos: int,
                *, heads: int, kv_heads: int, eps: float, theta: float,
                rope: tuple[torch.Tensor, torch.Tensor] | None = None, dtype=torch.float64,
                storage: torch.dtype | None = None):
    """One new token per sequence at position ``pos`` with keys 0..pos-1 cached.

    x [b, D]; k_cache, v_cache [b, >= pos, kv_heads, hd] holding the RoPE'd keys
    and the values of the earlier positions. Returns (out [b, D], k_new, v_new)
    with k_new, v_new [b, kv_heads, hd] the entries for position ``pos``.
    This is block_forward's causal arithmetic for query row ``pos`` only: the
    decode path of the BASELINE's decode configuration (the reference itself
    has no KV cache).

    ``storage`` (e.g. torch.bfloat16) rounds what a bf16 step keeps in that
    dtype: the normalised GEMM operands x*g (the RMS row scale is applied to
    the fp32 accumulators), q, k, v, the attention output, the residual where
    the MLP reads it and the SwiGLU product. Its distance from the unrounded
    step is the rounding floor of a correct bf16 implementation."""
    w = {k: v.to(dtype) for k, v in w.items()}
    x = x.to(dtype)
    b, dm = x.shape
    rnd = (lambda t: t.to(storage).to(dtype)) if storage is not None else (lambda t: t)

    def norm(t, g):
        return rnd(t * g) * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + eps)

    hd = dm // heads
    if rope is None:
        cos, sin = rope_tables(pos + 1, hd, theta, dtype)
    else:
        cos, sin = rope[0].to(dtype), rope[1].to(dtype)
    cos, sin = cos[pos], sin[pos]
    h = norm(x, w["input_norm.weight"])
    q = (h @ w["attn.q_proj.weight"].T).view(b, heads, hd)
    k = (h @ w["attn.k_proj.weight"].T).view(b, kv_heads, hd)
    v = (h @ w["attn.v_proj.weight"].T).view(b, kv_heads, hd)
    q = rnd(q * cos + rotate_half(q) * sin)
    k = rnd(k * cos + rotate_half(k) * sin)
    v = rnd(v)
    keys = torch.cat([k_cache[:, :pos].to(dtype), k[:, None]], 1).transpose(1, 2)    # [b, kvh, pos+1, hd]
    vals = torch.cat([v_cache[:, :pos].to(dtype), v[:, None]], 1).transpose(1, 2)
    a = rnd(attention(q[:, :, None], keys, vals, False).reshape(b, heads * hd))
    x = x + a @ w["attn.o_proj.weight"].T
    h2 = norm(rnd(x), w["post_norm.weight"])
    gate = h2 @ w["mlp.gate_proj.weight"].T
    up = h2 @ w["mlp.up_proj.weight"].T
    return x + rnd(gate * torch.sigmoid(gate) * up) @ w["mlp.down_proj.weight"].T, k, v
