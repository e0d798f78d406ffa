"""Offline weight transforms (reference: optimizer/param_transforms.py:13-51).

Each returns a new tensor; the passes store results as ``const`` nodes.
"""

from __future__ import annotations

import torch


def transpose_weight(w: torch.Tensor) -> torch.Tensor:
    """nn.Linear stores [N, K]; kernels consume [K, N]."""
    return w.t().contiguous()


def fold_gain_into_weight(gain: torch.Tensor, w_kn: torch.Tensor) -> torch.Tensor:
    """(x * g) @ W == x @ (diag(g) W) for a per-feature gain g[K]."""
    return (gain.float().reshape(-1, 1) * w_kn.float()).to(w_kn.dtype)


def rotate_half_matrix(head_dim: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """R with rotate_half(x) == x @ R for a row vector x[d]."""
    h = head_dim // 2
    r = torch.zeros(head_dim, head_dim, dtype=dtype)
    idx = torch.arange(h)
    r[idx + h, idx] = -1.0
    r[idx, idx + h] = 1.0
    return r


def rotate_half_heads_matrix(heads: int, head_dim: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    return torch.block_diag(*([rotate_half_matrix(head_dim, dtype)] * heads))


def rotate_columns(w_kn: torch.Tensor, heads: int, head_dim: int) -> torch.Tensor:
    """W @ R_heads, computed as a signed column permutation (exact in any dtype)."""
    k = w_kn.shape[0]
    w4 = w_kn.reshape(k, heads, head_dim)
    h = head_dim // 2
    return torch.cat((-w4[..., h:], w4[..., :h]), -1).reshape(k, heads * head_dim).contiguous()


def expand_rope_table(table: torch.Tensor, batch: int, heads: int) -> torch.Tensor:
    """[S, d] position table -> token-major [B*S, H*d]."""
    seq, d = table.shape
    return table.reshape(1, seq, 1, d).expand(batch, seq, heads, d).reshape(batch * seq, heads * d).contiguous()
