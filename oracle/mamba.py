"""Mamba-2 oracle (test infrastructure only).

* ``ssd_recurrence``: the direct O(S) state recurrence, the definition the
  reference's tests hold both scan forms to (reference tests/test_mamba.py:27-38):
  ``state_t = exp(dA_t) state_{t-1} + dt_t x_t B_t^T``, ``y_t = state_t C_t``.
* ``ssd_chunked_program``: the ``ssd_chunked`` OpIR kind on token-major
  operands (dt [T, H], B/C [T, G*N] shared by H/G heads each, x [T, H*P],
  per-head A and D), evaluated with the recurrence.
* ``block_forward`` / ``backbone_forward``: a functional restatement of the
  reference's Mamba-2 block and backbone (models/mamba.py:254-391): RMSNorm,
  in_proj split into z, xBC, dt; optional depthwise causal conv + SiLU on xBC;
  dt = softplus(dt + dt_bias); A = -exp(A_log); y = scan + D x; gated RMSNorm
  ``norm(y * silu(z))``; out_proj; residual; final RMSNorm for the backbone.
* ``model_forward``: token ids -> rows of the embedding table -> backbone ->
  logits against the same table (tied head, ``h E^T``). The reference's model
  takes hidden states (models/mamba.py:343-359); the ids front end and the
  tied head are the language-model form of that backbone. Pinned against the
  eager ``nn.Embedding`` model, whose lookup and head are torch's own.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def ssd_recurrence(x: torch.Tensor, dA: torch.Tensor, dt: torch.Tensor, B: torch.Tensor, C: torch.Tensor) -> torch.Tensor:
    """x [b,h,s,p], dA/dt [b,h,s], B/C [b,h,s,n] -> y [b,h,s,p]."""
    b, h, s, p = x.shape
    n = B.shape[-1]
    state = torch.zeros(b, h, p, n, dtype=x.dtype)
    ys = []
    for t in range(s):
        state = torch.exp(dA[:, :, t])[..., None, None] * state \
            + (dt[:, :, t][..., None, None] * x[:, :, t][..., :, None]) * B[:, :, t][..., None, :]
        ys.append((state * C[:, :, t][..., None, :]).sum(-1))
    return torch.stack(ys, dim=2)


def ssd_chunked_program(c, bm, x, dt, A, D, a) -> torch.Tensor:
    """Token-major ``ssd_chunked`` operands -> [T, H*P] (chunking does not change the value)."""
    bs, s, h, p, n = a["batch"], a["seq"], a["heads"], a["head_dim"], a["state_dim"]
    g = a.get("ngroups", h)
    rep = h // g
    x4 = x.reshape(bs, s, h, p).permute(0, 2, 1, 3)
    b4 = bm.reshape(bs, s, g, n).permute(0, 2, 1, 3).repeat_interleave(rep, dim=1)
    c4 = c.reshape(bs, s, g, n).permute(0, 2, 1, 3).repeat_interleave(rep, dim=1)
    dt3 = dt.reshape(bs, s, h).permute(0, 2, 1)
    y = ssd_recurrence(x4, dt3 * A.reshape(1, h, 1), dt3, b4, c4)
    y = y + x4 * D.reshape(1, h, 1, 1)
    return y.permute(0, 2, 1, 3).reshape(bs * s, h * p)


def rms_norm(x, g, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * g


def causal_depthwise_conv(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x [b, s, c], w [c, k]: y[b,t,c] = sum_j w[c,j] x[b, t-(k-1)+j, c]."""
    k = w.shape[1]
    xp = F.pad(x, (0, 0, k - 1, 0))
    return sum(w[:, j] * xp[:, j:j + x.shape[1]] for j in range(k))


def mixer_forward(h: torch.Tensor, w: dict[str, torch.Tensor], prefix: str, cfg) -> torch.Tensor:
    b, s, _ = h.shape
    di, nh, hp, n, g = cfg.d_inner, cfg.nheads, cfg.headdim, cfg.d_state, cfg.groups
    proj = h @ w[prefix + "in_proj.weight"].T
    z, xbc, dt = proj[..., :di], proj[..., di:2 * di + 2 * g * n], proj[..., 2 * di + 2 * g * n:]
    if cfg.use_conv:
        xbc = F.silu(causal_depthwise_conv(xbc, w[prefix + "conv_weight"]))
    x, B, C = xbc[..., :di], xbc[..., di:di + g * n], xbc[..., di + g * n:]
    dt = F.softplus(dt + w[prefix + "dt_bias"])
    A = -torch.exp(w[prefix + "A_log"])
    x4 = x.reshape(b, s, nh, hp).permute(0, 2, 1, 3)
    rep = nh // g
    B4 = B.reshape(b, s, g, n).permute(0, 2, 1, 3).repeat_interleave(rep, dim=1)
    C4 = C.reshape(b, s, g, n).permute(0, 2, 1, 3).repeat_interleave(rep, dim=1)
    dt3 = dt.permute(0, 2, 1)
    y = ssd_recurrence(x4, dt3 * A.reshape(1, nh, 1), dt3, B4, C4) + x4 * w[prefix + "D"].reshape(1, nh, 1, 1)
    y = y.permute(0, 2, 1, 3).reshape(b, s, di)
    gated = rms_norm(y * F.silu(z), w[prefix + "norm.weight"], cfg.eps)
    return gated @ w[prefix + "out_proj.weight"].T


def backbone_forward(u: torch.Tensor, w: dict[str, torch.Tensor], cfg, dtype=torch.float64) -> torch.Tensor:
    """Stacked blocks ``u + mixer(rmsnorm(u))`` then the final RMSNorm."""
    w = {k: v.to(dtype) for k, v in w.items()}
    u = u.to(dtype)
    for i in range(cfg.n_layers):
        pre = f"layers.{i}."
        u = u + mixer_forward(rms_norm(u, w[pre + "norm.weight"], cfg.eps), w, pre + "mixer.", cfg)
    return rms_norm(u, w["norm_f.weight"], cfg.eps)


def model_forward(ids: torch.Tensor, w: dict[str, torch.Tensor], cfg, dtype=torch.float64,
                  layers: int | None = None) -> torch.Tensor:
    """Logits [b, s, vocab] for token ids [b, s]: ``backbone(E[ids]) @ E^T``.
    ``layers`` keeps only the first layers (the model with fewer blocks)."""
    table = w["embedding.weight"].to(dtype)
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= table.shape[0]):
        raise IndexError("token id outside the embedding table")
    u = table[ids.long()]
    if layers is not None:
        cfg = _with_layers(cfg, layers)
    h = backbone_forward(u, w, cfg, dtype)
    return h @ table.T


def _with_layers(cfg, n: int):
    import copy

    c = copy.copy(cfg)
    c.n_layers = n
    return c
