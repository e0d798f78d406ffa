"""Mamba-2 (SSD) backbone in plain PyTorch (the benchmark workload).

Restates the reference's models/mamba.py:73-391: pre-norm residual blocks
whose mixer is in_proj -> (z, xBC, dt) -> optional depthwise causal conv +
SiLU on xBC -> softplus(dt + dt_bias) -> the SSD scan with A = -exp(A_log)
-> + D x -> gated RMSNorm norm(y * silu(z)) -> out_proj, then a final norm.
The scan has the reference's two exactly equivalent forms: ``quadratic``
(decay-masked attention, what the compiler captures) and ``chunked`` (the
linear-time evaluation, used for the eager model at long sequences).

Extensions for the BASELINE configs, all off by default:
* ``a_log_range``: draw A_log ~ U(lo, hi) (the configs use [0, ln 16], so
  A = -exp(A_log) in [-16, -1]) instead of the reference's A in [-1, -0.1];
* ``vocab``: an embedding in front and a tied LM head behind the final norm
  (config 4).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn


@dataclass
class MambaConfig:
    batch: int = 2
    seq: int = 256
    d_model: int = 512
    expand: int = 2
    headdim: int = 32
    d_state: int = 32
    chunk: int = 64
    n_layers: int = 2
    mode: str = "quadratic"
    ngroups: int | None = None
    d_conv: int = 4
    use_conv: bool = False
    eps: float = 1e-5
    dt_min: float = 0.001
    dt_max: float = 0.1
    dtype: torch.dtype = torch.float16
    a_log_range: tuple[float, float] | None = None
    vocab: int | None = None

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def nheads(self) -> int:
        assert self.d_inner % self.headdim == 0
        return self.d_inner // self.headdim

    @property
    def groups(self) -> int:
        return self.nheads if self.ngroups is None else self.ngroups

    @property
    def d_bc(self) -> int:
        return self.groups * self.d_state

    @property
    def d_in_proj(self) -> int:
        return 2 * self.d_inner + 2 * self.d_bc + self.nheads

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    @property
    def nchunks(self) -> int:
        assert self.seq % self.chunk == 0
        return self.seq // self.chunk


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float, dtype: torch.dtype) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        var = x.pow(2).mean(-1, keepdim=True)
        return x * torch.rsqrt(var + self.eps) * self.weight


def ssd_quadratic(x, dA, dt, B, C, causal):
    """y = ((C B^T) * exp(cumA_i - cumA_j) * causal * dt_j) x over [b, h, s, .]
    (reference models/mamba.py:226-251): the mask goes inside the exponent."""
    cum = torch.cumsum(dA, dim=-1)
    cb = torch.matmul(C, B.transpose(-1, -2))
    delta = (cum.unsqueeze(-1) - cum.unsqueeze(-2)) * causal
    m = cb * torch.exp(delta) * causal * dt.unsqueeze(-2)
    return torch.matmul(m, x)


def ssd_chunked(x, dA, dt, B, C, chunk: int):
    """Linear-time form over [b, h, s, .]: within-chunk quadratic block plus a
    carried [p, n] state per chunk (reference models/mamba.py:163-223)."""
    b, h, s, p = x.shape
    n = B.shape[-1]
    out = torch.empty_like(x)
    state = torch.zeros(b, h, p, n, dtype=x.dtype)
    for c0 in range(0, s, chunk):
        c1 = min(s, c0 + chunk)
        cum = torch.cumsum(dA[..., c0:c1], dim=-1)
        ll = c1 - c0
        tri = torch.ones(ll, ll, dtype=torch.bool).tril()
        diff = (cum.unsqueeze(-1) - cum.unsqueeze(-2)).masked_fill(~tri, 0.0)
        m = torch.matmul(C[..., c0:c1, :], B[..., c0:c1, :].transpose(-1, -2)) * torch.exp(diff) * tri * dt[..., c0:c1].unsqueeze(-2)
        y = torch.matmul(m, x[..., c0:c1, :])
        y = y + torch.matmul(C[..., c0:c1, :], state.transpose(-1, -2)) * torch.exp(cum).unsqueeze(-1)
        out[..., c0:c1, :] = y
        last = cum[..., -1:]
        w = (dt[..., c0:c1] * torch.exp(last - cum)).unsqueeze(-1)
        state = state * torch.exp(last).unsqueeze(-1) + torch.matmul((x[..., c0:c1, :] * w).transpose(-1, -2), B[..., c0:c1, :])
    return out


class Mamba2Mixer(nn.Module):
    def __init__(self, cfg: MambaConfig) -> None:
        super().__init__()
        self.cfg = cfg
        d = cfg.dtype
        self.in_proj = nn.Linear(cfg.d_model, cfg.d_in_proj, bias=False, dtype=d)
        self.out_proj = nn.Linear(cfg.d_inner, cfg.d_model, bias=False, dtype=d)
        self.norm = RMSNorm(cfg.d_inner, cfg.eps, d)
        self.A_log = nn.Parameter(torch.zeros(cfg.nheads, dtype=d))
        self.D = nn.Parameter(torch.ones(cfg.nheads, dtype=d))
        self.dt_bias = nn.Parameter(torch.zeros(cfg.nheads, dtype=d))
        if cfg.use_conv:
            self.conv_weight = nn.Parameter(torch.zeros(2 * cfg.d_bc + cfg.d_inner, cfg.d_conv, dtype=d))
        idx = torch.arange(cfg.seq)
        self.register_buffer("mask_causal", (idx.unsqueeze(1) >= idx.unsqueeze(0)).to(d))

    def _conv(self, xbc: torch.Tensor) -> torch.Tensor:
        b, s, w = xbc.shape
        pad = torch.nn.functional.pad(xbc.transpose(1, 2), (self.cfg.d_conv - 1, 0))
        out = torch.nn.functional.conv1d(pad, self.conv_weight.unsqueeze(1), groups=w)
        return torch.nn.functional.silu(out.transpose(1, 2))

    def forward(self, u: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        b, s, _ = u.shape
        h, p, n, g = cfg.nheads, cfg.headdim, cfg.d_state, cfg.groups
        proj = self.in_proj(u)
        z, xbc, dt = torch.split(proj, [cfg.d_inner, cfg.d_inner + 2 * cfg.d_bc, h], dim=-1)
        if cfg.use_conv:
            xbc = self._conv(xbc)
        x, B, C = torch.split(xbc, [cfg.d_inner, cfg.d_bc, cfg.d_bc], dim=-1)
        dt = torch.nn.functional.softplus(dt + self.dt_bias)
        A = -torch.exp(self.A_log)
        xq = x.reshape(b, s, h, p).permute(0, 2, 1, 3)
        Bq = B.reshape(b, s, g, n).permute(0, 2, 1, 3)
        Cq = C.reshape(b, s, g, n).permute(0, 2, 1, 3)
        if g != h:
            Bq = Bq.unsqueeze(2).expand(b, g, h // g, s, n).reshape(b, h, s, n)
            Cq = Cq.unsqueeze(2).expand(b, g, h // g, s, n).reshape(b, h, s, n)
        dtq = dt.permute(0, 2, 1)
        dAq = dtq * A.reshape(1, h, 1)
        if cfg.mode == "chunked":
            y = ssd_chunked(xq, dAq, dtq, Bq, Cq, cfg.chunk)
        else:
            y = ssd_quadratic(xq, dAq, dtq, Bq, Cq, self.mask_causal)
        y = y + xq * self.D.reshape(1, h, 1, 1)
        y = y.permute(0, 2, 1, 3).reshape(b, s, cfg.d_inner)
        return self.out_proj(self.norm(y * torch.nn.functional.silu(z)))


class Mamba2Block(nn.Module):
    def __init__(self, cfg: MambaConfig) -> None:
        super().__init__()
        self.norm = RMSNorm(cfg.d_model, cfg.eps, cfg.dtype)
        self.mixer = Mamba2Mixer(cfg)

    def forward(self, u: torch.Tensor) -> torch.Tensor:
        return u + self.mixer(self.norm(u))


class MambaModel(nn.Module):
    """``forward(u)`` with ``u: [B, S, D]`` (or token ids [B, S] when ``vocab`` is set)."""

    def __init__(self, cfg: MambaConfig) -> None:
        super().__init__()
        self.cfg = cfg
        if cfg.vocab:
            self.embedding = nn.Embedding(cfg.vocab, cfg.d_model, dtype=cfg.dtype)
        self.layers = nn.ModuleList([Mamba2Block(cfg) for _ in range(cfg.n_layers)])
        self.norm_f = RMSNorm(cfg.d_model, cfg.eps, cfg.dtype)

    def forward(self, u: torch.Tensor) -> torch.Tensor:
        if self.cfg.vocab:
            u = self.embedding(u)
        for layer in self.layers:
            u = layer(u)
        u = self.norm_f(u)
        if self.cfg.vocab:
            u = u @ self.embedding.weight.t()
        return u

    def example_inputs(self, seed: int | None = None) -> tuple[torch.Tensor]:
        cfg = self.cfg
        g = torch.Generator().manual_seed(seed) if seed is not None else None
        if cfg.vocab:
            return (torch.randint(0, cfg.vocab, (cfg.batch, cfg.seq), generator=g),)
        return (torch.randn(cfg.batch, cfg.seq, cfg.d_model, generator=g).to(cfg.dtype),)


def build_mamba_model(cfg: MambaConfig | None = None, seed: int = 0) -> MambaModel:
    """Deterministic init (reference models/mamba.py:362-384; A_log range as configured)."""
    cfg = cfg or MambaConfig()
    torch.manual_seed(seed)
    model = MambaModel(cfg)
    with torch.no_grad():
        for name, param in model.named_parameters():
            if param.ndim == 2 and "conv" not in name:
                param.normal_(0.0, 0.02)
            elif "A_log" in name:
                if cfg.a_log_range is not None:
                    lo, hi = cfg.a_log_range
                    param.copy_((torch.rand(param.shape, dtype=torch.float32) * (hi - lo) + lo).to(param.dtype))
                else:
                    param.copy_(torch.log(torch.rand(param.shape, dtype=torch.float32) * 0.9 + 0.1).to(param.dtype))
            elif "dt_bias" in name:
                dt = torch.rand(param.shape, dtype=torch.float32) * (math.log(cfg.dt_max) - math.log(cfg.dt_min)) + math.log(cfg.dt_min)
                dt = dt.exp().clamp(min=1e-4)
                param.copy_((dt + torch.log(-torch.expm1(-dt))).to(param.dtype))
            elif "D" in name and param.ndim == 1:
                param.fill_(1.0)
            elif param.ndim == 1:
                param.uniform_(0.9, 1.1)
            else:
                param.normal_(0.0, 0.02)
    return model.eval()


def build_mamba_block(cfg: MambaConfig | None = None, seed: int = 0) -> MambaModel:
    cfg = cfg or MambaConfig(n_layers=1)
    cfg.n_layers = 1
    return build_mamba_model(cfg, seed)


# BASELINE.json configs 1 and 3 (C2, C4)
def config_c2() -> MambaConfig:
    return MambaConfig(batch=2, seq=1024, d_model=512, expand=2, headdim=64, d_state=64, chunk=64, n_layers=1,
                       ngroups=1, d_conv=4, use_conv=True, dtype=torch.bfloat16, a_log_range=(0.0, math.log(16.0)))


def config_c4() -> MambaConfig:
    return MambaConfig(batch=8, seq=2048, d_model=1024, expand=2, headdim=64, d_state=128, chunk=256, n_layers=24,
                       ngroups=1, d_conv=4, use_conv=True, dtype=torch.bfloat16, a_log_range=(0.0, math.log(16.0)),
                       vocab=50280)
