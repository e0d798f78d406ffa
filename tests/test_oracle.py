"""Pinning the oracle: each oracle function against something independent of it.

* oracle.mamba.ssd_recurrence is the reference's definition (tests/test_mamba.py:27-38);
  it is pinned by a single-step closed form and by the two scan forms of the
  eager model (quadratic and chunked) agreeing with it to 1e-10 in float64,
  with a planted sign error that must be caught.
* oracle.llama.block_forward is pinned against the nn.Module restatement in
  targets/ (an independent implementation) and its attention against torch's
  scaled_dot_product_attention (causal and grouped KV).
* oracle.interpret is pinned against the reference's recorded Llama reference
  check (bit-exact max_rel_err from tests/golden) through the product
  interpreter agreeing with it to fp32 rounding, and per kind against the
  closed forms above.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

GOLDEN = Path(__file__).parent / "golden" / "reference_results"


def _ssd_inputs(b=2, h=3, s=24, p=4, n=5, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, h, s, p, generator=g, dtype=dtype)
    B = torch.randn(b, h, s, n, generator=g, dtype=dtype)
    C = torch.randn(b, h, s, n, generator=g, dtype=dtype)
    dt = torch.rand(b, h, s, generator=g, dtype=dtype) * 0.1 + 0.01
    A = -(torch.rand(b, h, 1, generator=g, dtype=dtype) * 15 + 1)
    return x, dt * A, dt, B, C


def test_recurrence_single_step_closed_form():
    from oracle.mamba import ssd_recurrence

    x, dA, dt, B, C = _ssd_inputs(s=1)
    y = ssd_recurrence(x, dA, dt, B, C)
    expect = dt[..., None] * x * (B * C).sum(-1, keepdim=True)
    assert torch.allclose(y, expect, atol=1e-14)


def test_recurrence_matches_both_scan_forms():
    from oracle.mamba import ssd_recurrence
    from targets.mamba import ssd_chunked, ssd_quadratic

    x, dA, dt, B, C = _ssd_inputs()
    ref = ssd_recurrence(x, dA, dt, B, C)
    s = x.shape[2]
    causal = torch.ones(s, s, dtype=torch.float64).tril()
    yq = ssd_quadratic(x, dA, dt, B, C, causal)
    assert (yq - ref).abs().max() / ref.abs().max() < 1e-10
    for chunk in (1, 5, 6, 24):
        yc = ssd_chunked(x, dA, dt, B, C, chunk)
        assert (yc - ref).abs().max() / ref.abs().max() < 1e-10, chunk
    # a planted mistake (decay sign flipped) is caught
    bad = ssd_recurrence(x, -dA, dt, B, C)
    assert (bad - ref).abs().max() / ref.abs().max() > 1e-2


def test_ssd_chunked_program_groups():
    """Token-major program form with shared B/C groups == per-head recurrence with repeated groups."""
    from oracle.mamba import ssd_chunked_program, ssd_recurrence

    bs, s, h, p, n, g = 2, 16, 4, 3, 5, 2
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(bs * s, h * p, generator=gen, dtype=torch.float64)
    bm = torch.randn(bs * s, g * n, generator=gen, dtype=torch.float64)
    c = torch.randn(bs * s, g * n, generator=gen, dtype=torch.float64)
    dt = torch.rand(bs * s, h, generator=gen, dtype=torch.float64) * 0.1
    A = -torch.rand(h, generator=gen, dtype=torch.float64) * 4
    D = torch.rand(h, generator=gen, dtype=torch.float64)
    a = {"batch": bs, "seq": s, "heads": h, "head_dim": p, "state_dim": n, "ngroups": g}
    y = ssd_chunked_program(c, bm, x, dt, A, D, a).reshape(bs, s, h, p)
    for head in range(h):
        gi = head // (h // g)
        xs = x.reshape(bs, s, h, p)[:, :, head].unsqueeze(1)
        Bs = bm.reshape(bs, s, g, n)[:, :, gi].unsqueeze(1)
        Cs = c.reshape(bs, s, g, n)[:, :, gi].unsqueeze(1)
        dts = dt.reshape(bs, s, h)[:, :, head].unsqueeze(1)
        ref = ssd_recurrence(xs, dts * A[head], dts, Bs, Cs)[:, 0] + D[head] * xs[:, 0]
        assert torch.allclose(y[:, :, head], ref, atol=1e-12)


@pytest.mark.parametrize("causal,hk", [(False, 4), (True, 4), (True, 2), (True, 1)])
def test_llama_attention_matches_sdpa(causal, hk):
    from oracle.llama import attention

    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 4, 33, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, hk, 33, 16, generator=g, dtype=torch.float64)
    v = torch.randn(2, hk, 33, 16, generator=g, dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=hk != 4)
    assert torch.allclose(attention(q, k, v, causal), ref, atol=1e-12)


@pytest.mark.parametrize("kv,causal", [(None, False), (2, True)])
def test_llama_oracle_matches_module(kv, causal):
    from oracle.llama import block_forward
    from targets.llama_block import LlamaBlockConfig, build_llama_block

    cfg = LlamaBlockConfig(batch=2, seq=32, hidden=64, heads=4, kv_heads=kv, intermediate=96, causal=causal,
                           dtype=torch.float64)
    m = build_llama_block(cfg, seed=3)
    x = m.example_inputs(seed=4)[0]
    with torch.no_grad():
        ref = m(x)
    w = {k: v for k, v in m.state_dict().items() if not k.startswith(("rope", "attn_bias"))}
    rope = (m.rope_cos, m.rope_sin)  # the module builds its tables in fp32 (reference models/llama_block.py:73-79)
    out = block_forward(x, w, heads=cfg.heads, kv_heads=cfg.n_kv, eps=cfg.eps, theta=cfg.rope_theta, causal=causal,
                        rope=rope)
    assert (out - ref).abs().max() < 1e-12
    from oracle.llama import rope_tables

    c64, s64 = rope_tables(cfg.seq, cfg.head_dim, cfg.rope_theta)
    assert (c64 - m.rope_cos).abs().max() < 1e-5 and (s64 - m.rope_sin).abs().max() < 1e-5


def test_mamba_oracle_matches_module():
    from oracle.mamba import backbone_forward
    from targets.mamba import MambaConfig, build_mamba_model

    cfg = MambaConfig(batch=2, seq=24, d_model=32, expand=2, headdim=16, d_state=8, chunk=8, n_layers=2,
                      ngroups=1, use_conv=True, dtype=torch.float64, a_log_range=(0.0, math.log(16.0)))
    for mode in ("quadratic", "chunked"):
        cfg.mode = mode
        m = build_mamba_model(cfg, seed=5)
        x = m.example_inputs(seed=6)[0]
        with torch.no_grad():
            ref = m(x)
        out = backbone_forward(x, dict(m.state_dict()), cfg)
        assert (out - ref).abs().max() / ref.abs().max() < 1e-10, mode


def test_mamba_oracle_model_forward_matches_embedding_module():
    """Ids -> nn.Embedding rows -> blocks -> tied head, against the oracle (float64);
    a wrong table orientation or a dropped final norm would fail this."""
    from oracle.mamba import model_forward
    from targets.mamba import MambaConfig, build_mamba_model

    cfg = MambaConfig(batch=2, seq=24, d_model=32, expand=2, headdim=16, d_state=8, chunk=8, n_layers=2,
                      ngroups=1, use_conv=True, dtype=torch.float64, a_log_range=(0.0, math.log(16.0)), vocab=97)
    m = build_mamba_model(cfg, seed=5)
    ids = m.example_inputs(seed=6)[0]
    with torch.no_grad():
        ref = m(ids)
    out = model_forward(ids, dict(m.state_dict()), cfg)
    assert out.shape == (2, 24, 97)
    assert (out - ref).abs().max() / ref.abs().max() < 1e-10
    # the first layers alone are the model with fewer blocks
    cfg1 = MambaConfig(**{**cfg.__dict__, "n_layers": 1})
    m1 = build_mamba_model(cfg1, seed=5)
    m1.load_state_dict({k: v for k, v in m.state_dict().items() if not k.startswith("layers.1.")})
    with torch.no_grad():
        ref1 = m1(ids)
    assert (model_forward(ids, dict(m.state_dict()), cfg, layers=1) - ref1).abs().max() < 1e-10
    with pytest.raises(IndexError):
        model_forward(ids.clone().fill_(-1), dict(m.state_dict()), cfg)


def test_interpreters_agree_and_reproduce_reference_check(tmp_path):
    """The oracle interpreter (float64) and the product interpreter (float32) agree on
    the reference's default Llama program; the product one reproduces the recorded check."""
    from oracle import interpret as oi
    from targets.llama_block import build_llama_block
    from torch_helion import CompileConfig, compile_model

    block = build_llama_block()
    x = block.example_inputs()
    res = compile_model(block, x, CompileConfig(run_name="r", results_dir=tmp_path, backend="none"))
    recorded = json.loads((GOLDEN / "llama_block" / "08_reference_check.json").read_text())
    assert res.reference_check["max_rel_err"] == recorded["max_rel_err"]
    from torch_helion.codegen.interpret import program_outputs

    mine = program_outputs(res.program, res.graph.params, list(x))[0]
    ora = oi.program_outputs(res.program, res.graph.params, list(x))[0]
    assert oi.max_rel_err(mine, ora) < 1e-5
    with torch.no_grad():
        eager = block(*x)
    assert abs(oi.max_rel_err(ora, eager) - recorded["max_rel_err"]) < 2e-4


def test_oracle_conv_matches_torch_conv1d():
    from oracle.interpret import conv1d

    g = torch.Generator().manual_seed(7)
    bs, s, c, k = 2, 11, 6, 4
    x = torch.randn(bs * s, c, generator=g, dtype=torch.float64)
    w = torch.randn(c, k, generator=g, dtype=torch.float64)
    y = conv1d(x, w, {"batch": bs, "seq": s, "activation": "silu"})
    xb = x.reshape(bs, s, c).transpose(1, 2)
    ref = F.silu(F.conv1d(F.pad(xb, (k - 1, 0)), w.unsqueeze(1), groups=c)).transpose(1, 2).reshape(bs * s, c)
    assert torch.allclose(y, ref, atol=1e-12)


def test_decode_step_matches_causal_prefill_row_by_row():
    """Decoding tokens 0..S-1 one at a time, each against the cache of the earlier ones,
    reproduces every row of the causal prefill block (GQA, RoPE), and a wrong cache position fails."""
    from oracle.llama import block_forward, decode_step
    from targets.llama_block import LlamaBlockConfig, build_llama_block

    cfg = LlamaBlockConfig(batch=2, seq=12, hidden=64, heads=4, kv_heads=2, intermediate=96, causal=True,
                           dtype=torch.float64, rope_theta=500000.0)
    m = build_llama_block(cfg, seed=4)
    x = m.example_inputs(seed=5)[0]
    w = {k: v for k, v in m.state_dict().items() if not k.startswith(("rope", "attn_bias"))}
    kw = dict(heads=cfg.heads, kv_heads=cfg.n_kv, eps=cfg.eps, theta=cfg.rope_theta)
    ref = block_forward(x, w, causal=True, **kw)
    hd = cfg.head_dim
    kc = torch.zeros(cfg.batch, cfg.seq, cfg.n_kv, hd, dtype=torch.float64)
    vc = torch.zeros_like(kc)
    for t in range(cfg.seq):
        out, kn, vn = decode_step(x[:, t], w, kc, vc, t, **kw)
        assert (out - ref[:, t]).abs().max() < 1e-12, t
        kc[:, t], vc[:, t] = kn, vn
    bad, _, _ = decode_step(x[:, 5], w, kc, vc, 4, **kw)  # planted: cache position off by one
    assert (bad - ref[:, 5]).abs().max() > 1e-3


def _ssd_program_operands(bs, s, h, p, n, pad, seed):
    """Token-major operands of the reference's quadratic ``ssd`` kind (optimizer/evaluate.py:123-138):
    C/B [T, H*N], x [T, H*P], cum/dt padded to ``pad`` columns per head (value in column 0,
    garbage in the rest so a wrong column is caught), a [S, S] mask and D broadcast to [T, H*P]."""
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(bs * s, h * n, generator=g, dtype=torch.float64)
    bm = torch.randn(bs * s, h * n, generator=g, dtype=torch.float64)
    x = torch.randn(bs * s, h * p, generator=g, dtype=torch.float64)
    dt = torch.rand(bs, s, h, generator=g, dtype=torch.float64) * 0.1 + 0.01
    A = -(torch.rand(h, generator=g, dtype=torch.float64) * 15 + 1)
    D = torch.rand(h, generator=g, dtype=torch.float64)
    cum = torch.cumsum(dt * A, dim=1)                                    # running sum over each sequence
    cum_pad = torch.randn(bs, s, h, pad, generator=g, dtype=torch.float64) * 50
    dt_pad = torch.randn(bs, s, h, pad, generator=g, dtype=torch.float64) * 50
    cum_pad[..., 0], dt_pad[..., 0] = cum, dt
    d_full = D.repeat_interleave(p).expand(bs * s, h * p).contiguous()
    return c, bm, x, cum_pad.reshape(bs * s, h * pad), dt_pad.reshape(bs * s, h * pad), d_full, (dt, A, D)


def test_interpret_ssd_quadratic_matches_recurrence():
    """oracle.interpret.ssd_quadratic (the reference's ``ssd`` kind) equals the O(S) recurrence
    (reference tests/test_mamba.py:27-38) when cum = cumsum(dt*A), the mask is the causal tril and
    D repeats per head; a full (non-causal) mask or reading cum from the wrong pad column fails."""
    from oracle.interpret import ssd_quadratic
    from oracle.mamba import ssd_recurrence

    bs, s, h, p, n, pad = 2, 19, 3, 4, 5, 8
    c, bm, x, cum_pad, dt_pad, d_full, (dt, A, D) = _ssd_program_operands(bs, s, h, p, n, pad, seed=11)
    a = {"batch": bs, "seq": s, "heads": h, "head_dim": p, "state_dim": n, "pad": pad}
    mask = torch.ones(s, s, dtype=torch.float64).tril()
    y = ssd_quadratic(c, bm, x, cum_pad, dt_pad, mask, d_full, a)
    x4 = x.reshape(bs, s, h, p).permute(0, 2, 1, 3)
    b4 = bm.reshape(bs, s, h, n).permute(0, 2, 1, 3)
    c4 = c.reshape(bs, s, h, n).permute(0, 2, 1, 3)
    dt3 = dt.permute(0, 2, 1)
    ref = ssd_recurrence(x4, dt3 * A.reshape(1, h, 1), dt3, b4, c4) + x4 * D.reshape(1, h, 1, 1)
    ref = ref.permute(0, 2, 1, 3).reshape(bs * s, h * p)
    assert (y - ref).abs().max() / ref.abs().max() < 1e-10
    # planted mistakes on the checker's inputs must be caught
    full = ssd_quadratic(c, bm, x, cum_pad, dt_pad, torch.ones(s, s, dtype=torch.float64), d_full, a)
    assert (full - ref).abs().max() / ref.abs().max() > 1e-2
    shifted = ssd_quadratic(c, bm, x, cum_pad.roll(1, dims=1), dt_pad, mask, d_full, a)
    assert (shifted - ref).abs().max() / ref.abs().max() > 1e-2


@pytest.mark.parametrize("h,hk,s,skv,causal", [(4, 4, 17, 17, False), (4, 4, 17, 17, True), (8, 2, 17, 17, True),
                                                (8, 1, 13, 13, True), (4, 2, 5, 23, True), (4, 2, 9, 23, False)])
def test_interpret_attention_matches_sdpa(h, hk, s, skv, causal):
    """oracle.interpret.attention on token-major [T, H*d] operands (the ``attention`` kind,
    reference optimizer/evaluate.py:139-146, extended with causal masking, grouped KV heads and
    seq_kv > seq) against torch's scaled_dot_product_attention. For seq_kv > seq the s queries
    are the LAST s positions of a causal sequence of length seq_kv: their rows must equal those
    rows of SDPA's full causal attention over all seq_kv positions (bottom-right alignment)."""
    from oracle.interpret import attention

    bs, d = 2, 16
    g = torch.Generator().manual_seed(h * 100 + hk * 10 + s)
    qf = torch.randn(bs, h, skv, d, generator=g, dtype=torch.float64)
    k = torch.randn(bs, hk, skv, d, generator=g, dtype=torch.float64)
    v = torch.randn(bs, hk, skv, d, generator=g, dtype=torch.float64)
    scale = 1.0 / math.sqrt(d)
    q = qf[:, :, skv - s:]

    def sdpa_rows(k_, v_):
        if causal:
            full = F.scaled_dot_product_attention(qf, k_, v_, is_causal=True, enable_gqa=k_.shape[1] != h, scale=scale)
            return full[:, :, skv - s:]
        return F.scaled_dot_product_attention(q, k_, v_, enable_gqa=k_.shape[1] != h, scale=scale)

    tok = lambda t: t.permute(0, 2, 1, 3).reshape(bs * t.shape[2], t.shape[1] * d)
    a = {"batch": bs, "seq": s, "seq_kv": skv, "heads": h, "kv_heads": hk, "head_dim": d, "scale": scale,
         "causal": causal}
    out = attention(tok(q), tok(k), tok(v), a)
    assert (out - tok(sdpa_rows(k, v))).abs().max() < 1e-12
    if 1 < hk < h:
        # planted: q heads mapped round-robin onto kv heads instead of in blocks of h / hk
        rr = torch.arange(h) % hk
        assert (out - tok(sdpa_rows(k[:, rr], v[:, rr]))).abs().max() > 1e-3
