"""Kernel-level parity: each libth_hip.so entry point vs a torch fp32 CPU reference.

Tolerances: fp32 kernels 1e-4 relative to the output's max magnitude; bf16
kernels 2e-2 max-abs against the fp32 reference computed from the same
(bf16-rounded) inputs, the north-star bound.
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
F32_REL = 1e-4


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / (b.abs().max() + 1e-6))


def _maxabs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float().cpu() - b.float().cpu()).abs().max())


def _rope_tables(seq: int, hd: int, theta: float = 10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    f = torch.outer(torch.arange(seq, dtype=torch.float32), inv)
    e = torch.cat((f, f), -1)
    return e.cos(), e.sin()


def _rot_heads(x: torch.Tensor, hd: int) -> torch.Tensor:
    x4 = x.reshape(*x.shape[:-1], x.shape[-1] // hd, hd)
    h = hd // 2
    return torch.cat((-x4[..., h:], x4[..., :h]), -1).reshape(x.shape)


@pytest.mark.parametrize("M,N,K", [(300, 200, 136), (1024, 256, 512), (8192, 4096, 256)])
def test_gemm_bf16_plain(gpu, M, N, K):
    from torch_helion.hip import abi, ops

    announce(f"gemm bf16 plain M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(K, N, generator=g) * 0.05).bfloat16()
    ref = a.float() @ w.float()
    ad, wd = a.to(gpu), w.to(gpu)
    packed = ops.pack_rhs([wd], torch.bfloat16)
    o16 = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    o32 = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 1, ad, packed, [ops.EpiSpec(abi.EPI_ACC, o16), ops.EpiSpec(abi.EPI_ACC, o32)]))
    torch.cuda.synchronize()
    assert _rel(o32, ref) < 1e-5
    assert _maxabs(o16, ref) < BF16_TOL


@pytest.mark.parametrize("M,N,K,n_acc", [(8200, 4096, 1024, 1), (2000, 768, 4096, 2), (777, 1024, 2048, 4)])
def test_gemm_bf16_deep_k_ragged_m(gpu, M, N, K, n_acc):
    """Many 64-wide K tiles, M not a multiple of the row tile (256-row tiles at 8200 x 4096), RMS fold on."""
    from torch_helion.hip import abi, ops

    announce(f"gemm bf16 deep-K M={M} N={N} K={K} n_acc={n_acc}")
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    ws = [(torch.randn(K, N, generator=g) * 0.02).bfloat16() for _ in range(n_acc)]
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + 1e-5).pow(-0.5)
    xd = x.to(gpu)
    packed = ops.pack_rhs([w.to(gpu) for w in ws], torch.bfloat16)
    outs = [torch.empty(M, N, dtype=torch.float32, device=gpu) for _ in range(n_acc)]
    ss = torch.empty(M, dtype=torch.float32, device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, n_acc, xd, packed, [ops.EpiSpec(abi.EPI_ACC, o, a=i) for i, o in enumerate(outs)],
                          sumsq=True, rscale_mask=(1 << n_acc) - 2, inv_k=1.0 / K, eps=1e-5, sumsq_out=ss))
    torch.cuda.synchronize()
    for i, (o, w) in enumerate(zip(outs, ws)):
        ref = xf @ w.float()
        if i > 0:
            ref = ref * r
        assert _rel(o, ref) < 1e-5, i
    assert _rel(ss, (xf * xf).sum(-1)) < 1e-5


@pytest.mark.parametrize("M,N,K,n_acc,mask", [(2000, 2192, 512, 1, 1), (2048, 2192, 512, 1, 0), (1000, 5000, 256, 1, 1),
                                              (2040, 1100, 512, 2, 2), (2048, 1100, 512, 1, 1), (2000, 700, 512, 1, 1)])
def test_gemm_direct_two_blocks_per_cu(gpu, M, N, K, n_acc, mask):
    """64-row tiles numbering between one and two per CU (288, 288, 320, 288, 288 and 352 tiles of
    64 x 256, 64 x 256, 64 x 256, 64 x 2 x 128, 64 x 128 and 64 x 64) run the direct loop with
    stages within 80 KiB, two workgroups per CU, the row scales kept in the stage memory:
    RMS-scaled and plain accumulators, the sums of squares, a ragged M and N."""
    from torch_helion.hip import abi, ops

    announce(f"gemm bf16 direct two per CU M={M} N={N} K={K} n_acc={n_acc} mask={mask}")
    g = torch.Generator().manual_seed(3 * M + N)
    x = torch.randn(M, K, generator=g).bfloat16()
    ws = [(torch.randn(K, N, generator=g) * 0.03).bfloat16() for _ in range(n_acc)]
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + 1e-5).pow(-0.5)
    packed = ops.pack_rhs([w.to(gpu) for w in ws], torch.bfloat16)
    outs = [torch.empty(M, N, dtype=torch.float32, device=gpu) for _ in range(n_acc)]
    o16 = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    ss = torch.empty(M, dtype=torch.float32, device=gpu)
    epi = [ops.EpiSpec(abi.EPI_ACC, o, a=i) for i, o in enumerate(outs)] + [ops.EpiSpec(abi.EPI_ACC, o16, a=n_acc - 1)]
    ops.gemm(ops.GemmCall(M, N, K, n_acc, x.to(gpu), packed, epi, sumsq=True, rscale_mask=mask, inv_k=1.0 / K,
                          eps=1e-5, sumsq_out=ss))
    torch.cuda.synchronize()
    for i, (o, w) in enumerate(zip(outs, ws)):
        ref = xf @ w.float()
        if (mask >> i) & 1:
            ref = ref * r
        assert _rel(o, ref) < 1e-5, i
        if i == n_acc - 1:
            assert _maxabs(o16, ref) < BF16_TOL
    assert _rel(ss, (xf * xf).sum(-1)) < 1e-5


def test_gemm_bf16_rms_swiglu(gpu):
    from torch_helion.hip import abi, ops

    announce("gemm bf16 n_acc=2 sumsq swiglu")
    M, N, K, eps = 1000, 384, 512, 1e-5
    g = torch.Generator().manual_seed(1)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(K, N, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(K, N, generator=g) * 0.02).bfloat16()
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + eps).pow(-0.5)
    hg, hu = (xf @ wg.float()) * r, (xf @ wu.float()) * r
    ref = hg * torch.sigmoid(hg) * hu
    xd = x.to(gpu)
    packed = ops.pack_rhs([wg.to(gpu), wu.to(gpu)], torch.bfloat16)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    ss = torch.empty(M, dtype=torch.float32, device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 2, xd, packed, [ops.EpiSpec(abi.EPI_SWIGLU, out, a=0, b=1)], sumsq=True,
                          rscale_mask=0b11, inv_k=1.0 / K, eps=eps, sumsq_out=ss))
    torch.cuda.synchronize()
    assert _maxabs(out, ref) < BF16_TOL
    assert _rel(ss, (xf * xf).sum(-1)) < 1e-5


@pytest.mark.parametrize("a,b,mask", [(0, 1, 0b11), (1, 0, 0b01), (0, 1, 0b00)])
def test_gemm_swiglu_register_epilogue(gpu, a, b, mask):
    """The persistent 256-row kernel forms a lone bf16 SWIGLU output from the accumulator
    registers (full tiles) and through the LDS slices otherwise (the ragged last row tile,
    or a second output). Both routes give the same bits, and both match fp32."""
    from torch_helion.hip import abi, ops

    announce(f"gemm swiglu register epilogue a={a} b={b} mask={mask:02b}")
    M, N, K, eps = 2000, 8192, 256, 1e-5     # 8 x 64 tiles of 256 x (2 x 128): persistent, last row tile ragged
    g = torch.Generator().manual_seed(7)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = [(torch.randn(K, N, generator=g) * 0.05).bfloat16() for _ in range(2)]
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + eps).pow(-0.5)
    h = [(xf @ wi.float()) * (r if (mask >> i) & 1 else 1.0) for i, wi in enumerate(w)]
    ref = h[a] * torch.sigmoid(h[a]) * h[b]
    xd = x.to(gpu)
    packed = ops.pack_rhs([wi.to(gpu) for wi in w], torch.bfloat16)
    lone = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    pair = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    copy32 = torch.empty(M, N, dtype=torch.float32, device=gpu)
    kw = dict(sumsq=mask != 0, rscale_mask=mask, inv_k=1.0 / K, eps=eps)
    ops.gemm(ops.GemmCall(M, N, K, 2, xd, packed, [ops.EpiSpec(abi.EPI_SWIGLU, lone, a=a, b=b)], **kw))
    ops.gemm(ops.GemmCall(M, N, K, 2, xd, packed, [ops.EpiSpec(abi.EPI_SWIGLU, pair, a=a, b=b),
                                                   ops.EpiSpec(abi.EPI_SWIGLU, copy32, a=a, b=b)], **kw))
    torch.cuda.synchronize()
    assert torch.equal(lone, pair)
    assert torch.equal(pair, copy32.bfloat16())
    # (outputs up to ~16 here: one bf16 rounding is up to 2^-9 of the value, so the bar is relative)
    assert _rel(lone, ref) < 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_qkv_rope(gpu, dtype):
    """QKV with the RMS fold and RoPE: fused rotation vs the pre-rotated accumulator."""
    from torch_helion.hip import abi, ops

    announce(f"gemm qkv rope {dtype}")
    B, S, H, hd, K, eps = 2, 96, 4, 64, 256, 1e-6
    M, N = B * S, H * hd
    g = torch.Generator().manual_seed(2)
    x = torch.randn(M, K, generator=g).to(dtype)
    wq, wk, wv = [(torch.randn(K, N, generator=g) * 0.05).to(dtype) for _ in range(3)]
    cos, sin = _rope_tables(S, hd)
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + eps).pow(-0.5)
    q, k, v = [(xf @ w.float()) * r for w in (wq, wk, wv)]
    cf, sf = cos.repeat(B, H), sin.repeat(B, H)
    q_ref = q * cf + _rot_heads(q, hd) * sf
    k_ref = k * cf + _rot_heads(k, hd) * sf
    xd = x.to(gpu)
    packed = ops.pack_rhs([w.to(gpu) for w in (wq, wk, wv)], dtype)
    wkr = _rot_heads(wk.float(), hd).contiguous().to(dtype)  # W @ R: rotate W's output columns
    packed2 = ops.pack_rhs([wk.to(gpu), wkr.to(gpu)], dtype)
    oq, ok, ov, ok2 = [torch.empty(M, N, dtype=dtype, device=gpu) for _ in range(4)]
    cd, sd = cos.to(gpu).contiguous(), sin.to(gpu).contiguous()
    common = dict(sumsq=True, inv_k=1.0 / K, eps=eps, rope_cos=cd, rope_sin=sd, rope_head_dim=hd, rope_period=S)
    ops.gemm(ops.GemmCall(M, N, K, 3, xd, packed, [ops.EpiSpec(abi.EPI_ROPE, oq, a=0), ops.EpiSpec(abi.EPI_ROPE, ok, a=1),
                                                    ops.EpiSpec(abi.EPI_ACC, ov, a=2)], rscale_mask=0b111, **common))
    ops.gemm(ops.GemmCall(M, N, K, 2, xd, packed2, [ops.EpiSpec(abi.EPI_ROPE_PAIR, ok2, a=0, b=1)], rscale_mask=0b11, **common))
    torch.cuda.synchronize()
    if dtype == torch.float32:
        for o, ref in ((oq, q_ref), (ok, k_ref), (ov, v), (ok2, k_ref)):
            assert _rel(o, ref) < F32_REL
    else:
        for o, ref in ((oq, q_ref), (ok, k_ref), (ov, v), (ok2, k_ref)):
            assert _maxabs(o, ref) < BF16_TOL


@pytest.mark.parametrize("hd,n_acc", [(128, 1), (64, 2)])
def test_gemm_rope_whole_heads_per_wave(gpu, hd, n_acc):
    """Fused RoPE where every wave's column half holds whole heads (the q-projection shape class),
    with the RMS fold, a table period shorter than M, and bf16 + fp32 outputs of the same op."""
    from torch_helion.hip import abi, ops

    announce(f"gemm bf16 rope hd={hd} n_acc={n_acc}")
    B, S, H, K, eps = 4, 250, 8, 512, 1e-5
    M, N = B * S, H * hd
    g = torch.Generator().manual_seed(hd + n_acc)
    x = torch.randn(M, K, generator=g).bfloat16()
    ws = [(torch.randn(K, N, generator=g) * 0.05).bfloat16() for _ in range(n_acc)]
    cos, sin = _rope_tables(S, hd, theta=500000.0)
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + eps).pow(-0.5)
    accs = [(xf @ w.float()) * r for w in ws]
    cf, sf = cos.repeat(B, H), sin.repeat(B, H)
    refs = [a * cf + _rot_heads(a, hd) * sf for a in accs]
    xd = x.to(gpu)
    packed = ops.pack_rhs([w.to(gpu) for w in ws], torch.bfloat16)
    o16 = [torch.empty(M, N, dtype=torch.bfloat16, device=gpu) for _ in range(n_acc)]
    o32 = [torch.empty(M, N, dtype=torch.float32, device=gpu) for _ in range(n_acc)]
    outs = [ops.EpiSpec(abi.EPI_ROPE, o, a=i) for i, o in enumerate(o16)] + \
           [ops.EpiSpec(abi.EPI_ROPE, o, a=i) for i, o in enumerate(o32)]
    ops.gemm(ops.GemmCall(M, N, K, n_acc, xd, packed, outs, sumsq=True, rscale_mask=(1 << n_acc) - 1,
                          inv_k=1.0 / K, eps=eps, rope_cos=cos.to(gpu).contiguous(), rope_sin=sin.to(gpu).contiguous(),
                          rope_head_dim=hd, rope_period=S))
    torch.cuda.synchronize()
    for i, ref in enumerate(refs):
        assert _rel(o32[i], ref) < 1e-5, i
        assert _maxabs(o16[i], ref) < BF16_TOL, i


@pytest.mark.parametrize("S", [512, 2048])
def test_gemm_kv_rope_head_wider_than_half_tile(gpu, S):
    """k and v projections in one launch (two accumulators, 128-column tiles) with RoPE on k at head_dim 128:
    a head spans both column halves of the tile, so each wave holds one whole accumulator instead. M = 8 S
    rows selects 128-row (S=512) and 256-row (S=2048) persistent tiles. RMS fold on both accumulators."""
    from torch_helion.hip import abi, ops

    B, Hkv, hd, K, eps = 8, 8, 128, 512, 1e-5
    M, N = B * S, Hkv * hd
    announce(f"gemm bf16 kv rope M={M} N={N} hd={hd}")
    g = torch.Generator().manual_seed(S)
    x = torch.randn(M, K, generator=g).bfloat16()
    wk, wv = [(torch.randn(K, N, generator=g) * 0.05).bfloat16() for _ in range(2)]
    cos, sin = _rope_tables(S, hd, theta=500000.0)
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + eps).pow(-0.5)
    k_acc, v_ref = (xf @ wk.float()) * r, (xf @ wv.float()) * r
    k_ref = k_acc * cos.repeat(B, Hkv) + _rot_heads(k_acc, hd) * sin.repeat(B, Hkv)
    xd = x.to(gpu)
    packed = ops.pack_rhs([wk.to(gpu), wv.to(gpu)], torch.bfloat16)
    ok, ov = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu) for _ in range(2)]
    ok32 = torch.full((M, N), float("nan"), device=gpu)
    ss = torch.full((M,), float("nan"), device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 2, xd, packed, [ops.EpiSpec(abi.EPI_ROPE, ok, a=0), ops.EpiSpec(abi.EPI_ACC, ov, a=1),
                                                    ops.EpiSpec(abi.EPI_ROPE, ok32, a=0)],
                          sumsq=True, rscale_mask=0b11, inv_k=1.0 / K, eps=eps, sumsq_out=ss,
                          rope_cos=cos.to(gpu).contiguous(), rope_sin=sin.to(gpu).contiguous(), rope_head_dim=hd,
                          rope_period=S))
    torch.cuda.synchronize()
    assert _rel(ok32, k_ref) < 1e-5
    assert _maxabs(ok, k_ref) < BF16_TOL
    assert _maxabs(ov, v_ref) < BF16_TOL
    assert _rel(ss, (xf * xf).sum(-1)) < 1e-5


def _quant_e4m3(w: torch.Tensor):
    """Per-output-channel e4m3: s_n = max|W[:, n]| / 448, q = e4m3(W / s_n)."""
    s = (w.abs().amax(0).clamp_min(1e-12) / 448.0).float()
    q = (w / s).to(torch.float8_e4m3fn)
    return q, s


@pytest.mark.parametrize("M,N,K,case", [(64, 4096, 4096, "add"), (64, 1024, 4096, "rope_kv"),
                                        (37, 2048, 1024, "swiglu"), (100, 512, 512, "acc"),
                                        (16, 1024, 2048, "add"), (20, 256, 992, "acc"),
                                        (64, 14336, 512, "swiglu"), (32, 24576, 256, "rope_q"),
                                        (64, 1024, 4096, "rope_qk")])
def test_gemm_fp8_weights(gpu, M, N, K, case):
    """bf16 activations x e4m3 weights with per-column scales (the decode projections), split-K,
    against fp32 math on the dequantised weights. K a multiple of 128 takes the shared-activation
    kernel (32-, 64- and 128-row variants here); K = 992 the per-wave split-K kernel. The two
    widest cases run as one split whose workgroups finish their tiles themselves (SwiGLU pairs
    and RoPE partners inside a tile); the others go through the reduce pass. rope_qk rotates
    both accumulators over the same columns: each output takes its own accumulator's partner."""
    from torch_helion.hip import abi, ops

    announce(f"gemm fp8 weights M={M} N={N} K={K} {case}")
    g = torch.Generator().manual_seed(M + N + K)
    n_acc = {"add": 1, "rope_kv": 2, "swiglu": 2, "acc": 1, "rope_q": 1, "rope_qk": 2}[case]
    x = torch.randn(M, K, generator=g).bfloat16()
    qs = [_quant_e4m3(torch.randn(K, N, generator=g) * 0.02) for _ in range(n_acc)]
    wdq = [q.float() * s[None, :] for q, s in qs]
    xf = x.float()
    accs = [xf @ w for w in wdq]
    kw = {}
    if case in ("rope_kv", "swiglu", "rope_q", "rope_qk"):
        r = ((xf * xf).sum(-1, keepdim=True) / K + 1e-5).pow(-0.5)
        accs = [a * r for a in accs]
        kw = dict(sumsq=True, rscale_mask=(1 << n_acc) - 1, inv_k=1.0 / K, eps=1e-5)
    extras, outs32 = [], []
    if case == "add":
        res = torch.randn(M, N, generator=g)
        refs = [accs[0] + res]
        extras = [res.to(gpu)]
        ops_ = [(abi.EPI_ADD, 0, -1, 0)]
    elif case == "rope_kv":
        hd, pos = 128, 4096
        cos, sin = _rope_tables(pos + 1, hd, theta=500000.0)
        c1, s1 = cos[pos:pos + 1].contiguous(), sin[pos:pos + 1].contiguous()
        refs = [accs[0] * c1.repeat(M, N // hd) + _rot_heads(accs[0], hd) * s1.repeat(M, N // hd), accs[1]]
        kw.update(rope_cos=c1.to(gpu), rope_sin=s1.to(gpu), rope_head_dim=hd, rope_period=1)
        ops_ = [(abi.EPI_ROPE, 0, -1, -1), (abi.EPI_ACC, 1, -1, -1)]
    elif case == "rope_qk":
        hd, pos = 128, 300
        cos, sin = _rope_tables(pos + 1, hd, theta=500000.0)
        c1, s1 = cos[pos:pos + 1].contiguous(), sin[pos:pos + 1].contiguous()
        refs = [a * c1.repeat(M, N // hd) + _rot_heads(a, hd) * s1.repeat(M, N // hd) for a in accs]
        kw.update(rope_cos=c1.to(gpu), rope_sin=s1.to(gpu), rope_head_dim=hd, rope_period=1)
        ops_ = [(abi.EPI_ROPE, 0, -1, -1), (abi.EPI_ROPE, 1, -1, -1)]
    elif case == "rope_q":
        hd, pos = 128, 77
        cos, sin = _rope_tables(pos + 1, hd, theta=10000.0)
        c1, s1 = cos[pos:pos + 1].contiguous(), sin[pos:pos + 1].contiguous()
        refs = [accs[0] * c1.repeat(M, N // hd) + _rot_heads(accs[0], hd) * s1.repeat(M, N // hd)]
        kw.update(rope_cos=c1.to(gpu), rope_sin=s1.to(gpu), rope_head_dim=hd, rope_period=1)
        ops_ = [(abi.EPI_ROPE, 0, -1, -1)]
    elif case == "swiglu":
        refs = [accs[0] * torch.sigmoid(accs[0]) * accs[1]]
        ops_ = [(abi.EPI_SWIGLU, 0, 1, -1)]
    else:
        refs = [accs[0]]
        ops_ = [(abi.EPI_ACC, 0, -1, -1)]
    packed = ops.pack_rhs([q.to(gpu) for q, _ in qs], torch.float8_e4m3fn)
    scale = torch.stack([s for _, s in qs]).to(gpu).contiguous()
    ws = torch.empty(ops.gemm_workspace_bytes(M, N, K, n_acc, torch.float8_e4m3fn), dtype=torch.uint8, device=gpu)
    o16 = [torch.empty(M, N, dtype=torch.bfloat16, device=gpu) for _ in ops_]
    o32 = [torch.empty(M, N, device=gpu) for _ in ops_]
    specs = [ops.EpiSpec(op, o, a=a, b=b, e=e) for (op, a, b, e), o in zip(ops_, o16)] + \
            [ops.EpiSpec(op, o, a=a, b=b, e=e) for (op, a, b, e), o in zip(ops_, o32)]
    ops.gemm(ops.GemmCall(M, N, K, n_acc, x.to(gpu), packed, specs, extras=extras, in_dtype=torch.float8_e4m3fn,
                          rhs_scale=scale, workspace=ws, **kw))
    torch.cuda.synchronize()
    for i, ref in enumerate(refs):
        assert _rel(o32[i], ref) < 1e-4, (case, i, _rel(o32[i], ref))
        assert _maxabs(o16[i], ref) < BF16_TOL, (case, i)


@pytest.mark.parametrize("M,N,K,n_acc", [(64, 6144, 4096, 1), (64, 14336, 4096, 2), (17, 1024, 8192, 1),
                                         (100, 512, 512, 1), (64, 2048, 992, 2)])
def test_gemm_fp8_lhs_gain(gpu, M, N, K, n_acc):
    """e4m3 weights with the RMSNorm gain on the activation side (lhs_gain): outputs are
    r * ((x * g) @ (q s)) with r from the UNSCALED rows, against fp32 math. Covers the
    shared-activation kernel with several splits (q|k|v), one split finishing in the kernel
    (gate/up), a K over the gain staging's 4096 (forced extra splits), the 128-row variant and the
    per-wave split-K kernel (K = 992). A gain applied twice, or a sum of squares of the scaled
    rows, would miss by far more than the tolerance (g ranges over 0.5..1.5)."""
    from torch_helion.hip import abi, ops

    announce(f"gemm fp8 lhs_gain M={M} N={N} K={K} n_acc={n_acc}")
    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    gain = torch.rand(K, generator=g) + 0.5
    qs = [_quant_e4m3(torch.randn(K, N, generator=g) * 0.02) for _ in range(n_acc)]
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + 1e-5).pow(-0.5)
    xg = (xf * gain).bfloat16().float()                  # the staged operand is bf16(x * g)
    accs = [(xg @ (q.float() * s[None, :])) * r for q, s in qs]
    ref = accs[0] * torch.sigmoid(accs[0]) * accs[1] if n_acc == 2 else accs[0]
    op = abi.EPI_SWIGLU if n_acc == 2 else abi.EPI_ACC
    packed = ops.pack_rhs([q.to(gpu) for q, _ in qs], torch.float8_e4m3fn)
    scale = torch.stack([s for _, s in qs]).to(gpu).contiguous()
    ws = torch.empty(ops.gemm_workspace_bytes(M, N, K, n_acc, torch.float8_e4m3fn), dtype=torch.uint8, device=gpu)
    o32 = torch.full((M, N), float("nan"), device=gpu)
    ss = torch.empty(M, device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, n_acc, x.to(gpu), packed, [ops.EpiSpec(op, o32, a=0, b=1 if n_acc == 2 else -1)],
                          in_dtype=torch.float8_e4m3fn, rhs_scale=scale, workspace=ws, sumsq=True,
                          rscale_mask=(1 << n_acc) - 1, inv_k=1.0 / K, eps=1e-5, lhs_gain=gain.to(gpu), sumsq_out=ss))
    torch.cuda.synchronize()
    assert _rel(o32, ref) < 1e-4, _rel(o32, ref)
    assert _rel(ss, (xf * xf).sum(-1)) < 1e-5


@pytest.mark.parametrize("M,N,K", [(64, 4096, 4096), (37, 2048, 1024), (32, 24576, 256)])
def test_gemm_fp8_gain_out_and_rs_parts(gpu, M, N, K):
    """The next RMSNorm's gain applied by an e4m3 GEMM's finishing pass (gain_out: the decode
    step's o-projection feeding gate/up) and consumed through rs_parts. Producer: the gained
    output is bit-for-bit bf16(bf16(v) * g) of the plain call's output, the fp32 output is
    unchanged, and each 256-column part is that slice's sum of bf16(v)^2. Consumer: a SwiGLU
    GEMM on the gained rows with rs_parts matches the lhs_gain path on the plain rows. Covers
    8 and 2 splits and one split (which gain_out sends through the reduce pass), and consumers
    finishing in the main kernel and in the reduce pass."""
    from torch_helion.hip import abi, ops

    announce(f"gemm fp8 gain_out + rs_parts M={M} N={N} K={K}")
    f8 = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(M + 3 * N + K)
    x = torch.randn(M, K, generator=g).bfloat16().to(gpu)
    res = torch.randn(M, N, generator=g).bfloat16().to(gpu)
    gain = (torch.rand(N, generator=g) + 0.5).to(gpu)
    q, s = _quant_e4m3(torch.randn(K, N, generator=g) * 0.02)
    packed = ops.pack_rhs([q.to(gpu)], f8)
    scale = s[None, :].to(gpu).contiguous()
    ws = torch.empty(ops.gemm_workspace_bytes(M, N, K, 1, f8), dtype=torch.uint8, device=gpu)

    def produce(gain_out):
        o16 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        o32 = torch.full((M, N), float("nan"), device=gpu)
        ops.gemm(ops.GemmCall(M, N, K, 1, x, packed, [ops.EpiSpec(abi.EPI_ADD, o16, e=0),
                                                      ops.EpiSpec(abi.EPI_ADD, o32, e=0)],
                              extras=[res], in_dtype=f8, rhs_scale=scale, workspace=ws, gain_out=gain_out))
        torch.cuda.synchronize()
        return o16, o32

    plain16, plain32 = produce(None)
    parts = torch.full((M, N // 256), float("nan"), device=gpu)
    gained16, gained32 = produce((0, gain, parts))
    ref32 = x.float().cpu() @ (q.float() * s[None, :]) + res.float().cpu()
    assert _rel(plain32, ref32) < 1e-4
    assert torch.equal(gained32, plain32)
    assert torch.equal(gained16, (plain16.float() * gain).bfloat16())
    sq = plain16.double() ** 2
    want = sq.view(M, N // 256, 256).sum(-1)
    assert ((parts.double() - want).abs() / want).max().item() < 1e-5

    # consumer: gate/up on the gained rows with the producer's row sums (the C5 width runs as one
    # split finished in the main kernel; 512 columns through the reduce pass)
    F = 14336 if N == 4096 else 512
    qs = [_quant_e4m3(torch.randn(N, F, generator=g) * 0.02) for _ in range(2)]
    pk2 = ops.pack_rhs([qq.to(gpu) for qq, _ in qs], f8)
    sc2 = torch.stack([ss for _, ss in qs]).to(gpu).contiguous()
    ws2 = torch.empty(ops.gemm_workspace_bytes(M, F, N, 2, f8), dtype=torch.uint8, device=gpu)
    norm = dict(sumsq=True, rscale_mask=0b11, inv_k=1.0 / N, eps=1e-5)
    outs = []
    for lhs, kw in ((plain16, dict(lhs_gain=gain)), (gained16, dict(rs_parts=parts))):
        o = torch.full((M, F), float("nan"), device=gpu)
        ss = torch.full((M,), float("nan"), device=gpu)
        ops.gemm(ops.GemmCall(M, F, N, 2, lhs, pk2, [ops.EpiSpec(abi.EPI_SWIGLU, o, a=0, b=1)], in_dtype=f8,
                              rhs_scale=sc2, workspace=ws2, sumsq_out=ss, **norm, **kw))
        torch.cuda.synchronize()
        outs.append((o, ss))
    (o_a, ss_a), (o_b, ss_b) = outs
    assert _rel(ss_b, ss_a) < 1e-6, _rel(ss_b, ss_a)
    assert _rel(o_b, o_a) < 1e-5, _rel(o_b, o_a)


def test_gemm_gain_out_rejected_for_bf16(gpu):
    """gain_out exists for e4m3 weights only: a bf16 GEMM asked for it fails loudly."""
    from torch_helion.hip import abi, ops

    x = torch.randn(64, 256, device=gpu).bfloat16()
    packed = ops.pack_rhs([torch.randn(256, 1024, device=gpu).bfloat16()], torch.bfloat16)
    out = torch.empty(64, 1024, dtype=torch.bfloat16, device=gpu)
    parts = torch.empty(64, 4, device=gpu)
    with pytest.raises(abi.HipBackendError, match="gain_out"):
        ops.gemm(ops.GemmCall(64, 1024, 256, 1, x, packed, [ops.EpiSpec(abi.EPI_ACC, out, a=0)],
                              gain_out=(0, torch.ones(1024, device=gpu), parts)))


def test_gemm_lhs_gain_rejected_for_bf16(gpu):
    """lhs_gain exists for e4m3 weights only: a bf16 GEMM asked for it fails loudly."""
    from torch_helion.hip import abi, ops

    x = torch.randn(64, 256, device=gpu).bfloat16()
    packed = ops.pack_rhs([torch.randn(256, 128, device=gpu).bfloat16()], torch.bfloat16)
    out = torch.empty(64, 128, device=gpu)
    with pytest.raises(abi.HipBackendError, match="lhs_gain"):
        ops.gemm(ops.GemmCall(64, 128, 256, 1, x, packed, [ops.EpiSpec(abi.EPI_ACC, out, a=0)],
                              lhs_gain=torch.ones(256, device=gpu)))


@pytest.mark.parametrize("M,N,K", [(64, 2048, 1024), (32, 24576, 256)])
def test_gemm_fp8_column_windows(gpu, M, N, K):
    """e4m3 weights, one accumulator split into column-window outputs (the merged q | k | v
    projection of the decode step): RoPE on the first half, add-extra on the second (the extra
    read at the window-relative column). N = 2048 goes through the reduce pass, N = 24576 is a
    single split finished inside the main kernel."""
    from torch_helion.hip import abi, ops

    announce(f"gemm fp8 column windows M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    q, s = _quant_e4m3(torch.randn(K, N, generator=g) * 0.02)
    acc = x.float() @ (q.float() * s[None, :])
    hd, pos, h = 128, 9, N // 2
    cos, sin = _rope_tables(pos + 1, hd, theta=10000.0)
    c1, s1 = cos[pos:pos + 1].contiguous(), sin[pos:pos + 1].contiguous()
    a0 = acc[:, :h]
    ref0 = a0 * c1.repeat(M, h // hd) + _rot_heads(a0, hd) * s1.repeat(M, h // hd)
    extra = torch.randn(M, N - h, generator=g)
    ref1 = acc[:, h:] + extra
    packed = ops.pack_rhs([q.to(gpu)], torch.float8_e4m3fn)
    ws = torch.empty(ops.gemm_workspace_bytes(M, N, K, 1, torch.float8_e4m3fn), dtype=torch.uint8, device=gpu)
    o0 = torch.full((M, h), float("nan"), device=gpu)
    o1 = torch.full((M, N - h), float("nan"), device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 1, x.to(gpu), packed,
                          [ops.EpiSpec(abi.EPI_ROPE, o0, a=0, cols=(0, h)),
                           ops.EpiSpec(abi.EPI_ADD, o1, a=0, e=0, cols=(h, N))],
                          extras=[extra.to(gpu)], in_dtype=torch.float8_e4m3fn, rhs_scale=s[None, :].to(gpu).contiguous(),
                          workspace=ws, rope_cos=c1.to(gpu), rope_sin=s1.to(gpu), rope_head_dim=hd, rope_period=1))
    torch.cuda.synchronize()
    assert _rel(o0, ref0) < 1e-4 and _rel(o1, ref1) < 1e-4, (_rel(o0, ref0), _rel(o1, ref1))


def test_gemm_fp8_workspace_reuse(gpu):
    """One workspace, holding garbage (0xff bytes: NaN floats) to begin with, serves fp8 calls
    of different shapes in any order: no call depends on what an earlier one left in it."""
    from torch_helion.hip import abi, ops

    announce("gemm fp8 shared workspace A B A B")
    g = torch.Generator().manual_seed(11)
    shapes = [(64, 1024, 2048, 1), (48, 512, 1024, 2)]
    cases = []
    for M, N, K, n_acc in shapes:
        x = torch.randn(M, K, generator=g).bfloat16()
        qs = [_quant_e4m3(torch.randn(K, N, generator=g) * 0.02) for _ in range(n_acc)]
        accs = [x.float() @ (q.float() * s[None, :]) for q, s in qs]
        packed = ops.pack_rhs([q.to(gpu) for q, _ in qs], torch.float8_e4m3fn)
        scale = torch.stack([s for _, s in qs]).to(gpu).contiguous()
        outs = [torch.empty(M, N, device=gpu) for _ in range(n_acc)]
        cases.append((M, N, K, n_acc, x.to(gpu), packed, scale, outs, accs))
    nbytes = max(ops.gemm_workspace_bytes(M, N, K, n_acc, torch.float8_e4m3fn) for M, N, K, n_acc in shapes)
    ws = torch.full((nbytes,), 255, dtype=torch.uint8, device=gpu)
    for rep in range(2):
        for M, N, K, n_acc, x, packed, scale, outs, accs in cases:
            for o in outs:
                o.fill_(float("nan"))
            specs = [ops.EpiSpec(abi.EPI_ACC, o, a=i) for i, o in enumerate(outs)]
            ops.gemm(ops.GemmCall(M, N, K, n_acc, x, packed, specs, in_dtype=torch.float8_e4m3fn,
                                  rhs_scale=scale, workspace=ws))
            torch.cuda.synchronize()
            for o, ref in zip(outs, accs):
                assert _rel(o, ref) < 1e-4, (rep, M, N, K)


def test_gemm_extra_ops(gpu):
    from torch_helion.hip import abi, ops

    announce("gemm bf16 add/softplus/mul extras")
    M, N, K = 513, 160, 64
    g = torch.Generator().manual_seed(3)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(K, N, generator=g) * 0.1).bfloat16()
    e0 = torch.randn(M, N, generator=g).bfloat16()
    e1 = torch.randn(M, N, generator=g).float()
    acc = a.float() @ w.float()
    ad = a.to(gpu)
    packed = ops.pack_rhs([w.to(gpu)], torch.bfloat16)
    o = [torch.empty(M, N, dtype=torch.bfloat16, device=gpu) for _ in range(3)]
    o.append(torch.empty(M, N, dtype=torch.float32, device=gpu))
    ops.gemm(ops.GemmCall(M, N, K, 1, ad, packed,
                          [ops.EpiSpec(abi.EPI_ADD, o[0], e=0), ops.EpiSpec(abi.EPI_SOFTPLUS_ADD, o[1], e=1),
                           ops.EpiSpec(abi.EPI_MUL, o[2], e=1), ops.EpiSpec(abi.EPI_SILU, o[3])],
                          extras=[e0.to(gpu), e1.to(gpu)]))
    torch.cuda.synchronize()
    assert _maxabs(o[0], acc + e0.float()) < BF16_TOL
    assert _maxabs(o[1], torch.log(1 + torch.exp(acc + e1))) < BF16_TOL
    assert _maxabs(o[2], acc * e1) < BF16_TOL
    assert _rel(o[3], acc * torch.sigmoid(acc)) < 1e-5


@pytest.mark.parametrize("M", [16384, 16300])
def test_gemm_whole_wave_wide_tiles(gpu, M):
    """One accumulator over 1024 columns at 64 row tiles of 256: exactly one wave of
    256 x 256 tiles on a 256-CU device, the tile th_gemm then takes instead of two
    256 x 128 tiles per CU (the Mamba-2 out-projection with its fp32 residual; a ragged
    last row tile in the second case)."""
    from torch_helion.hip import abi, ops

    announce(f"gemm bf16 whole-wave 256x256 tiles M={M}")
    N, K = 1024, 2048
    g = torch.Generator().manual_seed(M)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(K, N, generator=g) * 0.03).bfloat16()
    res = torch.randn(M, N, generator=g)
    ref = a.float() @ w.float() + res
    packed = ops.pack_rhs([w.to(gpu)], torch.bfloat16)
    o16 = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    o32 = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 1, a.to(gpu), packed,
                          [ops.EpiSpec(abi.EPI_ADD, o16, e=0), ops.EpiSpec(abi.EPI_ADD, o32, e=0)],
                          extras=[res.to(gpu)]))
    torch.cuda.synchronize()
    assert _rel(o32, ref) < 1e-5
    assert _maxabs(o16, ref) < 4 * BF16_TOL   # |ref| up to ~8: bf16 rounding of the output itself
    assert _rel(o16, ref) < 1e-2


@pytest.mark.parametrize("M,N,K,case", [(128, 1376, 512, "add"), (128, 1376, 512, "rms_swiglu"),
                                         (100, 200, 136, "acc"), (77, 96, 1380, "add"), (4096, 512, 256, "add")])
def test_gemm_f32_small(gpu, M, N, K, case):
    """fp32 GEMMs: small grids (the C1 shapes, ragged rows, K not a multiple of 8, a long K) on
    the 32-row split-K kernel, and a grid that fills the GPU on the 64-row kernel."""
    from torch_helion.hip import abi, ops

    announce(f"gemm f32 M={M} N={N} K={K} {case}")
    g = torch.Generator().manual_seed(4)
    a = torch.randn(M, K, generator=g)
    n_acc = 2 if case == "rms_swiglu" else 1
    w = [torch.randn(K, N, generator=g) * 0.02 for _ in range(n_acc)]
    res = torch.randn(M, N, generator=g)
    packed = ops.pack_rhs([wi.to(gpu) for wi in w], torch.float32)
    out = torch.empty(M, N, device=gpu)
    kw = {}
    if case == "add":
        ref = res + a @ w[0]
        epi = [ops.EpiSpec(abi.EPI_ADD, out, e=0)]
        kw["extras"] = [res.to(gpu)]
    elif case == "acc":
        ref = a @ w[0]
        epi = [ops.EpiSpec(abi.EPI_ACC, out)]
    else:
        r = ((a * a).sum(-1, keepdim=True) / K + 1e-5).pow(-0.5)
        hg, hu = (a @ w[0]) * r, (a @ w[1]) * r
        ref = hg * torch.sigmoid(hg) * hu
        epi = [ops.EpiSpec(abi.EPI_SWIGLU, out, a=0, b=1)]
        kw.update(sumsq=True, rscale_mask=0b11, inv_k=1.0 / K, eps=1e-5)
    ops.gemm(ops.GemmCall(M, N, K, n_acc, a.to(gpu), packed, epi, **kw))
    torch.cuda.synchronize()
    assert _rel(out, ref) < F32_REL
    # with a workspace, small grids split K over workgroups (a second pass sums the slices)
    nb = ops.gemm_workspace_bytes(M, N, K, n_acc, torch.float32)
    assert (nb > 0) == (M < 1024), nb
    if nb:
        ws = torch.full((nb,), 255, dtype=torch.uint8, device=gpu)   # stale contents must not matter
        out2 = torch.empty_like(out)
        epi2 = [ops.EpiSpec(e.op, out2, a=e.a, b=e.b, e=e.e) for e in epi]
        ops.gemm(ops.GemmCall(M, N, K, n_acc, a.to(gpu), packed, epi2, workspace=ws, **kw))
        torch.cuda.synchronize()
        assert _rel(out2, ref) < F32_REL


def _attn_ref(q, k, v, B, S, Hq, Hkv, hd, scale, causal):
    q4 = q.float().reshape(B, S, Hq, hd).transpose(1, 2)
    k4 = k.float().reshape(B, S, Hkv, hd).transpose(1, 2).repeat_interleave(Hq // Hkv, dim=1)
    v4 = v.float().reshape(B, S, Hkv, hd).transpose(1, 2).repeat_interleave(Hq // Hkv, dim=1)
    s = (q4 @ k4.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    return (torch.softmax(s, -1) @ v4).transpose(1, 2).reshape(B * S, Hq * hd)


@pytest.mark.parametrize("B,S,Hq,Hkv,hd,causal", [(2, 200, 4, 2, 128, True), (1, 256, 8, 8, 64, False),
                                                  (2, 384, 8, 2, 128, False), (1, 130, 4, 1, 64, True),
                                                  (8, 320, 8, 2, 128, True), (1, 1100, 4, 1, 128, True),
                                                  (2, 700, 4, 4, 64, False)])
def test_attention_bf16(gpu, B, S, Hq, Hkv, hd, causal):
    from torch_helion.hip import ops

    announce(f"attention bf16 B={B} S={S} Hq={Hq} Hkv={Hkv} hd={hd} causal={causal}")
    g = torch.Generator().manual_seed(S + hd)
    q = torch.randn(B * S, Hq * hd, generator=g).bfloat16()
    k = torch.randn(B * S, Hkv * hd, generator=g).bfloat16()
    v = torch.randn(B * S, Hkv * hd, generator=g).bfloat16()
    scale = hd ** -0.5
    ref = _attn_ref(q, k, v, B, S, Hq, Hkv, hd, scale, causal)
    out = torch.empty(B * S, Hq * hd, dtype=torch.bfloat16, device=gpu)
    ops.attention_prefill(q.to(gpu), k.to(gpu), v.to(gpu), out, batch=B, seq_q=S, seq_kv=S, heads_q=Hq, heads_kv=Hkv,
                          head_dim=hd, scale=scale, causal=causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert _maxabs(out, ref) < BF16_TOL


@pytest.mark.parametrize("B,S,Hq,Hkv,hd,causal", [(1, 128, 8, 8, 64, True), (2, 200, 4, 2, 128, True),
                                                  (1, 77, 4, 1, 64, False), (2, 33, 2, 2, 32, True),
                                                  (1, 700, 2, 1, 128, False), (1, 300, 2, 2, 64, True)])
def test_attention_f32(gpu, B, S, Hq, Hkv, hd, causal):
    """fp32 prefill attention: the matrix-core kernel (head_dim 64/128; C1 is the first case),
    ragged query and key blocks, grouped KV heads, and the scalar kernel (head_dim 32). The
    matrix-core kernel deals a query block's key blocks over four waves and merges them: query
    blocks with fewer key blocks than waves (causal), and with several per wave (S = 700)."""
    from torch_helion.hip import ops

    announce(f"attention f32 B={B} S={S} Hq={Hq} Hkv={Hkv} hd={hd} causal={causal}")
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B * S, Hq * hd, generator=g)
    k, v = [torch.randn(B * S, Hkv * hd, generator=g) for _ in range(2)]
    ref = _attn_ref(q, k, v, B, S, Hq, Hkv, hd, hd ** -0.5, causal)
    out = torch.empty(B * S, Hq * hd, device=gpu)
    ops.attention_prefill(q.to(gpu), k.to(gpu), v.to(gpu), out, batch=B, seq_q=S, seq_kv=S, heads_q=Hq,
                          heads_kv=Hkv, head_dim=hd, scale=hd ** -0.5, causal=causal)
    torch.cuda.synchronize()
    assert _rel(out, ref) < F32_REL


@pytest.mark.parametrize("B,Hq,Hkv,hd,max_len,lens,n_split", [
    (3, 8, 2, 128, 1000, [1000, 517, 1], 0), (3, 8, 2, 128, 1000, [1000, 517, 1], 5),
    (2, 4, 4, 64, 300, [300, 33], 1), (2, 16, 1, 64, 777, [777, 640], 0),
    (64, 32, 8, 128, 4097, None, 0), (2, 8, 2, 128, 300, [1000, -3], 0),
])
def test_attention_decode(gpu, B, Hq, Hkv, hd, max_len, lens, n_split):
    """KV-cache decode attention vs the oracle attention (pinned against SDPA) per sequence.
    Lengths outside 1..max_len are clamped to it (the last case), so no read leaves the cache."""
    from oracle.llama import attention
    from torch_helion.hip import ops

    announce(f"attention decode B={B} Hq={Hq} Hkv={Hkv} hd={hd} max_len={max_len} lens={lens} split={n_split}")
    g = torch.Generator().manual_seed(B * 7 + hd)
    q = torch.randn(B, Hq * hd, generator=g).bfloat16()
    kc = torch.randn(B, max_len, Hkv, hd, generator=g).bfloat16()
    vc = torch.randn(B, max_len, Hkv, hd, generator=g).bfloat16()
    scale = 1.0 / math.sqrt(hd)
    lengths = lens if lens is not None else [max_len] * B
    refs = []
    for b in range(B):
        L = min(max(lengths[b], 1), max_len)
        qb = q[b].float().reshape(1, Hq, 1, hd)
        kb = kc[b, :L].float().permute(1, 0, 2).unsqueeze(0)
        vb = vc[b, :L].float().permute(1, 0, 2).unsqueeze(0)
        refs.append(attention(qb.double(), kb.double(), vb.double(), False).reshape(Hq * hd))
    ref = torch.stack(refs)
    ws = torch.empty(max(ops.attention_decode_workspace_bytes(B, Hq, Hkv, hd, max_len, n_split) // 4, 1), device=gpu)
    out = torch.empty(B, Hq * hd, dtype=torch.bfloat16, device=gpu)
    lt = torch.tensor(lengths, dtype=torch.int32, device=gpu) if lens is not None else None
    ops.attention_decode(q.to(gpu), kc.to(gpu), vc.to(gpu), out, scale=scale, lengths=lt,
                         fixed_len=0 if lens is not None else max_len, n_split=n_split, workspace=ws)
    torch.cuda.synchronize()
    assert _maxabs(out, ref) < BF16_TOL


@pytest.mark.parametrize("dtype,M,K", [(torch.bfloat16, 1000, 4096), (torch.float32, 77, 512), (torch.bfloat16, 33, 40960)])
def test_rmsnorm(gpu, dtype, M, K):
    from torch_helion.hip import ops

    announce(f"rmsnorm {dtype} M={M} K={K}")
    g = torch.Generator().manual_seed(K)
    x = torch.randn(M, K, generator=g).to(dtype)
    gain = torch.rand(K, generator=g) + 0.5
    xf = x.float()
    ref = xf * ((xf * xf).mean(-1, keepdim=True) + 1e-5).rsqrt() * gain
    out = torch.empty(M, K, dtype=dtype, device=gpu)
    ops.rmsnorm(x.to(gpu), gain.to(gpu), 1e-5, out)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert _rel(out, ref) < F32_REL
    else:
        assert _maxabs(out, ref) < BF16_TOL


def test_epilogue_vm(gpu):
    from torch_helion.hip import abi, ops

    announce("epilogue vm")
    M, N = 70, 50
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, N, generator=g)
    col = torch.rand(M, 1, generator=g) + 0.5
    # y = exp(x * col - rowmax(x)) / rowsum(...)   (a softmax-like chain)
    ref_t = x * col
    ref_e = torch.exp(ref_t - ref_t.amax(-1, keepdim=True))
    ref = ref_e / ref_e.sum(-1, keepdim=True)
    ws = torch.empty(6 * M * N, device=gpu)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    ops_ = [(abi.VM_LOAD, 0, 0, -1, 0.0, 0), (abi.VM_LOAD, 1, 1, -1, 0.0, 0), (abi.VM_MUL, 2, 0, 1, 0.0, 0),
            (abi.VM_ROW_MAX, 3, 2, -1, 0.0, 0), (abi.VM_SUB, 4, 2, 3, 0.0, 0), (abi.VM_EXP, 4, 4, -1, 0.0, 0),
            (abi.VM_ROW_SUM, 5, 4, -1, 0.0, 0), (abi.VM_DIV, 4, 4, 5, 0.0, 0), (abi.VM_MUL, 4, 4, -1, 1.0, 1)]
    ops.epilogue_vm(M, N, [(x.to(gpu), False), (col.to(gpu), True)], ops_, [(out, 4)], 6, ws)
    torch.cuda.synchronize()
    assert _maxabs(out, ref) < 1e-2


def _ssd_case(bs, s, h, p, n, g, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(bs * s, h * p, generator=gen)
    bm = torch.randn(bs * s, g * n, generator=gen) * 0.5
    cm = torch.randn(bs * s, g * n, generator=gen) * 0.5
    dt = torch.rand(bs * s, h, generator=gen) * 0.099 + 0.001
    A = -torch.exp(torch.rand(h, generator=gen) * math.log(16.0))
    D = torch.rand(h, generator=gen)
    gate = torch.randn(bs * s, h * p, generator=gen)
    return [t.to(dtype) for t in (x, bm, cm, dt)] + [A, D, gate.to(dtype)]


@pytest.mark.parametrize("bs,s,h,p,n,g,chunk,dtype", [
    (2, 256, 4, 64, 64, 1, 64, torch.float32), (1, 200, 4, 32, 32, 2, 64, torch.float32),
    (2, 512, 2, 64, 128, 1, 256, torch.float32), (2, 1024, 16, 64, 64, 1, 64, torch.bfloat16),
    # bf16 runs on the MFMA path: ragged length, groups, N=32, N=128 with 256-row chunks, 128- and 32-row chunks
    (1, 200, 4, 32, 32, 2, 64, torch.bfloat16), (2, 512, 2, 64, 128, 1, 256, torch.bfloat16),
    (2, 300, 4, 64, 64, 1, 128, torch.bfloat16), (1, 100, 2, 64, 64, 1, 32, torch.bfloat16),
    (1, 300, 2, 128, 128, 1, 256, torch.bfloat16),   # 4 p-tiles per unit, ragged last chunk
    (2, 2048, 4, 64, 128, 1, 256, torch.bfloat16),   # C4 head shape and length (4 of its 32 heads)
])
def test_ssd_chunked_vs_recurrence(gpu, bs, s, h, p, n, g, chunk, dtype):
    from oracle.mamba import ssd_chunked_program
    from torch_helion.hip import ops

    announce(f"ssd_chunked bs={bs} s={s} h={h} p={p} n={n} g={g} chunk={chunk} {dtype}")
    x, bm, cm, dt, A, D, gate = _ssd_case(bs, s, h, p, n, g, dtype, seed=s + h)
    a = {"batch": bs, "seq": s, "heads": h, "head_dim": p, "state_dim": n, "ngroups": g}
    ref = ssd_chunked_program(cm.double(), bm.double(), x.double(), dt.double(), A.double(), D.double(), a)
    ref = ref * gate.double()
    ws = torch.empty(ops.ssd_workspace_bytes(bs, s, h, p, n, chunk) // 4 + 1, device=gpu)
    out = torch.empty(bs * s, h * p, dtype=dtype, device=gpu)
    out32 = torch.empty(bs * s, h * p, device=gpu)
    ops.ssd_chunked(x=x.to(gpu), b=bm.to(gpu), c=cm.to(gpu), dt=dt.to(gpu), out=out, out32=out32, workspace=ws,
                    batch=bs, seq=s, heads=h, head_dim=p, state_dim=n, ngroups=g, chunk=chunk, A=A.to(gpu),
                    D=D.to(gpu), gate=gate.to(gpu))
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert _rel(out32, ref) < F32_REL
    else:
        assert _maxabs(out32, ref) < BF16_TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ssd_reference_form_padded_cum(gpu, dtype):
    """The reference's ssd kind: cum and dt padded to 32 columns per head, cum centred, full D."""
    from oracle.interpret import ssd_quadratic
    from torch_helion.hip import ops

    announce(f"ssd reference form {dtype}")
    bs, s, h, p, n, pad = 2, 256, 4, 32, 32, 32
    x, bm, cm, dt, A, D, _ = _ssd_case(bs, s, h, p, n, h, dtype, seed=11)
    dt = dt.float()
    da = (dt * A).reshape(bs, s, h)
    cum = torch.cumsum(da, 1) - 0.5 * da.sum(1, keepdim=True)             # centred per sequence
    cum_pad = cum.reshape(bs * s, h, 1).expand(bs * s, h, pad).reshape(bs * s, h * pad).contiguous()
    dt_pad = dt.reshape(bs * s, h, 1).expand(bs * s, h, pad).reshape(bs * s, h * pad).contiguous()
    d_full = D.repeat_interleave(p).reshape(1, -1).expand(bs * s, h * p).contiguous()
    mask = torch.ones(s, s).tril()
    attrs = {"batch": bs, "seq": s, "heads": h, "head_dim": p, "state_dim": n, "pad": pad}
    if dtype != torch.float32:  # the kernel reads every operand in one dtype
        cum_pad, dt_pad, d_full = cum_pad.to(dtype), dt_pad.to(dtype), d_full.to(dtype)
    ref = ssd_quadratic(cm.double(), bm.double(), x.double(), cum_pad.double(), dt_pad.double(), mask.double(),
                        d_full.double(), attrs)
    ws = torch.empty(ops.ssd_workspace_bytes(bs, s, h, p, n, 64) // 4 + 1, device=gpu)
    out = torch.empty(bs * s, h * p, device=gpu)
    ops.ssd_chunked(x=x.to(gpu), b=bm.to(gpu), c=cm.to(gpu), dt=dt_pad.to(gpu), out=out, workspace=ws, batch=bs,
                    seq=s, heads=h, head_dim=p, state_dim=n, ngroups=h, chunk=64, cum=cum_pad.to(gpu), dt_stride=pad,
                    dskip=d_full.to(gpu))
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert _rel(out, ref) < F32_REL
    else:
        assert _maxabs(out, ref) < BF16_TOL


@pytest.mark.parametrize("bs,s,h,p,n,g,chunk", [
    (2, 2048, 8, 64, 128, 1, 256),     # C4's head shape and length (8 of its 32 heads), 2 p-tiles per unit
    (1, 300, 4, 128, 128, 1, 256),     # 4 p-tiles, 2 per unit, ragged last chunk
    (1, 200, 4, 64, 128, 2, 64),       # two groups of two heads, 64-row chunks (1 p-tile per unit), ragged
    (2, 300, 6, 64, 128, 2, 128),      # three heads per group, 128-row chunks, ragged
])
def test_ssd_shared_g_tiles_bit_exact(gpu, bs, s, h, p, n, g, chunk):
    """With room for the shared G^T tiles (th_ssd_gtile_workspace_bytes, state_dim 128) the
    state kernels of a group form each chunk's C_t B_s^T once between them and the out kernel
    loads it; the tiles come from the same MFMA chain on the same operands as the per-head
    chain, so y and y32 equal the minimum-workspace call's bit for bit, and the tiles' region
    is written."""
    from oracle.mamba import ssd_chunked_program
    from torch_helion.hip import ops

    announce(f"ssd shared G tiles bs={bs} s={s} h={h} p={p} n={n} g={g} chunk={chunk}")
    x, bm, cm, dt, A, D, gate = _ssd_case(bs, s, h, p, n, g, torch.bfloat16, seed=3 * s + h)
    args = dict(x=x.to(gpu), b=bm.to(gpu), c=cm.to(gpu), dt=dt.to(gpu), batch=bs, seq=s, heads=h, head_dim=p,
                state_dim=n, ngroups=g, chunk=chunk, A=A.to(gpu), D=D.to(gpu), gate=gate.to(gpu))
    base = ops.ssd_workspace_bytes(bs, s, h, p, n, chunk)
    big = ops.ssd_workspace_bytes(bs, s, h, p, n, chunk, g)
    # tiles [batch][group][chunk][pair] of 32 x 32 floats, pairs (t-block, s-block <= t-block)
    nt = chunk // 32
    nc, npair = -(-s // chunk), nt * (nt + 1) // 2
    assert big - base == bs * g * nc * npair * 1024 * 4
    outs = []
    for nbytes in (base, big):
        ws = torch.full((nbytes // 4,), float("nan"), device=gpu)
        out = torch.empty(bs * s, h * p, dtype=torch.bfloat16, device=gpu)
        out32 = torch.empty(bs * s, h * p, device=gpu)
        ops.ssd_chunked(out=out, out32=out32, workspace=ws, **args)
        torch.cuda.synchronize()
        outs.append((out, out32, ws))
    # chunk 0 of the last (batch, group) is full: its last pair is written
    last = base // 4 + (((bs - 1) * g + g - 1) * nc * npair + npair - 1) * 1024
    assert torch.isfinite(outs[1][2][base // 4:base // 4 + 1024]).all(), "the first G^T tile was not written"
    assert torch.isfinite(outs[1][2][last:last + 1024]).all(), "the last pair of a full chunk was not written"
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    a = {"batch": bs, "seq": s, "heads": h, "head_dim": p, "state_dim": n, "ngroups": g}
    ref = ssd_chunked_program(cm.double(), bm.double(), x.double(), dt.double(), A.double(), D.double(), a)
    assert _maxabs(outs[1][1], ref * gate.double()) < BF16_TOL


@pytest.mark.parametrize("bs,s,h,p,n,g,chunk", [(1, 512, 8, 64, 128, 1, 256), (2, 200, 4, 32, 64, 2, 64)])
def test_ssd_output_gain_and_row_sums(gpu, bs, s, h, p, n, g, chunk):
    """y_gain / rs_parts: the scan stores y times a per-column gain (the next RMSNorm's) and
    the sums of squares of y per token and 32 columns. Against the same scan's fp32 copy of
    y: the stored values are bf16(y * g) bit for bit, the sums those of y^2 within fp32
    rounding (the kernel adds 8 per lane, then across the 4 lanes of a row)."""
    from torch_helion.hip import ops

    announce(f"ssd output gain + row sums bs={bs} s={s} h={h} p={p} n={n} g={g} chunk={chunk}")
    x, bm, cm, dt, A, D, gate = _ssd_case(bs, s, h, p, n, g, torch.bfloat16, seed=7 * s + h)
    args = dict(x=x.to(gpu), b=bm.to(gpu), c=cm.to(gpu), dt=dt.to(gpu), batch=bs, seq=s, heads=h, head_dim=p,
                state_dim=n, ngroups=g, chunk=chunk, A=A.to(gpu), D=D.to(gpu), gate=gate.to(gpu))
    ws = torch.empty(ops.ssd_workspace_bytes(bs, s, h, p, n, chunk, g) // 4 + 1, device=gpu)
    y16 = torch.empty(bs * s, h * p, dtype=torch.bfloat16, device=gpu)
    y32 = torch.empty(bs * s, h * p, device=gpu)
    ops.ssd_chunked(out=y16, out32=y32, workspace=ws, **args)
    gain = (torch.rand(h * p, generator=torch.Generator().manual_seed(5)) + 0.5).to(gpu)
    yg = torch.empty(bs * s, h * p, dtype=torch.bfloat16, device=gpu)
    parts = torch.full((bs * s, h * p // 32), float("nan"), device=gpu)
    ops.ssd_chunked(out=yg, workspace=ws, y_gain=gain, rs_parts=parts, **args)
    torch.cuda.synchronize()
    assert torch.equal(yg, (y32 * gain).bfloat16())
    ref = (y32.double() ** 2).reshape(bs * s, h * p // 32, 32).sum(-1)
    assert torch.isfinite(parts).all()
    assert _rel(parts, ref) < 1e-6


@pytest.mark.parametrize("M,N,K", [(16384, 1024, 2048), (300, 512, 256)])  # persistent 256 x 256; direct loop
def test_gemm_row_sums_from_producer(gpu, M, N, K):
    """rs_parts: the row scale from the lhs producer's partial sums of squares (of the values
    before its gain) instead of the GEMM's own sum over its lhs. With parts that are the
    per-32-column sums of x^2 and the lhs x * g, the output is RMSNorm(x) * g times W plus the
    residual, as the th_rmsnorm-then-GEMM route computes it, within bf16 rounding of the lhs."""
    from torch_helion.hip import abi, ops

    announce(f"gemm row sums from producer M={M} N={N} K={K}")
    gen = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=gen)
    gain = torch.rand(K, generator=gen) + 0.5
    w = (torch.randn(K, N, generator=gen) * 0.03).bfloat16()
    res = torch.randn(M, N, generator=gen).bfloat16()
    lhs = (x * gain).bfloat16()
    parts = (x * x).reshape(M, K // 32, 32).sum(-1)
    r = ((x * x).sum(-1, keepdim=True) / K + 1e-5).rsqrt()
    ref = (lhs.float() @ w.float()) * r + res.float()
    packed = ops.pack_rhs([w.to(gpu)], torch.bfloat16)
    out = torch.empty(M, N, device=gpu)
    ss = torch.empty(M, device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 1, lhs.to(gpu), packed, [ops.EpiSpec(abi.EPI_ADD, out, e=0)], sumsq=True,
                          rscale_mask=1, inv_k=1.0 / K, eps=1e-5, extras=[res.to(gpu)], sumsq_out=ss,
                          rs_parts=parts.to(gpu)))
    torch.cuda.synchronize()
    assert _rel(ss, (x * x).sum(-1)) < 1e-5
    assert _rel(out, ref) < 1e-5


@pytest.mark.parametrize("dtype,bs,s,c,k,col0", [
    (torch.float32, 2, 300, 1152, 4, 0),
    (torch.bfloat16, 2, 300, 1152, 4, 0),     # 16-byte vector path, ragged last token run
    (torch.bfloat16, 3, 17, 128, 4, 128),     # input is a column slice of a wider tensor (row stride 384)
    (torch.bfloat16, 2, 40, 64, 3, 0),        # kernel width 3: element-wise path
])
def test_conv1d_causal(gpu, dtype, bs, s, c, k, col0):
    from oracle.interpret import conv1d
    from torch_helion.hip import ops

    announce(f"conv1d {dtype} bs={bs} s={s} c={c} k={k} col0={col0}")
    gen = torch.Generator().manual_seed(5 + c + k)
    wide = torch.randn(bs * s, c + 2 * col0, generator=gen).to(dtype)
    x = wide[:, col0:col0 + c]
    w = torch.randn(c, k, generator=gen) * 0.3
    ref = conv1d(x.double(), w.double(), {"batch": bs, "seq": s, "activation": "silu"})
    xd = wide.to(gpu)[:, col0:col0 + c]
    out = torch.empty(bs * s, c, dtype=dtype, device=gpu)
    out32 = torch.empty(bs * s, c, device=gpu)
    ops.conv1d_causal(xd, w.to(gpu), out, batch=bs, seq=s, activation="silu", out32=out32)
    torch.cuda.synchronize()
    assert _rel(out32, ref) < F32_REL
    if dtype == torch.float32:
        assert _rel(out, ref) < F32_REL
    else:
        assert _maxabs(out, ref) < BF16_TOL


@pytest.mark.parametrize("dtype,ids_dtype,V,D,T", [
    (torch.bfloat16, torch.int64, 50280, 1024, 16384),  # C4 lookup, 16-byte vector path
    (torch.float32, torch.int32, 1000, 64, 333),
    (torch.bfloat16, torch.int32, 500, 256, 37),         # a ragged last workgroup (1184 chunks of 16 bytes)
    (torch.bfloat16, torch.int64, 77, 100, 129),         # 200-byte rows: element-wise path
])
def test_embedding_gather_exact(gpu, dtype, ids_dtype, V, D, T):
    """out[t] = table[ids[t]] bit for bit (a copy), with and without the fp32 copy;
    ids outside [0, V) give zero rows and are counted."""
    from torch_helion.hip import ops

    announce(f"embedding {dtype} ids {ids_dtype} V={V} D={D} T={T}")
    g = torch.Generator().manual_seed(V + D + T)
    table = torch.randn(V, D, generator=g).to(dtype)
    ids = torch.randint(0, V, (T,), generator=g).to(ids_dtype)
    ids[0], ids[-1] = 0, V - 1
    td, idd = table.to(gpu), ids.to(gpu)
    out = torch.full((T, D), float("nan"), dtype=dtype, device=gpu)
    out32 = torch.full((T, D), float("nan"), device=gpu)
    ops.embedding(td, idd, out, out32=out32)
    torch.cuda.synchronize()
    ref = table[ids.long()]
    assert torch.equal(out.cpu(), ref)
    assert torch.equal(out32.cpu(), ref.float())
    bad = ids.clone()
    bad[1], bad[T // 2] = -3, V
    cnt = torch.zeros(1, dtype=torch.int32, device=gpu)
    out.fill_(float("nan"))
    ops.embedding(td, bad.to(gpu), out, n_invalid=cnt)
    torch.cuda.synchronize()
    got = out.cpu()
    assert int(cnt.item()) == 2
    assert torch.equal(got[1], torch.zeros(D, dtype=dtype)) and torch.equal(got[T // 2], torch.zeros(D, dtype=dtype))
    keep = torch.ones(T, dtype=torch.bool)
    keep[1] = keep[T // 2] = False
    assert torch.equal(got[keep], ref[keep])


def test_gemm_tied_lm_head_ragged_vocab(gpu):
    """The C4 head: [T, 1024] x E^T [1024, 50280] (vocab not a multiple of 32) with the
    final RMSNorm's row scale, bf16 and fp32 logits against a torch fp32 reference."""
    from torch_helion.hip import abi, ops

    M, N, K = 512, 50280, 1024
    announce(f"gemm lm head M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(11)
    h = torch.randn(M, K, generator=g).bfloat16()
    table = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    w = table.T.contiguous()
    r = (h.float().pow(2).mean(-1, keepdim=True) + 1e-5).rsqrt()
    ref = (h.float() @ w.float()) * r
    hd = h.to(gpu)
    packed = ops.pack_rhs([w.to(gpu)], torch.bfloat16)
    o16 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
    o32 = torch.full((M, N), float("nan"), device=gpu)
    ops.gemm(ops.GemmCall(M, N, K, 1, hd, packed, [ops.EpiSpec(abi.EPI_ACC, o16), ops.EpiSpec(abi.EPI_ACC, o32)],
                          sumsq=True, inv_k=1.0 / K, eps=1e-5, rscale_mask=0b1))
    torch.cuda.synchronize()
    assert _rel(o32, ref) < 1e-5
    assert _maxabs(o16, ref) < BF16_TOL * max(1.0, float(ref.abs().max()))
    assert not torch.isnan(o16).any()


@pytest.mark.parametrize("M", [2048, 16384])
def test_gemm_column_windows(gpu, M):
    """One accumulator over concatenated weights with outputs on column windows (the merged
    in-projection of a Mamba layer: B | C | dt | z | x), each with its own op, extra operand and
    RMS row scale: every window equals the separate projection; no output writes outside its window."""
    from torch_helion.hip import abi, ops

    K, eps = 512, 1e-5
    widths = [64, 64, 16, 1024, 1024]
    announce(f"gemm column windows M={M} widths={widths}")
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).bfloat16()
    ws = [(torch.randn(K, n, generator=g) * 0.05).bfloat16() for n in widths]
    bias = torch.randn(M, widths[2], generator=g)
    xf = x.float()
    r = ((xf * xf).sum(-1, keepdim=True) / K + eps).pow(-0.5)
    accs = [(xf @ w.float()) * r for w in ws]
    refs = [accs[0], accs[1], torch.nn.functional.softplus(accs[2] + bias, threshold=1e9),
            accs[3] * torch.sigmoid(accs[3]), accs[4]]
    ops_ = [abi.EPI_ACC, abi.EPI_ACC, abi.EPI_SOFTPLUS_ADD, abi.EPI_SILU, abi.EPI_ACC]
    xd = x.to(gpu)
    packed = ops.pack_rhs([torch.cat([w.to(gpu) for w in ws], dim=1).contiguous()], torch.bfloat16)
    # outputs padded by 8 columns on the right: the pad must stay untouched
    outs = [torch.full((M, n + 8), float("nan"), dtype=torch.bfloat16, device=gpu) for n in widths]
    epi, c0 = [], 0
    for n, op, o in zip(widths, ops_, outs):
        epi.append(ops.EpiSpec(op, o, a=0, e=0 if op == abi.EPI_SOFTPLUS_ADD else -1, cols=(c0, c0 + n)))
        c0 += n
    ops.gemm(ops.GemmCall(M, c0, K, 1, xd, packed, epi, sumsq=True, rscale_mask=1, inv_k=1.0 / K, eps=eps,
                          extras=[bias.to(gpu)]))
    torch.cuda.synchronize()
    for i, (n, o, ref) in enumerate(zip(widths, outs, refs)):
        got = o.cpu()
        assert torch.isnan(got[:, n:].float()).all(), i
        assert _maxabs(got[:, :n], ref) < BF16_TOL * max(1.0, float(ref.abs().max())), i
