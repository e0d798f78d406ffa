"""th_gemm_noalloc, the allocation-free variant of th_gemm, against th_gemm itself.

The variant keeps the e4m3 path's split-K partials in the library's fixed
per-GPU scratch array instead of a caller workspace; the kernels and split
counts are th_gemm's, so the outputs must be bit-identical. Two calls in a row
(the second smaller) show that nothing left in the shared array from the first
call leaks into the second.
"""

from __future__ import annotations

import ctypes as C

import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


def _quant_e4m3(w: torch.Tensor):
    s = (w.abs().amax(0).clamp_min(1e-12) / 448.0).float()
    return (w / s).to(torch.float8_e4m3fn), s


def _call(gpu, M, N, K, n_acc, seed):
    from torch_helion.hip import abi, ops

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16().to(gpu)
    qs = [_quant_e4m3(torch.randn(K, N, generator=g) * 0.02) for _ in range(n_acc)]
    packed = ops.pack_rhs([q.to(gpu) for q, _ in qs], torch.float8_e4m3fn)
    scale = torch.stack([s for _, s in qs]).to(gpu).contiguous()
    gain = (torch.rand(K, generator=g) + 0.5).to(gpu)
    extra = torch.randn(M, N, generator=g).to(gpu)
    if n_acc == 2:
        outs = [torch.full((M, N), float("nan"), device=gpu)]
        specs = [ops.EpiSpec(abi.EPI_SWIGLU, outs[0], a=0, b=1)]
    else:
        outs = [torch.full((M, N), float("nan"), device=gpu), torch.full((M, N), float("nan"), device=gpu).bfloat16()]
        specs = [ops.EpiSpec(abi.EPI_ADD, outs[0], a=0, e=0), ops.EpiSpec(abi.EPI_ACC, outs[1], a=0)]
    call = ops.GemmCall(M, N, K, n_acc, x, packed, specs, extras=[extra] if n_acc == 1 else [],
                        in_dtype=torch.float8_e4m3fn, rhs_scale=scale, sumsq=True, rscale_mask=(1 << n_acc) - 1,
                        inv_k=1.0 / K, eps=1e-5, lhs_gain=gain)
    return call, outs


@pytest.mark.parametrize("shapes", [[(64, 6144, 4096, 1), (16, 1024, 1024, 2)],
                                    [(64, 4096, 14336, 1), (32, 2048, 4096, 1)]])
def test_noalloc_matches_th_gemm_on_two_calls(gpu, shapes):
    """Per shape: th_gemm with its own workspace, then th_gemm_noalloc with new output buffers;
    the outputs are equal bit for bit. The second shape is the smaller one."""
    from torch_helion.hip import abi, ops

    lib = abi.load()
    for i, (M, N, K, n_acc) in enumerate(shapes):
        announce(f"th_gemm_noalloc call {i}: M={M} N={N} K={K} n_acc={n_acc}")
        need = lib.th_gemm_workspace_bytes(M, N, K, n_acc, abi.TH_F8E4M3)
        assert 0 < need <= abi.GEMM_NOALLOC_SCRATCH_BYTES
        call, ref = _call(gpu, M, N, K, n_acc, seed=10 + i)
        call.workspace = torch.empty(need, dtype=torch.uint8, device=gpu)
        ops.gemm(call)
        torch.cuda.synchronize()
        call.outs = [ops.EpiSpec(s.op, torch.full_like(s.out, float("nan")), a=s.a, b=s.b, e=s.e) for s in call.outs]
        call.workspace = None
        ops.gemm_noalloc(call)
        torch.cuda.synchronize()
        for r, s in zip(ref, call.outs):
            assert torch.isfinite(s.out.float()).all()
            assert torch.equal(s.out, r), (i, (s.out.float() - r.float()).abs().max().item())


def test_noalloc_refuses_sizes_beyond_its_scratch(gpu):
    """A shape whose partial sums exceed the fixed scratch is refused with a clear error before
    any launch (the output keeps its contents). The operands are full-size (uninitialised), so
    even a launch would stay inside them."""
    from torch_helion.hip import abi, ops

    lib = abi.load()
    M, N, K = 128, 4096, 131072
    assert lib.th_gemm_workspace_bytes(M, N, K, 1, abi.TH_F8E4M3) > abi.GEMM_NOALLOC_SCRATCH_BYTES
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=gpu)
    packed = torch.zeros(lib.th_gemm_packed_bytes(N, K, 1, abi.TH_F8E4M3), dtype=torch.uint8, device=gpu)
    out = torch.full((M, N), float("nan"), device=gpu)
    call = ops.GemmCall(M, N, K, 1, x, packed, [ops.EpiSpec(abi.EPI_ACC, out, a=0)], in_dtype=torch.float8_e4m3fn,
                        rhs_scale=torch.ones(1, N, device=gpu))
    with pytest.raises(abi.HipBackendError, match="scratch"):
        ops.gemm_noalloc(call)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()


def test_noalloc_bf16_is_th_gemm(gpu):
    """bf16 weights need no scratch: the variant is th_gemm itself (same output, bit for bit)."""
    from torch_helion.hip import abi, ops

    g = torch.Generator().manual_seed(5)
    x = torch.randn(256, 512, generator=g).bfloat16().to(gpu)
    packed = ops.pack_rhs([(torch.randn(512, 384, generator=g) * 0.05).bfloat16().to(gpu)], torch.bfloat16)
    a, b = torch.empty(256, 384, device=gpu), torch.empty(256, 384, device=gpu)
    ops.gemm(ops.GemmCall(256, 384, 512, 1, x, packed, [ops.EpiSpec(abi.EPI_ACC, a, a=0)]))
    ops.gemm_noalloc(ops.GemmCall(256, 384, 512, 1, x, packed, [ops.EpiSpec(abi.EPI_ACC, b, a=0)]))
    torch.cuda.synchronize()
    assert torch.equal(a, b)
