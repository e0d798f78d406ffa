"""Fused-epilogue matching against the reference's recorded OpIR programs (CPU).

The HIP gemm kernel runs a fixed catalogue of output ops (th_epi_op in
include/th_hip.h) instead of the reference's per-kernel epilogue SSA
(reference codegen/emit.py:188-221). ``match_epilogue`` decides, per kernel,
which catalogue op reproduces each stored output. Here every gemm kernel of
the reference's three recorded programs (tests/golden/reference_results) is
matched, the matched plan is evaluated with the catalogue's definitions as the
header states them, and the result is compared with the oracle interpreter
running the kernel's own SSA on the same random operands. A plan that names a
wrong accumulator, a wrong extra operand or a dropped row scale fails here.
"""

from __future__ import annotations

from pathlib import Path

import pytest
import torch

GOLDEN = Path(__file__).parent / "golden" / "reference_results"
RUNS = ("llama_block", "mamba_block", "mamba")


def _catalogue(op: int, a: torch.Tensor, b: torch.Tensor | None, e: torch.Tensor | None,
               cos: torch.Tensor | None, sin: torch.Tensor | None) -> torch.Tensor:
    """th_epi_op definitions (include/th_hip.h), float64."""
    from torch_helion.hip import abi

    if op == abi.EPI_ACC:
        return a
    if op == abi.EPI_ROPE_PAIR:
        return a * cos + b * sin
    if op == abi.EPI_SILU:
        return a * torch.sigmoid(a)
    if op == abi.EPI_SWIGLU:
        return a * torch.sigmoid(a) * b
    if op == abi.EPI_ADD:
        return a + e
    if op == abi.EPI_SOFTPLUS_ADD:
        return torch.log1p(torch.exp(a + e))
    if op == abi.EPI_MUL:
        return a * e
    raise AssertionError(f"op {op} not evaluated here")


def _kernels():
    from torch_helion.optimizer.opir import Program

    out = []
    for run in RUNS:
        prog = Program.from_json(GOLDEN / run / "06_opir.json")
        for k in prog.kernels:
            if k.kind == "gemm":
                out.append(pytest.param(run, prog, k, id=f"{run}-{k.name}"))
    return out


# Kernels whose epilogue is outside the catalogue and runs on the epilogue VM:
# stand-alone norms (no accumulator; th_rmsnorm) and the reference's mamba k5,
# which scales three *extra* operands by the row RMS factor.
EXPECTED_VM = {("mamba_block", "k6_gemm"), ("mamba", "k5_gemm"), ("mamba", "k14_gemm")}


@pytest.mark.parametrize("run,prog,spec", _kernels())
def test_reference_epilogues_match_the_catalogue(run, prog, spec):
    from oracle import interpret as oi
    from torch_helion.hip.epilogue import match_epilogue

    plan = match_epilogue(spec)
    if (run, spec.name) in EXPECTED_VM:
        assert not plan.fused, "expected the VM fallback"
        return
    assert plan.fused, plan.reason

    g = torch.Generator().manual_seed(11)
    env: dict[str, torch.Tensor] = {}
    for a in spec.args:
        shape = prog.tensors[a.tensor].shape
        env[a.tensor] = torch.randn(*shape, generator=g, dtype=torch.float64) * 0.5
    ref = oi.run_kernel(spec, env)

    lhs = env[spec.arg("lhs").tensor]
    accs = [lhs @ env[spec.arg(gm.rhs).tensor] for gm in spec.gemms]
    if plan.rscale is not None:
        inv_k, eps = plan.rscale
        r = (lhs.pow(2).sum(1, keepdim=True) * inv_k + eps).rsqrt()
        accs = [acc * r if plan.scaled.get(i) else acc for i, acc in enumerate(accs)]
    else:
        assert not any(plan.scaled.values())
    for o in plan.outs:
        e = env[spec.arg(o.extra).tensor] if o.extra else None
        cos = sin = None
        if o.rope:
            cos, sin = (env[spec.arg(n).tensor] for n in o.rope)
        got = _catalogue(o.op, accs[o.a], accs[o.b] if o.b >= 0 else None, e, cos, sin)
        want = ref[o.tensor]
        assert got.shape == want.shape
        assert (got - want).abs().max() <= 1e-9 * (1 + want.abs().max()), (spec.name, o.tensor, o.op)


def test_a_wrong_plan_is_caught():
    """Swapping the accumulators of the reference Llama's RoPE pair changes the value (the check has teeth)."""
    from oracle import interpret as oi
    from torch_helion.hip import abi
    from torch_helion.hip.epilogue import match_epilogue
    from torch_helion.optimizer.opir import Program

    prog = Program.from_json(GOLDEN / "llama_block" / "06_opir.json")
    spec = next(k for k in prog.kernels if k.name == "k0_gemm")
    plan = match_epilogue(spec)
    pair = next(o for o in plan.outs if o.op == abi.EPI_ROPE_PAIR)
    g = torch.Generator().manual_seed(3)
    env = {a.tensor: torch.randn(*prog.tensors[a.tensor].shape, generator=g, dtype=torch.float64)
           for a in spec.args}
    ref = oi.run_kernel(spec, env)[pair.tensor]
    lhs = env[spec.arg("lhs").tensor]
    inv_k, eps = plan.rscale
    r = (lhs.pow(2).sum(1, keepdim=True) * inv_k + eps).rsqrt()
    accs = [(lhs @ env[spec.arg(gm.rhs).tensor]) * r for gm in spec.gemms]
    cos, sin = (env[spec.arg(n).tensor] for n in pair.rope)
    good = _catalogue(pair.op, accs[pair.a], accs[pair.b], None, cos, sin)
    bad = _catalogue(pair.op, accs[pair.b], accs[pair.a], None, cos, sin)
    assert (good - ref).abs().max() < 1e-9
    assert (bad - ref).abs().max() > 1e-2
