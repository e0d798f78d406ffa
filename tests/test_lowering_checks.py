"""Lowering decisions of the device runtime that need no GPU: the checks run
before any buffer is touched on the device, so plain CPU stand-ins serve."""

from __future__ import annotations

from collections import defaultdict
from types import SimpleNamespace

import pytest
import torch

from torch_helion.hip import abi
from torch_helion.optimizer.opir import KernelArg, KernelSpec


def _ssd_spec(kind: str) -> KernelSpec:
    roles = ["x", "b", "c", "dt", "A", "D"] if kind == "ssd_chunked" else ["x", "b", "c", "dt", "cum", "mask", "dskip"]
    return KernelSpec("k_ssd", kind, args=[KernelArg(r, r, r) for r in roles],
                      attrs={"batch": 1, "seq": 4, "heads": 2, "head_dim": 8, "state_dim": 8, "chunk": 4, "pad": 1})


def _dp(values: dict[str, torch.Tensor], host: dict[str, torch.Tensor] | None = None):
    bufs = defaultdict(lambda: torch.zeros(1))
    bufs.update(values)
    host = host or {}
    return SimpleNamespace(buffers=bufs, _host=lambda name: host.get(name))


def test_ssd_chunked_refuses_positive_A():
    """The scan's split decay exponents need a non-increasing running sum of dt*A."""
    from torch_helion.hip.ssd import lower_ssd

    with pytest.raises(abi.HipBackendError, match="A <= 0"):
        lower_ssd(_dp({"A": torch.tensor([-1.0, 0.5])}), _ssd_spec("ssd_chunked"))


def test_ssd_refuses_increasing_cum():
    from torch_helion.hip.ssd import lower_ssd

    cum = torch.tensor([[0.0, 0.0], [-0.1, -0.2], [0.3, -0.3], [0.2, -0.5]])   # head 0 rises at t = 2
    host = {"mask": torch.ones(4, 4).tril(), "cum": cum}
    with pytest.raises(abi.HipBackendError, match="non-increasing"):
        lower_ssd(_dp({}, host), _ssd_spec("ssd"))


@pytest.fixture(scope="module")
def decode_case(tmp_path_factory):
    from targets.llama_block import LlamaBlockConfig
    from targets.llama_decode import build_llama_decode_block
    from torch_helion import CompileConfig, compile_model

    cfg = LlamaBlockConfig(batch=2, seq=16, hidden=128, heads=2, kv_heads=1, intermediate=256, causal=True,
                           dtype=torch.bfloat16)
    m = build_llama_decode_block(cfg, pos=5, seed=0)
    res = compile_model(m, m.example_inputs(seed=0), CompileConfig(
        run_name="dec", results_dir=tmp_path_factory.mktemp("dec"), backend="none", planner_mode="greedy"))
    return res


def test_e4m3_weights_never_unfold_a_gain(decode_case):
    """Even where a fold record names an e4m3 weight (a DeviceProgram built with fold_sources
    for a decode program), the runtime must not take a gain back out of it: the gain is the
    kernel's own ``gain`` argument and would be applied twice."""
    from torch_helion.hip.epilogue import match_epilogue
    from torch_helion.hip.runtime import DeviceProgram

    prog = decode_case.program
    k = next(k for k in prog.kernels if len(k.gemms) == 2 and any(a.role == "gain" for a in k.args))
    plan = match_epilogue(k)
    used = sorted({o.a for o in plan.outs} | {o.b for o in plan.outs if o.b >= 0})
    gain = decode_case.graph.params[k.arg("gain").tensor]
    folds = {k.arg(k.gemms[i].rhs).tensor: (gain, torch.zeros(1)) for i in used}
    fake = SimpleNamespace(fold_sources=folds, program=prog)
    assert plan.rscale is not None
    assert DeviceProgram._unfold_gain(fake, k, plan, used) is None
    # the same kernel with bf16 weights would unfold it: the refusal is the dtype's
    bf16 = SimpleNamespace(fold_sources=folds, program=SimpleNamespace(tensors={
        **prog.tensors, **{t: SimpleNamespace(dtype="bfloat16", shape=prog.tensors[t].shape) for t in folds}}))
    assert DeviceProgram._unfold_gain(bf16, k, plan, used) is gain
