"""compile_model on a decode-step module: the Program it derives (e4m3 weight tensors with
per-column scales, activation-side norm gains, an attention_decode kernel over the cache)
against the oracle's decode step. CPU only: backend "none", the oracle interpreter."""

from __future__ import annotations

import pytest
import torch

from oracle import interpret as oi
from oracle.llama import decode_step

POS = 77


@pytest.fixture(scope="module")
def case(tmp_path_factory):
    from targets.llama_block import LlamaBlockConfig
    from targets.llama_decode import build_llama_decode_block
    from torch_helion import CompileConfig, compile_model

    cfg = LlamaBlockConfig(batch=4, seq=80, hidden=256, heads=4, kv_heads=2, intermediate=512, causal=True,
                           dtype=torch.bfloat16, rope_theta=500000.0)
    m = build_llama_decode_block(cfg, pos=POS, seed=3)
    x, kc, vc = m.example_inputs(seed=1)
    res = compile_model(m, (x, kc, vc), CompileConfig(run_name="decode", results_dir=tmp_path_factory.mktemp("dec"),
                                                      backend="none", planner_mode="greedy"))
    return cfg, m, (x, kc, vc), res


def _exact_weights(m):
    """The dequantised projections q * s in float64 and the model's gains: what the step computes with."""
    from targets.llama_decode import PROJECTIONS

    w = {name: getattr(m, f"{s}_q").double() * getattr(m, f"{s}_s").double()[:, None] for s, name in PROJECTIONS.items()}
    w["input_norm.weight"], w["post_norm.weight"] = m.g1, m.g2
    return w


def _oracle_step(cfg, m, inputs):
    x, kc, vc = inputs
    rope = (m.rope_cos.expand(POS + 1, -1), m.rope_sin.expand(POS + 1, -1))
    return decode_step(x, _exact_weights(m), kc, vc, POS, heads=cfg.heads, kv_heads=cfg.n_kv, eps=cfg.eps,
                       theta=cfg.rope_theta, rope=rope)


def _rel(a, b):
    return ((a - b.reshape(a.shape)).abs().max() / b.abs().max()).item()


def test_decode_program_structure(case):
    cfg, m, inputs, res = case
    prog = res.program
    kinds = [k.kind for k in prog.kernels]
    assert kinds.count("attention_decode") == 1 and "attention" not in kinds
    assert prog.inputs[1:] == ["k_cache", "v_cache"] and len(prog.outputs) == 3
    for k in prog.kernels:
        if k.kind != "gemm":
            continue
        names = {a.name for a in k.args}
        for g in k.gemms:
            assert prog.tensors[k.arg(g.rhs).tensor].dtype == "float8_e4m3fn"
            assert g.rhs + "_scale" in names
    # the q/kv and gate/up projections read the normalised input: their gain is an argument
    gains = [k for k in prog.kernels if any(a.role == "gain" for a in k.args)]
    assert len(gains) == 3
    slots = prog.metadata["cache_slots"]
    assert {v["cache"] for v in slots.values()} == {"k_cache", "v_cache"} and set(slots) == set(prog.outputs[1:])
    att = next(k for k in prog.kernels if k.kind == "attention_decode")
    assert res.program.kernels[kinds.index("attention_decode")].cost["bound"] == "hbm"
    assert att.attrs["pos"] == POS and att.attrs["max_len"] == cfg.seq


def test_decode_program_matches_oracle_step(case):
    """The oracle interpreter on the derived Program equals the oracle's decode step in float64
    (weights q * s exactly, the model's RoPE rows): the output and the new key/value rows."""
    cfg, m, inputs, res = case
    outs = oi.program_outputs(res.program, res.graph.params, list(inputs))
    ref = _oracle_step(cfg, m, inputs)
    for o, r in zip(outs, ref):
        assert _rel(o, r) < 1e-12


def test_decode_program_planted_mistakes_fail(case):
    """Mistakes the derivation could make are visible to the check above: a gain left off, a
    scale left off, and the attention reading the cache's row pos instead of the new key."""
    import copy

    cfg, m, inputs, res = case
    ref = _oracle_step(cfg, m, inputs)
    params = res.graph.params
    bad = copy.deepcopy(res.program)
    k = next(k for k in bad.kernels if any(a.role == "gain" for a in k.args))
    k.args = [a for a in k.args if a.role != "gain"]
    assert _rel(oi.program_outputs(bad, params, list(inputs))[0], ref[0]) > 1e-3
    bad = copy.deepcopy(res.program)
    k = next(k for k in bad.kernels if k.kind == "gemm")
    k.args = [a for a in k.args if a.role != "scale"]
    assert _rel(oi.program_outputs(bad, params, list(inputs))[0], ref[0]) > 1e-1
    bad = copy.deepcopy(res.program)
    att = next(k for k in bad.kernels if k.kind == "attention_decode")
    att.attrs["pos"] = POS + 1      # keys 0..pos of the cache (its stale row pos) plus the new one
    assert _rel(oi.program_outputs(bad, params, list(inputs))[0], ref[0]) > 1e-4


def test_decode_program_product_interpreter(case):
    """The product's fp32 interpreter runs the same Program to within fp32 rounding of the oracle."""
    from torch_helion.codegen.interpret import program_outputs

    cfg, m, inputs, res = case
    outs = program_outputs(res.program, res.graph.params, list(inputs))
    ref = _oracle_step(cfg, m, inputs)
    for o, r in zip(outs, ref):
        assert _rel(o.double(), r) < 1e-5


def test_decode_kernel_files(case):
    """Launch plans name the decode entry points: e4m3 GEMMs and th_attention_decode."""
    cfg, m, inputs, res = case
    plans = {p.name for p in res.kernel_files.values()}
    assert any("attention_decode" in p for p in plans)


@pytest.mark.parametrize("mistake", ["one_unfolded", "different_gain"])
def test_decode_program_refuses_inconsistent_gains(case, monkeypatch, tmp_path, mistake):
    """A kernel whose GEMM weights do not all carry the same folded norm gain is refused: one
    gain argument multiplies the kernel's shared lhs, so a weight folded without it (or with
    another gain) would be computed wrongly without any error."""
    import torch_helion.decode as dec

    cfg, m, inputs, res = case
    pair = next(k for k in res.program.kernels if len(k.gemms) == 2 and any(a.role == "gain" for a in k.args))
    t2 = pair.arg(pair.gemms[1].rhs).tensor
    real = dec._prefill_form

    def mutated(model, batch, config, run_dir):
        pre = real(model, batch, config, run_dir)
        folds = pre.graph.fold_sources
        assert t2 in folds
        if mistake == "one_unfolded":
            pre.graph.params[t2] = folds.pop(t2)[1]   # the model's own weight, no gain folded in
        else:
            g, w = folds[t2]
            folds[t2] = (g * 2, w)
        return pre

    monkeypatch.setattr(dec, "_prefill_form", mutated)
    with pytest.raises(ValueError, match="gain"):
        dec.decode_program(m, cfg.batch, res.config, tmp_path)
