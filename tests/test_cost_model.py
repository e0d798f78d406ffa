"""Cost model on the CPU: the GEMM tile choice mirrors th_gemm's, the calibration fit
recovers the parameters that generated its samples, and merged sibling launches are
priced with the fitted merged-launch factor (the planner's merge-or-split decision);
and the counters tool's per-symbol table."""

from __future__ import annotations

import dataclasses

import pytest


def test_gemm_tiles_mirror_th_gemm():
    """th_gemm's rules (csrc/gemm.hip): 256-row tiles when they give two blocks per CU,
    128 when one, else 64; one accumulator over a multiple of 256 columns takes
    256 x 256 tiles when those make whole waves of the 256 CUs."""
    from torch_helion.cost_models.roofline import gemm_tiles

    assert gemm_tiles(1024, 1, 16384, "bfloat16") == (256, 256)   # 64 x 4 = 256 tiles: one whole wave
    assert gemm_tiles(1280, 1, 16384, "bfloat16") == (256, 128)   # 64 x 5 = 320: not whole waves
    assert gemm_tiles(1024, 1, 8192, "bfloat16") == (128, 128)    # 128 wide tiles: too few
    assert gemm_tiles(1000, 1, 16384, "bfloat16") == (256, 128)   # not a multiple of 256 columns
    assert gemm_tiles(2048, 2, 16384, "bfloat16") == (256, 128)   # two accumulators: unchanged
    assert gemm_tiles(4096, 1, 16384, "bfloat16") == (256, 256)
    assert gemm_tiles(512, 1, 64, "bfloat16") == (64, 64)


def _rec(kernel, cat, ideal, waves, measured):
    return {"run": "r", "kernel": kernel, "category": cat, "ideal_us": ideal, "waves": waves,
            "measured_us": measured, "bound": "mfma"}


def test_calibration_fit_recovers_parameters():
    """Samples generated from known parameters: the weighted NNLS fit returns them, the
    merged-launch factor is the one the merged samples carry, and predict() reproduces
    every sample."""
    from torch_helion.cost_models.calibrate import fit, predict

    eff, tile, fixed, factor = 0.5, 10.0, 8.0, 1.25
    recs = [_rec(f"k{i}", "gemm_bf16", ideal, waves, ideal / eff + waves * tile + fixed)
            for i, (ideal, waves) in enumerate([(5, 1), (40, 2), (100, 4), (300, 4), (800, 8), (20, 0.25),
                                                (2, 0.0625)])]
    recs += [_rec(f"m{i}", "gemm_bf16_merged", ideal, waves, factor * (ideal / eff + waves * tile + fixed))
             for i, (ideal, waves) in enumerate([(60, 3), (3, 1), (150, 5)])]
    c = fit(recs)
    assert c["efficiency"]["gemm_bf16"] == pytest.approx(eff, rel=1e-3)
    assert c["tile_us"]["gemm_bf16"] == pytest.approx(tile, rel=1e-3)
    assert c["fixed_us"]["gemm_bf16"] == pytest.approx(fixed, abs=0.01)
    assert c["merged_launch_factor"] == pytest.approx(factor, abs=1e-3)
    assert c["kernels_fitted"] == {"gemm_bf16": 7, "gemm_bf16_merged": 3}
    for r in recs:
        assert predict(r, c) == pytest.approx(r["measured_us"], rel=2e-3)


def test_calibration_without_merged_samples_has_no_factor():
    from torch_helion.cost_models.calibrate import fit

    recs = [_rec(f"k{i}", "gemm_bf16", ideal, waves, 2 * ideal + 10 * waves + 8)
            for i, (ideal, waves) in enumerate([(5, 1), (40, 2), (100, 4), (300, 8)])]
    assert "merged_launch_factor" not in fit(recs)


@pytest.fixture(scope="module")
def mamba_program(tmp_path_factory):
    from targets.mamba import MambaConfig, build_mamba_block
    from torch_helion import CompileConfig, compile_model

    cfg = MambaConfig(batch=2, seq=64, d_model=256, expand=2, headdim=32, d_state=32, chunk=32, n_layers=1)
    m = build_mamba_block(cfg)
    x = m.example_inputs(seed=0)
    res = compile_model(m, x, CompileConfig(run_name="cm", results_dir=tmp_path_factory.mktemp("cm"), backend="none",
                                            planner_mode="greedy", reference_check=False))
    return res.program


def _sibling_group(program):
    """GEMM kernels reading the same lhs over the same K (the in-projection's parts), with
    the accumulators each uses."""
    from torch_helion.hip.epilogue import match_epilogue

    by_lhs: dict = {}
    for k in program.kernels:
        if k.kind == "gemm" and k.gemms:
            by_lhs.setdefault((k.arg("lhs").tensor, k.k_extent), []).append(k)
    group = max(by_lhs.values(), key=len)
    assert len(group) >= 2, "the Mamba in-projection lowers to several GEMM kernels on one lhs"
    return [(k.name, len({o.a for o in match_epilogue(k).outs})) for k in group]


def test_merge_decision_follows_merged_launch_factor(mamba_program):
    """The merged price is the GEMM model of the concatenated weights times the fitted
    factor; the split price does not depend on it; a large enough factor turns the
    decision to split, and the plan report shows both prices."""
    from torch_helion.cost_models.hw_spec import HardwareSpec
    from torch_helion.optimizer.planner import launch_merge_report, price_launch_merges

    hw = HardwareSpec.load()
    assert hw.calibration.get("efficiency", {}).get("gemm_bf16"), "the shipped spec carries a bf16 GEMM fit"

    def with_factor(f):
        return dataclasses.replace(hw, raw={**hw.raw, "calibration": {**hw.calibration, "merged_launch_factor": f}})

    group = _sibling_group(mamba_program)
    one = price_launch_merges(mamba_program, [group], with_factor(1.0))[0]
    big = price_launch_merges(mamba_program, [group], with_factor(50.0))[0]
    assert big.split_us == pytest.approx(one.split_us)
    assert big.merged_us == pytest.approx(50.0 * one.merged_us)
    assert not big.merged and big.to_dict()["merged"] is False
    rep = launch_merge_report([one, big])
    assert f"{big.merged_us:,.1f}" in rep and f"{big.split_us:,.1f}" in rep
    assert rep.rstrip().endswith("| split |")


def test_counter_table_groups_by_symbol():
    """The counters tool's table: one row per kernel symbol (parameters dropped), averaged over
    its positions, longest total first; a dispatch above --split-us gets a row of its own."""
    from torch_helion.hip.counters import by_symbol

    def pos(sym, us, util, fetch):
        return {"symbol": sym, "duration_us": us, "mfma_util": util, "clock_ghz": 2.0, "FETCH_SIZE": fetch,
                "WRITE_SIZE": 1024.0}

    g = "void th::gemm<256, 1>(th::GemmK)"
    rows = by_symbol([pos(g, 90.0, 0.3, 2048.0), pos("th::carry(th::SsdK)", 20.0, 0.0, 1024.0), pos(g, 110.0, 0.5, 4096.0),
                      pos(g, 1800.0, 0.47, 8192.0)], split_us=1000.0).splitlines()
    assert rows[2] == "| `th::gemm<256, 1> (long)` | 1 | 1800.0 | 47.0% | 2.00 | 8.0 | 1.0 |"
    assert rows[3] == "| `th::gemm<256, 1>` | 2 | 100.0 | 40.0% | 2.00 | 3.0 | 1.0 |"
    assert rows[4] == "| `th::carry` | 1 | 20.0 | 0.0% | 2.00 | 1.0 | 1.0 |"
    assert len(by_symbol([pos(g, 90.0, 0.3, 2048.0), pos(g, 1800.0, 0.4, 2048.0)]).splitlines()) == 3
