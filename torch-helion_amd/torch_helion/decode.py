"""compile_model for the decode step: e4m3 weights and an ``attention_decode`` kernel in the OpIR.

The reference has no decode path (models/llama_block.py:82-105 has no KV
cache; capture/opgraph.py:26 has no fp8 type). A decode step is the block at
one query row per sequence, with the attention reading a cache. Its OpIR is
derived from the block's own capture:

1. the block is captured and canonicalised at S = 1 with the step's
   dequantised weights and RoPE tables at position ``pos`` (the ordinary
   capture -> OpGraph -> passes -> plan pipeline, which yields the q, k/v,
   attention, o, gate/up and down kernels with their fused epilogues);
2. every GEMM weight is replaced by its e4m3 form: the tensor becomes
   ``float8_e4m3fn`` ``[K, N]`` and the kernel gains an argument
   ``<rhs>_scale`` (role ``scale``, fp32 ``[N]``, W = q * s per column);
   weights the front end folded an RMSNorm gain into are taken back to the
   model's own and the gain becomes an argument ``gain`` (role ``gain``,
   ``[K]``: the products use lhs * g, the row sum of squares the unscaled
   lhs); the pre-rotated RoPE siblings are the same signed column
   permutation of the e4m3 values and scales;
3. the attention kernel becomes ``attention_decode``: arguments q, k_new,
   v_new (the projections of the new token) and the caches k_cache, v_cache
   (program inputs, token-major ``[B * L, Hkv * d]``), attrs ``pos``,
   ``max_len``; keys and values are the cache's first ``pos`` rows of each
   sequence followed by the new token's. k_new and v_new are program outputs;
   ``metadata["cache_slots"]`` tells the device runtime it may write them
   straight into the cache at row ``pos`` (what a serving loop keeps).
"""

from __future__ import annotations

import dataclasses
import time
from typing import Any

import torch

from .capture.opgraph import TensorType
from .optimizer.opir import KernelArg, KernelSpec, Program
from .optimizer.param_transforms import rotate_columns

FP8 = "float8_e4m3fn"


def _prefill_form(model, batch: int, config, run_dir):
    """Compile the block at S = 1 with the step's dequantised weights and pos-row RoPE tables.

    The decode module supplies that block itself (``model.prefill_block(batch)``,
    an nn.Module taking ``[batch, 1, hidden]``), so this module depends on no
    particular model class."""
    from .pipeline import compile_model

    blk = model.prefill_block(batch)
    x = torch.zeros(batch, 1, model.cfg.hidden, dtype=model.cfg.dtype)
    sub = dataclasses.replace(config, run_name="prefill_form", results_dir=run_dir, backend="none", bench=False,
                              reference_check=False, verify_passes=False, device_check=False)
    return compile_model(blk.eval(), (x,), sub)


def _match_weight(w_kn: torch.Tensor, model) -> tuple[str, bool]:
    """Which projection ``w_kn`` ([K, N]) is, and whether it is its RoPE-rotated copy."""
    cfg = model.cfg
    for short in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
        w = model.weight(short).T
        if w.shape == w_kn.shape and torch.equal(w.float(), w_kn.float()):
            return short, False
        if short in ("wq", "wk") and w.shape == w_kn.shape:
            heads = w.shape[1] // cfg.head_dim
            if torch.equal(rotate_columns(w.float(), heads, cfg.head_dim), w_kn.float()):
                return short, True
    raise ValueError("a GEMM weight of the prefill form matches no projection of the decode block")


def decode_program(model, batch: int, config, run_dir) -> tuple[Program, dict[str, torch.Tensor], Any]:
    """The decode step's Program and parameter values (see the module docstring)."""
    pre = _prefill_form(model, batch, config, run_dir)
    P, params_in, folds = pre.program, pre.graph.params, pre.graph.fold_sources
    cfg, pos, hd = model.cfg, model.pos, model.cfg.head_dim
    tensors = dict(P.tensors)
    params: dict[str, torch.Tensor] = {}
    kernels: list[KernelSpec] = []
    param_names = list(P.params)
    for k in P.kernels:
        k = KernelSpec.from_dict(k.to_dict())
        if k.kind == "gemm" and k.gemms:
            gains: list[torch.Tensor] = []
            for g in k.gemms:
                t = k.arg(g.rhs).tensor
                folded = t in folds
                w_kn = folds[t][1] if folded else params_in[t]
                short, rotated = _match_weight(w_kn, model)
                q = getattr(model, f"{short}_q").T.float()           # [K, N], e4m3 values
                s = getattr(model, f"{short}_s").float()[None, :]    # [1, N]
                if rotated:
                    heads = q.shape[1] // hd
                    q = rotate_columns(q, heads, hd)
                    s = rotate_columns(s, heads, hd).abs()
                params[t] = q.to(torch.float8_e4m3fn).contiguous()
                tensors[t] = TensorType(tuple(q.shape), FP8)
                sname = t + "_scale"
                params[sname] = s.reshape(-1).contiguous()
                tensors[sname] = TensorType((q.shape[1],), "float32")
                param_names.append(sname)
                k.args.append(KernelArg(g.rhs + "_scale", sname, "scale"))
                if folded:
                    gains.append(folds[t][0].float())
            if gains:
                # one gain multiplies the kernel's shared lhs, so it must hold for every product
                if len(gains) != len(k.gemms):
                    raise ValueError(f"{k.name}: {len(gains)} of {len(k.gemms)} GEMM weights carry a folded "
                                     "norm gain; a kernel's products must all carry it or none")
                gain = gains[0]
                if not all(g.shape == gain.shape and torch.equal(g, gain) for g in gains[1:]):
                    raise ValueError(f"{k.name}: the GEMM weights were folded with different norm gains")
                gname = f"{k.name}_gain"
                params[gname] = gain.reshape(-1).contiguous()
                tensors[gname] = TensorType((gain.numel(),), "float32")
                param_names.append(gname)
                k.args.append(KernelArg("gain", gname, "gain"))
        elif k.kind == "attention":
            a = k.attrs
            kv = a.get("kv_heads", a["heads"])
            q_t, k_t, v_t = (k.arg(r).tensor for r in ("q", "k", "v"))
            for name in ("k_cache", "v_cache"):
                tensors[name] = TensorType((batch * cfg.seq, kv * hd), str(cfg.dtype).replace("torch.", ""))
            k = KernelSpec(k.name.replace("attention", "attention_decode"), "attention_decode",
                           args=[KernelArg("q", q_t, "q"), KernelArg("k_cache", "k_cache", "k_cache"),
                                 KernelArg("v_cache", "v_cache", "v_cache"), KernelArg("k_new", k_t, "k_new"),
                                 KernelArg("v_new", v_t, "v_new")],
                           outputs=k.outputs,
                           attrs={"batch": batch, "heads": a["heads"], "kv_heads": kv, "head_dim": hd,
                                  "scale": a["scale"], "pos": pos, "max_len": cfg.seq},
                           notes=["attention over the cache's first pos rows and the new key/value"])
            k_new, v_new = k_t, v_t
        kernels.append(k)
    for t in P.params:
        if t not in params:
            params[t] = params_in[t]
    used = {a.tensor for k in kernels for a in k.args}
    param_names = [t for t in dict.fromkeys(param_names) if t in used]
    out = P.outputs[0]
    prog = Program(type(model).__name__, [P.inputs[0], "k_cache", "v_cache"], [out, k_new, v_new], tensors, kernels,
                   param_names, dict(P.metadata))
    prog.metadata["output_shapes"] = {out: [batch, cfg.hidden], k_new: [batch, cfg.n_kv, hd],
                                      v_new: [batch, cfg.n_kv, hd]}
    prog.metadata["decode"] = {"pos": pos, "max_len": cfg.seq, "batch": batch}
    prog.metadata["cache_slots"] = {k_new: {"cache": "k_cache", "pos": pos}, v_new: {"cache": "v_cache", "pos": pos}}
    return prog, params, pre


def compile_decode(model, example_args, config):
    """compile_model's path for a decode-step module (``model.is_decode_step``)."""
    from .codegen.emit import emit_program
    from .cost_models.hw_spec import HardwareSpec
    from .cost_models.roofline import kernel_cost
    from .pipeline import CompileResult, cost_report_json, cost_report_md, max_rel_err
    from .results import ResultsWriter

    rw = ResultsWriter(config.run_dir)
    timings: dict[str, float] = {}
    t0 = time.time()
    x, k_cache, v_cache = example_args
    batch = x.shape[0]
    rw.write_text("00_model.txt", f"{model!r}\n\ndecode step at pos {model.pos}\n\nconfig: {config!r}\n")
    prog, params, pre = decode_program(model, batch, config, rw.run_dir)
    hw = HardwareSpec.load(config.hw_spec)
    for k in prog.kernels:
        k.cost = kernel_cost(k, prog.tensors, hw).to_dict()
    prog.metadata.setdefault("plan", {})["total_us"] = sum(k.cost["us"] for k in prog.kernels)
    prog.to_json(rw.path("06_opir.json"))
    rw.write_text("06_opir.txt", prog.summary())
    timings["build"] = time.time() - t0
    kernel_files = emit_program(prog, config, rw.path("kernels"))
    device_program = None
    if config.backend == "hip":
        from .hip.runtime import DeviceProgram

        device_program = DeviceProgram(prog, params, config.device, fp32_outputs=config.fp32_outputs,
                                       residual_fp32=config.residual_fp32, reuse_buffers=config.reuse_buffers,
                                       merge_siblings=config.merge_siblings)
        rw.write_json("kernels/launches.json", [{"kernel": l.kernel, "entry": l.entry, "info": l.info}
                                                for l in device_program.launches])
    validation: dict[str, Any] = {}
    if device_program is not None and config.device_check:
        device_program.run([x, k_cache, v_cache])
        torch.cuda.synchronize()
        with torch.no_grad():
            refs = model(x, k_cache, v_cache)
        validation = {"outputs": []}
        ok = True
        for o, r in zip(device_program.outputs(fp32=True), refs):
            rel = max_rel_err(o.float().cpu().reshape(-1), r.float().reshape(-1))
            validation["outputs"].append({"max_rel_err": rel, "ok": rel <= config.tolerance})
            ok &= rel <= config.tolerance
        validation["ok"] = ok
        rw.write_json("07_validation.json", validation)
    rw.write_json("09_cost_report.json", cost_report_json(prog, hw, config))
    rw.write_text("09_cost_report.md", cost_report_md(prog, hw, config))
    rw.write_json("timings.json", timings)
    # the result's graph is the prefill form's, carrying the decode program's parameter values
    graph = pre.graph.copy()
    graph.params = params
    return CompileResult(config, rw.run_dir, pre.fx, pre.raw_graph, graph, hw, pre.plan, prog, kernel_files,
                         validation, {}, {}, timings, device_program)
