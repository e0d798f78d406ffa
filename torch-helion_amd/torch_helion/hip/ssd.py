"""Lowering of the scan and convolution kinds to th_ssd_chunked / th_conv1d_causal.

``ssd_chunked`` (dt [T, H], A, D per head) and the reference's ``ssd`` kind
(padded cum/dt, full D constant, reference optimizer/passes.py:528-610) run on
the same scan kernel. An epilogue of the form ``acc * e`` (the Mamba gate
``y * silu(z)``, reference results/mamba_block k4_ssd) is fused as the
kernel's gate; any other epilogue runs on the epilogue VM from an fp32 copy.
"""

from __future__ import annotations

import torch

from ..optimizer.opir import KernelSpec
from . import abi, ops
from .epilogue import build_trees


def _gate_of(spec: KernelSpec) -> tuple[str | None, bool]:
    """(extra arg name, fused) for an epilogue that is exactly ``acc * extra``."""
    if not spec.epilogue:
        return None, True
    trees = build_trees(spec)
    if len(spec.outputs) != 1:
        return None, False
    e = trees[spec.outputs[0].value]
    if len(e) == 4 and e[0] == "mul" and not dict(e[1]):
        for x, y in ((e[2], e[3]), (e[3], e[2])):
            if x == ("acc", 0) and y[0] == "extra":
                return y[1], True
    return None, False


def lower_ssd(dp, spec: KernelSpec):
    from .runtime import Launch

    a = spec.attrs
    bs, s, h, p, n = a["batch"], a["seq"], a["heads"], a["head_dim"], a["state_dim"]
    buf = lambda role: dp.buffers[spec.arg(role).tensor]
    x, bm, cm, dt = buf("x"), buf("b"), buf("c"), buf("dt")
    kw: dict = dict(batch=bs, seq=s, heads=h, head_dim=p, state_dim=n)
    if spec.kind == "ssd_chunked":
        A = buf("A").float().contiguous()
        # The scan splits decay exponents at block boundaries and needs each part <= 0,
        # which holds when the running sum of dt*A never increases: A <= 0 with dt >= 0
        # (Mamba's A = -exp(A_log), dt = softplus(.)). A is a parameter: check it here.
        if not bool((A <= 0).all()):
            raise abi.HipBackendError("lower", abi.TH_ERR_UNSUPPORTED,
                                      "ssd_chunked needs A <= 0 for every head (the running sum of dt*A "
                                      "must not increase)", spec.name)
        kw.update(ngroups=a.get("ngroups", h), chunk=int(a.get("chunk", 64)), dt_stride=1,
                  A=A, D=buf("D").float().contiguous())
    else:
        mask = dp._host(spec.arg("mask").tensor)
        if mask is None or not torch.equal(mask.float(), torch.ones(s, s).tril()):
            raise abi.HipBackendError("lower", abi.TH_ERR_UNSUPPORTED, "ssd mask is not the causal lower triangle", spec.name)
        # The ssd kind takes cum as an operand: it must be non-increasing along each
        # sequence (a running sum of dt*A with dt*A <= 0), which the scan's split decay
        # exponents rely on. Known at lowering only when cum is a parameter.
        cum_host = dp._host(spec.arg("cum").tensor)
        if cum_host is not None:
            c = cum_host.float().reshape(bs, s, -1)
            if s > 1 and not bool((c[:, 1:] <= c[:, :-1]).all()):
                raise abi.HipBackendError("lower", abi.TH_ERR_UNSUPPORTED,
                                          "ssd needs cum non-increasing along the sequence (a running sum of "
                                          "dt*A with dt*A <= 0)", spec.name)
        kw.update(ngroups=h, chunk=64 if s % 64 == 0 or s > 64 else s, dt_stride=int(a["pad"]), cum=buf("cum"),
                  dskip=buf("dskip"))
    gate_arg, fused = _gate_of(spec)
    # (with room for the chunks' G^T tiles: shared by the heads of a B/C group)
    ws = dp._workspace((ops.ssd_workspace_bytes(bs, s, h, p, n, kw["chunk"], kw["ngroups"]) + 3) // 4)
    out_name = spec.outputs[0].tensor if spec.outputs else None
    if fused:
        out = dp.buffers[out_name]
        gate = dp.operand(spec.arg(gate_arg).tensor) if gate_arg else None
        out32 = dp.shadow.get(out_name)
        info = {"gate": gate_arg is not None, "chunk": kw["chunk"]}
        fold = dp._norm_folds.get(spec.name)
        if fold is not None:
            # The only reader normalises this output with a gain: store y times the gain
            # and the per-32-column sums of squares of y; that GEMM takes this buffer as
            # its normalised lhs and applies the row scale from the sums.
            kw["y_gain"] = fold["gain"].float().reshape(-1).to(dp.device).contiguous()
            kw["rs_parts"] = dp._device_buffer((bs * s, h * p // 32), torch.float32, dp._last.get(out_name, dp._cur))
            dp._normed[fold["key"]] = out
            dp._rs_parts[fold["key"]] = kw["rs_parts"]
            info["norm_gain_for"] = fold["gemm"]

        def run() -> None:
            ops.ssd_chunked(x=x, b=bm, c=cm, dt=dt, out=out, workspace=ws, gate=gate, out32=out32, kernel=spec.name, **kw)

        return [Launch(spec.name, spec.kind, run, "th_ssd_chunked", info)]
    acc = dp._workspace(bs * s * h * p).view(bs * s, h * p)

    def run_acc() -> None:
        ops.ssd_chunked(x=x, b=bm, c=cm, dt=dt, out=acc, workspace=ws, kernel=spec.name, **kw)

    launches = [Launch(spec.name, spec.kind, run_acc, "th_ssd_chunked", {"vm": True})]
    launches.append(dp._vm_launch(spec, {"acc": acc}, None, None))
    return launches


def lower_conv1d(dp, spec: KernelSpec):
    from .runtime import Launch

    a = spec.attrs
    x = dp.buffers[spec.arg("x").tensor]
    host_w = dp._host(spec.arg("w").tensor)
    w = (host_w if host_w is not None else dp.buffers[spec.arg("w").tensor]).float().contiguous().to(dp.device)
    act = a.get("activation")
    if not spec.epilogue and len(spec.outputs) == 1 and spec.outputs[0].value == "acc":
        name = spec.outputs[0].tensor
        out, out32 = dp.buffers[name], dp.shadow.get(name)

        def run() -> None:
            ops.conv1d_causal(x, w, out, batch=a["batch"], seq=a["seq"], activation=act, out32=out32, kernel=spec.name)

        return [Launch(spec.name, "conv1d", run, "th_conv1d_causal", {"activation": act})]
    acc = dp._workspace(x.shape[0] * a["width"]).view(x.shape[0], a["width"])

    def run_acc() -> None:
        ops.conv1d_causal(x, w, acc, batch=a["batch"], seq=a["seq"], activation=act, kernel=spec.name)

    return [Launch(spec.name, "conv1d", run_acc, "th_conv1d_causal", {"vm": True}),
            dp._vm_launch(spec, {"acc": acc}, None, None)]
