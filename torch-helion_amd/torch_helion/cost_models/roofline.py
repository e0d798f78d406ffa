"""Roofline cost model for OpIR kernels on MI355X.

Replaces the reference's mesh-cycle model (cost_models/analytic.py:109-266)
with what bounds a gfx950 kernel: ``max(MFMA time, HBM time)`` where

* MFMA time counts the work of whole block tiles (tile quantisation: a
  ragged edge tile costs a full tile) spread over 256 CUs in waves (wave
  quantisation: a partial last wave costs a full wave), at the dtype's dense
  peak times an achievable efficiency from ``hwspec``;
* HBM time is the kernel's algorithmic bytes at peak bandwidth times an
  efficiency;

plus a fixed launch overhead in microseconds. ``algorithmic`` FLOPs/bytes are
also reported; they are what bench.py's roofline fraction divides by.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass, field
from typing import Any

from ..capture.opgraph import DTYPE_BYTES, TensorType
from ..optimizer.opir import KernelSpec
from .hw_spec import HardwareSpec


class CostModelError(RuntimeError):
    pass


@dataclass
class CostBreakdown:
    us: float
    flops: float
    bytes: float
    bound: str
    tiles: dict[str, int] = field(default_factory=dict)
    blocks: int = 0
    waves: int = 0
    t_mfma_us: float = 0.0
    t_hbm_us: float = 0.0
    detail: dict[str, Any] = field(default_factory=dict)

    @property
    def cycles(self) -> float:
        """Kept for reports that expect the reference's ``cycles`` key: µs here."""
        return self.us

    def to_dict(self) -> dict[str, Any]:
        d = asdict(self)
        d["cycles"] = self.us
        return d


def _dtype(spec: KernelSpec, tensors: dict[str, TensorType]) -> str:
    for a in spec.args:
        t = tensors.get(a.tensor)
        if t is not None and a.role in ("lhs", "q", "x") and t.dtype.startswith(("bfloat", "float")):
            return t.dtype
    return "float32"


def _bytes(t: TensorType) -> int:
    return t.numel * DTYPE_BYTES.get(t.dtype, 4)


def gemm_tiles(N: int, n_acc: int, M: int, dtype: str, cus: int = 256) -> tuple[int, int]:
    """(BM, per-accumulator column tile) the HIP GEMM picks (mirrors th_gemm in csrc/gemm.hip:
    256-row tiles when they still give two blocks per CU, 128 when they give one, else 64;
    one accumulator over a multiple of 256 columns takes 256 x 256 tiles when they make
    whole waves)."""
    if dtype == "float32":
        bn = {1: 128 if N > 64 else 64, 2: 64 if N > 32 else 32, 3: 64}.get(n_acc, 64 if N > 32 else 32)
        return 64, bn
    bn = {1: 256 if N >= 2048 else (128 if N >= 768 else 64), 2: 128 if N >= 128 else (64 if N > 32 else 32),
          3: 64}.get(n_acc, 64 if N > 32 else 32)
    if n_acc == 1 and bn == 128 and N % 256 == 0:
        t256 = math.ceil(M / 256) * (N // 256)
        if t256 >= cus and t256 % cus == 0:    # whole waves of 256 x 256 tiles
            return 256, 256
    tn = math.ceil(N / bn)
    if math.ceil(M / 256) * tn >= 2 * cus:
        return 256, bn
    return (128 if math.ceil(M / 128) * tn >= cus else 64), bn


def category(spec: KernelSpec, tensors: dict[str, TensorType]) -> str:
    """Calibration category of a kernel: kernels of one category share an efficiency."""
    dtype = _dtype(spec, tensors)
    if spec.kind == "gemm":
        if not spec.gemms:
            return "norm"
        if tensors[spec.arg(spec.gemms[0].rhs).tensor].dtype == "float8_e4m3fn":
            return "gemm_fp8"
        return "gemm_fp32" if dtype == "float32" else "gemm_bf16"
    if spec.kind == "attention":
        return "attention_fp32" if dtype == "float32" else "attention"
    if spec.kind in ("ssd", "ssd_chunked"):
        return "ssd"
    return spec.kind


def _compose(hw: HardwareSpec, flops: float, nbytes: float, mfma_flops: float, blocks: int, dtype: str,
             tiles: dict[str, int], detail: dict[str, Any], cat: str, wave_scale: float = 1.0) -> CostBreakdown:
    """Time of the binding roofline. With a calibration fitted for ``cat``: ideal time at
    100% of peak over the fitted efficiency plus the fitted launch overhead, plus the fitted
    cost per wave of tiles times ``wave_scale`` (a GEMM tile's area relative to 256 x 256:
    its pipeline fill and epilogue); without one, the hardware spec's generic MFMA / HBM
    efficiencies and overhead."""
    calib = hw.calibration
    fitted = calib.get("efficiency", {}).get(cat)
    eff_m = fitted if fitted else hw.efficiency.get("mfma", 0.6)
    eff_h = fitted if fitted else hw.efficiency.get("hbm", 0.7)
    overhead = hw.launch_overhead_us
    if fitted:
        overhead = calib.get("fixed_us", {}).get(cat, calib.get("launch_overhead_us", hw.launch_overhead_us))
    waves = max(1, math.ceil(blocks / hw.compute_units)) if blocks else 1
    per_block = mfma_flops / max(blocks, 1)
    t_mfma = waves * per_block / (hw.peak_flops(dtype) / hw.compute_units * eff_m) * 1e6 if mfma_flops else 0.0
    t_hbm = nbytes / (hw.hbm_bytes_per_s() * eff_h) * 1e6
    us = max(t_mfma, t_hbm) + overhead
    if fitted:
        us += waves * wave_scale * calib.get("tile_us", {}).get(cat, 0.0)
    bound = "mfma" if t_mfma >= t_hbm else "hbm"
    detail = {**detail, "category": cat, "calibrated": bool(fitted), "wave_scale": wave_scale}
    return CostBreakdown(us, flops, nbytes, bound, tiles, blocks, waves, t_mfma, t_hbm, detail)


def gemm_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec) -> CostBreakdown:
    from ..hip.epilogue import fused_acc_count  # structural, no parameter values needed

    T, N, K = spec.grid["rows"], spec.grid["cols"], spec.k_extent
    dtype = _dtype(spec, tensors)
    eb = DTYPE_BYTES.get(dtype, 4)
    n_acc = fused_acc_count(spec) if spec.gemms else 0
    extras = [a for a in spec.args if a.role in ("extra", "scale", "gain")]
    # weight bytes at the weight's own type (e4m3 weights: one byte per element)
    wb = DTYPE_BYTES.get(tensors[spec.arg(spec.gemms[0].rhs).tensor].dtype, eb) if spec.gemms else eb
    nbytes = T * K * eb + n_acc * K * N * wb + sum(_bytes(tensors[a.tensor]) for a in extras) + len(spec.outputs) * T * N * eb
    if n_acc == 0:  # stand-alone normalisation: HBM bound
        return _compose(hw, 3.0 * T * K, nbytes, 0.0, 0, dtype, {"tile_t": 4}, {"n_acc": 0}, "norm")
    if wb == 1:
        # e4m3 weights (decode): a weight stream, bound by HBM; the MFMA term is the products at fp8 rate
        flops = 2.0 * T * N * K * n_acc
        return _compose(hw, flops, nbytes, flops, math.ceil(N / 64), "float8_e4m3fn", {"tile_n": 64},
                        {"n_acc": n_acc, "weights": "float8_e4m3fn"}, "gemm_fp8")
    return _gemm_compose(hw, T, N, K, n_acc, dtype, nbytes,
                         {"n_acc": n_acc, "sumsq": spec.sumsq, "extras": len(extras), "outputs": len(spec.outputs)})


def _gemm_compose(hw: HardwareSpec, T: int, N: int, K: int, n_acc: int, dtype: str, nbytes: float,
                  detail: dict[str, Any]) -> CostBreakdown:
    """bf16 / fp32 GEMM of T x (n_acc N) x K on the HIP kernel's tiles."""
    flops = 2.0 * T * N * K * n_acc
    bm, bn = gemm_tiles(N, n_acc, T, dtype, hw.compute_units)
    tiles_m, tiles_n = math.ceil(T / bm), math.ceil(N / bn)
    kq = math.ceil(K / (16 if dtype == "float32" else 64)) * (16 if dtype == "float32" else 64)
    if dtype == "float32" and tiles_m * tiles_n < hw.compute_units:
        # fp32 grids too small for the GPU: 32-row tiles, K split over about one
        # workgroup per CU (th_gemm's workspace path), a second pass sums the slices
        tiles_m = math.ceil(T / 32)
        ksg = max(1, min(math.ceil(hw.compute_units / (tiles_m * tiles_n)), math.ceil(K / 16), 64))
        mfma = 2.0 * tiles_m * 32 * tiles_n * bn * n_acc * kq
        return _compose(hw, flops, nbytes, mfma, tiles_m * tiles_n * ksg, dtype,
                        {"tile_t": 32, "tile_n": bn, "k_slices": ksg}, detail, "gemm_fp32",
                        wave_scale=32 * bn * n_acc / 65536.0)
    mfma = 2.0 * tiles_m * bm * tiles_n * bn * n_acc * kq
    return _compose(hw, flops, nbytes, mfma, tiles_m * tiles_n, dtype,
                    {"tile_t": bm, "tile_n": bn, "tile_k": 16 if dtype == "float32" else 64}, detail,
                    "gemm_fp32" if dtype == "float32" else "gemm_bf16", wave_scale=bm * bn * n_acc / 65536.0)


def merged_gemm_cost(specs: list[KernelSpec], used: list[int], tensors: dict[str, TensorType],
                     hw: HardwareSpec) -> CostBreakdown:
    """Sibling GEMM kernels (one lhs, one K) run as ONE launch: the used weight
    columns of every kernel concatenated into a single accumulator, each output
    on its own column window (hip/runtime.py's merged launch). ``used[i]``: the
    accumulators kernel i contributes."""
    s0 = specs[0]
    T, K = s0.grid["rows"], s0.k_extent
    dtype = _dtype(s0, tensors)
    eb = DTYPE_BYTES.get(dtype, 4)
    n_tot = sum(sp.grid["cols"] * u for sp, u in zip(specs, used))
    extras = {a.tensor for sp in specs for a in sp.args if a.role == "extra"}
    outs = sum(len(sp.outputs) * T * sp.grid["cols"] for sp in specs)
    nbytes = T * K * eb + n_tot * K * eb + sum(_bytes(tensors[t]) for t in extras) + outs * eb
    c = _gemm_compose(hw, T, n_tot, K, 1, dtype, nbytes, {"merged": [sp.name for sp in specs], "cols": n_tot})
    # Measured merged launches run slower than a plain GEMM of their shape (every output
    # window through the general LDS-staged epilogue, a partial last wave of wide tiles):
    # the calibration fits that as one factor over the merged launches it has seen.
    f = hw.calibration.get("merged_launch_factor")
    if f and c.detail.get("calibrated"):
        c.us *= f
        c.detail["merged_launch_factor"] = f
    return c


def attention_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec) -> CostBreakdown:
    a = spec.attrs
    b, s, h, d = a["batch"], a["seq"], a["heads"], a["head_dim"]
    hk = a.get("kv_heads", h)
    skv = a.get("seq_kv", s)
    dtype = _dtype(spec, tensors)
    eb = DTYPE_BYTES.get(dtype, 4)
    pairs = s * skv
    if a.get("causal"):
        pairs = sum(min(skv, i + 1 + skv - s) for i in range(s))
    flops = 4.0 * b * h * pairs * d
    nbytes = (2 * b * s * h * d + 2 * b * skv * hk * d) * eb
    qb = math.ceil(s / 128)
    blocks = b * h * qb
    kv_tiles = sum(math.ceil(min(skv, (i + 1) * 128 + skv - s) / 64) for i in range(qb)) if a.get("causal") else qb * math.ceil(skv / 64)
    mfma = 4.0 * b * h * 128 * 64 * d * kv_tiles
    return _compose(hw, flops, nbytes, mfma, blocks, dtype, {"tile_m": 128, "tile_n": 64}, {"kv_heads": hk},
                    "attention_fp32" if dtype == "float32" else "attention")


def attention_decode_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec) -> CostBreakdown:
    """One query row per (sequence, head) against pos cached rows plus the new one: the
    cache read dominates (HBM bound)."""
    a = spec.attrs
    b, h, d, pos = a["batch"], a["heads"], a["head_dim"], a["pos"]
    hk = a.get("kv_heads", h)
    dtype = _dtype(spec, tensors)
    eb = DTYPE_BYTES.get(dtype, 4)
    n = pos + 1
    flops = 4.0 * b * h * n * d
    nbytes = (2 * b * h * d + 2 * b * n * hk * d) * eb
    return _compose(hw, flops, nbytes, 0.0, b * hk, dtype, {}, {"kv_heads": hk, "keys": n}, "attention_decode")


def ssd_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec) -> CostBreakdown:
    a = spec.attrs
    b, s, h, p, n = a["batch"], a["seq"], a["heads"], a["head_dim"], a["state_dim"]
    q = a.get("chunk", 64)
    dtype = _dtype(spec, tensors)
    eb = DTYPE_BYTES.get(dtype, 4)
    # intra-chunk C B^T and M X, chunk states, carried-state output
    flops = 2.0 * b * h * s * (q * n + q * p + 2 * n * p)
    nbytes = sum(_bytes(tensors[x.tensor]) for x in spec.args) + len(spec.outputs) * b * s * h * p * eb
    blocks = b * h * max(1, math.ceil(s / q))
    return _compose(hw, flops, nbytes, flops, blocks, dtype, {"chunk": q}, {}, "ssd")


def elementwise_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec) -> CostBreakdown:
    dtype = _dtype(spec, tensors)
    nbytes = sum(_bytes(tensors[x.tensor]) for x in spec.args) + sum(_bytes(tensors[o.tensor]) for o in spec.outputs)
    a = spec.attrs
    flops = 2.0 * a.get("batch", 1) * a.get("seq", 1) * a.get("width", 1) * a.get("kernel", 1)
    return _compose(hw, flops, nbytes, 0.0, 0, dtype, {}, {}, spec.kind)


def gather_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec) -> CostBreakdown:
    """Embedding gather: only the looked-up rows of the table move (ids + rows in, rows out)."""
    dtype = _dtype(spec, tensors)
    out = tensors[spec.outputs[0].tensor]
    nbytes = 2 * _bytes(out) + _bytes(tensors[spec.arg("ids").tensor])
    return _compose(hw, 0.0, nbytes, 0.0, 0, dtype, {}, {}, "embedding")


def kernel_cost(spec: KernelSpec, tensors: dict[str, TensorType], hw: HardwareSpec, tiles: dict[str, int] | None = None) -> CostBreakdown:
    if spec.kind == "gemm":
        return gemm_cost(spec, tensors, hw)
    if spec.kind == "attention":
        return attention_cost(spec, tensors, hw)
    if spec.kind == "attention_decode":
        return attention_decode_cost(spec, tensors, hw)
    if spec.kind in ("ssd", "ssd_chunked"):
        return ssd_cost(spec, tensors, hw)
    if spec.kind == "conv1d":
        return elementwise_cost(spec, tensors, hw)
    if spec.kind == "embedding":
        return gather_cost(spec, tensors, hw)
    raise CostModelError(f"unknown kernel kind {spec.kind}")
