"""ctypes mirror of ``include/th_hip.h`` and loader of ``libth_hip.so``.

The structures below follow the header field by field (the CPU test
``tests/test_abi.py`` compiles the header with gcc and compares every
offset). The library is loaded lazily, after ``import torch``, so it binds to
the HIP runtime torch has already mapped.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

from .build import LIB_PATH

ABI_VERSION = 7

# th_status
TH_OK = 0
TH_ERR_INVALID = -1
TH_ERR_UNSUPPORTED = -2
TH_ERR_HIP = -3
TH_ERR_NOT_INIT = -4

# th_dtype
TH_F32, TH_BF16, TH_F16, TH_F8E4M3, TH_I32, TH_I64 = range(6)

# th_epi_op
EPI_ACC, EPI_ROPE, EPI_ROPE_PAIR, EPI_SILU, EPI_SWIGLU, EPI_ADD, EPI_SOFTPLUS_ADD, EPI_MUL = range(8)

MAX_ACC, MAX_OUT, MAX_EXTRA = 4, 6, 4
GEMM_NOALLOC_SCRATCH_BYTES = 32 << 20
VM_MAX_IN, VM_MAX_OPS, VM_MAX_OUT = 16, 96, 8

# th_vm_code
(VM_LOAD, VM_ADD, VM_SUB, VM_MUL, VM_DIV, VM_MAX, VM_POW, VM_EXP, VM_LOG,
 VM_ROW_SUM, VM_ROW_MAX, VM_COPY) = range(12)

TORCH_TO_TH = {"float32": TH_F32, "bfloat16": TH_BF16, "float16": TH_F16, "float8_e4m3fn": TH_F8E4M3,
               "int32": TH_I32, "int64": TH_I64}

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64


class EpiOut(C.Structure):
    _fields_ = [("op", _i32), ("a", _i32), ("b", _i32), ("e", _i32), ("ptr", _p), ("ld", _i64),
                ("dtype", _i32), ("col_begin", _i32), ("col_end", _i32), ("pad_", _i32)]


class GemmDesc(C.Structure):
    _fields_ = [
        ("M", _i64), ("N", _i64), ("K", _i64),
        ("n_acc", _i32), ("in_dtype", _i32),
        ("lhs", _p), ("ld_lhs", _i64), ("rhs_packed", _p),
        ("sumsq", _i32), ("rscale_mask", C.c_uint32), ("inv_k", C.c_float), ("eps", C.c_float),
        ("n_extra", _i32), ("pad_", _i32),
        ("extra", _p * MAX_EXTRA), ("ld_extra", _i64 * MAX_EXTRA), ("extra_dtype", _i32 * MAX_EXTRA),
        ("rope_cos", _p), ("rope_sin", _p),
        ("rope_head_dim", _i32), ("rope_period", _i32), ("n_out", _i32), ("pad2_", _i32),
        ("out", EpiOut * MAX_OUT),
        ("sumsq_out", _p),
        ("rhs_scale", _p), ("workspace", _p), ("workspace_bytes", _i64),
        ("lhs_gain", _p),
        ("rs_parts", _p), ("ld_rs_parts", _i64), ("n_rs_parts", _i32), ("pad3_", _i32),
        ("gain_out", _p), ("ss_parts_out", _p), ("ld_ss_parts_out", _i64), ("gain_out_index", _i32), ("pad4_", _i32),
    ]


class RmsNormDesc(C.Structure):
    _fields_ = [
        ("M", _i64), ("K", _i64),
        ("x", _p), ("ld_x", _i64), ("x_dtype", _i32), ("out_dtype", _i32),
        ("gain", _p), ("out", _p), ("ld_out", _i64), ("inv_k", C.c_float), ("eps", C.c_float),
        ("out32", _p), ("ld_out32", _i64),
    ]


class AttnDesc(C.Structure):
    _fields_ = [
        ("batch", _i32), ("seq_q", _i32), ("seq_kv", _i32), ("heads_q", _i32), ("heads_kv", _i32),
        ("head_dim", _i32), ("scale", C.c_float), ("causal", _i32), ("dtype", _i32), ("pad_", _i32),
        ("q", _p), ("ld_q", _i64), ("k", _p), ("ld_k", _i64), ("v", _p), ("ld_v", _i64),
        ("o", _p), ("ld_o", _i64),
    ]


class DecodeDesc(C.Structure):
    _fields_ = [
        ("batch", _i32), ("heads_q", _i32), ("heads_kv", _i32), ("head_dim", _i32),
        ("max_len", _i32), ("n_split", _i32), ("fixed_len", _i32), ("dtype", _i32),
        ("scale", C.c_float), ("pad_", _i32), ("lengths", _p),
        ("q", _p), ("ld_q", _i64),
        ("k_cache", _p), ("k_stride_b", _i64), ("k_stride_t", _i64),
        ("v_cache", _p), ("v_stride_b", _i64), ("v_stride_t", _i64),
        ("o", _p), ("ld_o", _i64), ("workspace", _p), ("workspace_bytes", _i64),
    ]


class SsdDesc(C.Structure):
    _fields_ = [
        ("batch", _i32), ("seq", _i32), ("heads", _i32), ("head_dim", _i32), ("state_dim", _i32), ("ngroups", _i32),
        ("chunk", _i32), ("dtype", _i32),
        ("x", _p), ("ld_x", _i64), ("b", _p), ("ld_b", _i64), ("c", _p), ("ld_c", _i64), ("dt", _p), ("ld_dt", _i64),
        ("dt_stride", _i32), ("pad_", _i32),
        ("cum", _p), ("ld_cum", _i64), ("A", _p), ("D", _p), ("dskip", _p), ("ld_dskip", _i64),
        ("gate", _p), ("ld_gate", _i64), ("gate_dtype", _i32), ("y_dtype", _i32),
        ("y", _p), ("ld_y", _i64), ("y32", _p), ("ld_y32", _i64), ("workspace", _p), ("workspace_bytes", _i64),
        ("y_gain", _p), ("rs_parts", _p), ("ld_rs_parts", _i64),
    ]


class ConvDesc(C.Structure):
    _fields_ = [
        ("batch", _i32), ("seq", _i32), ("width", _i32), ("kernel", _i32), ("activation", _i32),
        ("x_dtype", _i32), ("y_dtype", _i32), ("pad_", _i32),
        ("x", _p), ("ld_x", _i64), ("w", _p), ("y", _p), ("ld_y", _i64), ("y32", _p), ("ld_y32", _i64),
    ]


class EmbeddingDesc(C.Structure):
    _fields_ = [
        ("tokens", _i64), ("dim", _i32), ("vocab", _i32), ("dtype", _i32), ("ids_dtype", _i32),
        ("table", _p), ("ld_table", _i64), ("ids", _p), ("out", _p), ("ld_out", _i64),
        ("out32", _p), ("ld_out32", _i64), ("n_invalid", _p),
    ]


class VmOperand(C.Structure):
    _fields_ = [("ptr", _p), ("ld", _i64), ("dtype", _i32), ("column", _i32)]


class VmOp(C.Structure):
    _fields_ = [("code", _i32), ("dst", _i32), ("a", _i32), ("b", _i32), ("scalar", C.c_float), ("mode", _i32)]


class VmOut(C.Structure):
    _fields_ = [("ptr", _p), ("ld", _i64), ("dtype", _i32), ("slot", _i32)]


class VmDesc(C.Structure):
    _fields_ = [
        ("M", _i64), ("N", _i64),
        ("n_in", _i32), ("n_ops", _i32), ("n_out", _i32), ("n_slots", _i32),
        ("in_", VmOperand * VM_MAX_IN), ("ops", VmOp * VM_MAX_OPS), ("out", VmOut * VM_MAX_OUT),
        ("workspace", _p),
    ]


# entry point name -> (restype, argtypes); every symbol include/th_hip.h declares
SIGNATURES: dict[str, tuple] = {
    "th_abi_version": (_i32, []),
    "th_init": (_i32, [_i32]),
    "th_last_error": (C.c_char_p, []),
    "th_gemm_acc_tile": (_i32, [_i64, _i32, _i32]),
    "th_gemm_packed_bytes": (_i64, [_i64, _i64, _i32, _i32]),
    "th_gemm_pack_rhs": (_i32, [C.POINTER(_p), C.POINTER(_i64), _i32, _i64, _i64, _i32, _i32, _p, _p]),
    "th_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "th_gemm": (_i32, [C.POINTER(GemmDesc), _p]),
    "th_gemm_noalloc": (_i32, [C.POINTER(GemmDesc), _p]),
    "th_rmsnorm": (_i32, [C.POINTER(RmsNormDesc), _p]),
    "th_attention_prefill": (_i32, [C.POINTER(AttnDesc), _p]),
    "th_attention_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "th_attention_decode": (_i32, [C.POINTER(DecodeDesc), _p]),
    "th_epilogue_vm": (_i32, [C.POINTER(VmDesc), _p]),
    "th_ssd_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "th_ssd_gtile_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "th_ssd_chunked": (_i32, [C.POINTER(SsdDesc), _p]),
    "th_conv1d_causal": (_i32, [C.POINTER(ConvDesc), _p]),
    "th_embedding": (_i32, [C.POINTER(EmbeddingDesc), _p]),
}


class HipBackendError(RuntimeError):
    """A libth_hip.so entry point returned an error status."""

    def __init__(self, entry: str, status: int, message: str, kernel: str | None = None) -> None:
        where = f" [{kernel}]" if kernel else ""
        super().__init__(f"{entry}{where} failed with status {status}: {message}")
        self.entry, self.status, self.kernel = entry, status, kernel


_LIB: C.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def load(path: str | Path | None = None) -> C.CDLL:
    """Load libth_hip.so (raises if it has not been built)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise HipBackendError("load", TH_ERR_NOT_INIT,
                              f"{p} is missing; build it with __graft_entry__.build() "
                              f"or python torch-helion_amd/torch_helion/hip/build.py")
    import torch  # noqa: F401  -- map torch's HIP runtime first (one runtime per process)

    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.th_abi_version() != ABI_VERSION:
        raise HipBackendError("load", TH_ERR_INVALID, f"ABI version {lib.th_abi_version()} != {ABI_VERSION}")
    if path is None:
        _LIB = lib
    return lib


def last_error(lib: C.CDLL | None = None) -> str:
    lib = lib or load()
    return (lib.th_last_error() or b"").decode(errors="replace")


def check(status: int, entry: str, kernel: str | None = None) -> None:
    if status != TH_OK:
        raise HipBackendError(entry, status, last_error(), kernel)


_INIT: set[int] = set()


def init_device(device: int) -> C.CDLL:
    lib = load()
    if device not in _INIT:
        check(lib.th_init(device), "th_init")
        _INIT.add(device)
    return lib
