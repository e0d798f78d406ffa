"""C ABI of libth_hip.so on the CPU: exports, struct layouts, host-side validation.

No compute call is made here: every call either is a pure query or fails
host-side validation before any HIP call (or, for a valid descriptor on a
machine without a GPU, stops at the "th_init was not called" check).
"""

from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "th_hip.h"


@pytest.fixture(scope="module")
def lib():
    from torch_helion.hip import abi

    if not abi.library_path().exists():
        pytest.skip("libth_hip.so not built (run __graft_entry__.build())")
    return abi.load()


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(th_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported_and_bound(lib):
    from torch_helion.hip import abi

    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
        assert n in abi.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.th_abi_version() == abi.ABI_VERSION


_STRUCTS = {
    "th_epi_out": "EpiOut", "th_gemm_desc": "GemmDesc", "th_rmsnorm_desc": "RmsNormDesc",
    "th_attn_desc": "AttnDesc", "th_decode_desc": "DecodeDesc", "th_ssd_desc": "SsdDesc", "th_conv_desc": "ConvDesc",
    "th_embedding_desc": "EmbeddingDesc", "th_vm_operand": "VmOperand", "th_vm_op": "VmOp", "th_vm_out": "VmOut",
    "th_vm_desc": "VmDesc",
}


def test_struct_layouts_match_the_header(tmp_path):
    """Compile a C probe against include/th_hip.h and compare sizeof/offsetof with ctypes."""
    from torch_helion.hip import abi

    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "th_hip.h"', "int main(void){"]
    for cname, pyname in _STRUCTS.items():
        st = getattr(abi, pyname)
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in st._fields_:
            cf = "in" if (cname == "th_vm_desc" and fname == "in_") else fname
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {cf}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l.strip()}
    for cname, pyname in _STRUCTS.items():
        st = getattr(abi, pyname)
        assert got[(cname, "size")] == C.sizeof(st), cname
        for fname, _ in st._fields_:
            assert got[(cname, fname)] == getattr(st, fname).offset, (cname, fname)


def test_pure_queries(lib):
    from torch_helion.hip import abi

    assert lib.th_gemm_acc_tile(4096, 1, abi.TH_BF16) == 256
    assert lib.th_gemm_acc_tile(1024, 2, abi.TH_BF16) == 128
    assert lib.th_gemm_acc_tile(512, 3, abi.TH_BF16) == 64
    assert lib.th_gemm_acc_tile(0, 1, abi.TH_BF16) == 0
    # rows = ceil(N / tile) * tile * n_acc, K padded to 8 bf16 elements
    assert lib.th_gemm_packed_bytes(1000, 100, 2, abi.TH_BF16) == 8 * 128 * 2 * 104 * 2
    assert lib.th_gemm_packed_bytes(10, 10, 9, abi.TH_BF16) == -1
    # the scan's shared G^T tiles: 4 KiB each (32 x 32 fp32), nt (nt + 1) / 2 per chunk and
    # group, nt = chunk / 32; only state_dim 128 with several heads per group takes them
    base = lib.th_ssd_workspace_bytes(8, 2048, 32, 64, 128, 256)
    assert base == (2 * 8 * 32 * 8 * 64 * 128 + 8 * 32 * 8) * 4
    assert lib.th_ssd_gtile_workspace_bytes(8, 2048, 32, 64, 128, 256, 1) == base + 8 * 1 * 8 * 36 * 4096
    assert lib.th_ssd_gtile_workspace_bytes(2, 300, 6, 64, 128, 128, 2) == (
        lib.th_ssd_workspace_bytes(2, 300, 6, 64, 128, 128) + 2 * 2 * 3 * 10 * 4096)
    assert lib.th_ssd_gtile_workspace_bytes(8, 2048, 32, 64, 128, 256, 32) == base      # one head per group
    assert lib.th_ssd_gtile_workspace_bytes(2, 1024, 16, 64, 64, 64, 1) == lib.th_ssd_workspace_bytes(
        2, 1024, 16, 64, 64, 64)                                                           # state_dim 64
    assert lib.th_ssd_gtile_workspace_bytes(8, 2048, 32, 64, 128, 256, 5) == -1           # 32 heads, 5 groups


def _gemm_desc(**over):
    from torch_helion.hip import abi

    d = abi.GemmDesc()
    d.M = d.N = d.K = 64
    d.n_acc, d.in_dtype = 1, abi.TH_BF16
    d.lhs, d.ld_lhs, d.rhs_packed = 4096, 64, 8192
    d.n_out = 1
    d.out[0].ptr, d.out[0].ld, d.out[0].dtype = 12288, 64, abi.TH_BF16
    for k, v in over.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("window,ld,msg", [
    ((4, 32), 64, "multiples of 8"), ((32, 32), 64, "column window"), ((0, 72), 64, "column window"),
    ((16, 48), 24, "ld < its width"),
])
def test_gemm_rejects_bad_column_windows(lib, window, ld, msg):
    from torch_helion.hip import abi

    d = _gemm_desc()
    d.out[0].col_begin, d.out[0].col_end = window
    d.out[0].ld = ld
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_INVALID
    assert msg in abi.last_error(lib)


def test_gemm_column_windows_accepted_for_fp8(lib):
    """e4m3 weights take column windows too: a valid window passes every argument check (the
    call then stops at the missing device, not at the window)."""
    from torch_helion.hip import abi

    d = _gemm_desc(in_dtype=abi.TH_F8E4M3, rhs_scale=16384, workspace=20480, workspace_bytes=1 << 30)
    d.out[0].col_begin, d.out[0].col_end = 0, 32
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_NOT_INIT, abi.last_error(lib)


@pytest.mark.parametrize("field,value,msg", [
    ("n_acc", 7, "n_acc"), ("K", 60, "multiple of 8"), ("in_dtype", 2, "in_dtype"), ("n_out", 0, "n_out"),
    ("rscale_mask", 1, "without sumsq"), ("lhs", 4100, "aligned"),
])
def test_gemm_rejects_bad_descriptors(lib, field, value, msg):
    from torch_helion.hip import abi

    d = _gemm_desc(**{field: value})
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_INVALID
    assert msg in abi.last_error(lib)


def test_null_descriptors_are_rejected(lib):
    from torch_helion.hip import abi

    for fn in ("th_gemm", "th_rmsnorm", "th_attention_prefill", "th_attention_decode", "th_epilogue_vm", "th_ssd_chunked",
               "th_conv1d_causal", "th_embedding"):
        assert getattr(lib, fn)(None, None) == abi.TH_ERR_INVALID, fn
        assert "null descriptor" in abi.last_error(lib)


def test_attention_rejects_bad_heads(lib):
    from torch_helion.hip import abi

    d = abi.AttnDesc()
    d.batch, d.seq_q, d.seq_kv, d.heads_q, d.heads_kv, d.head_dim = 1, 16, 16, 6, 4, 64
    d.dtype = abi.TH_BF16
    d.q = d.k = d.v = d.o = 4096
    d.ld_q = d.ld_k = d.ld_v = d.ld_o = 384
    assert lib.th_attention_prefill(C.byref(d), None) == abi.TH_ERR_INVALID
    assert "multiple of heads_kv" in abi.last_error(lib)
    d.heads_q, d.head_dim = 4, 96
    assert lib.th_attention_prefill(C.byref(d), None) == abi.TH_ERR_INVALID
    assert "head_dim" in abi.last_error(lib)
    d.head_dim, d.scale = 64, -0.125  # the bf16 kernel folds a positive scale into exp2
    assert lib.th_attention_prefill(C.byref(d), None) == abi.TH_ERR_INVALID
    assert "scale > 0" in abi.last_error(lib)
    d.scale, d.ld_k = 0.125, 1 << 24  # the bf16 kernel keeps a tile's k/v row offsets in 32 bits
    assert lib.th_attention_prefill(C.byref(d), None) == abi.TH_ERR_INVALID
    assert "under 2^24" in abi.last_error(lib)


def test_attention_decode_rejects_wide_token_strides(lib):
    """The decode kernel keeps a 32-key tile's row offsets in 32 bits: cache token strides of
    2^24 elements or more are refused before any launch."""
    from torch_helion.hip import abi

    d = abi.DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.head_dim, d.max_len, d.fixed_len = 2, 8, 2, 128, 64, 64
    d.dtype, d.scale = abi.TH_BF16, 0.088
    d.q = d.k_cache = d.v_cache = d.o = 4096
    d.ld_q = d.ld_o = 8 * 128
    d.k_stride_t = d.v_stride_t = 1 << 24
    d.k_stride_b = d.v_stride_b = (1 << 24) * 64
    assert lib.th_attention_decode(C.byref(d), None) == abi.TH_ERR_INVALID
    assert "under 2^24" in abi.last_error(lib), abi.last_error(lib)
    d.k_stride_t = d.v_stride_t = 256
    d.k_stride_b = d.v_stride_b = 256 * 64
    assert lib.th_attention_decode(C.byref(d), None) == abi.TH_ERR_NOT_INIT, abi.last_error(lib)


def test_valid_descriptor_without_init_stops_before_the_device(lib):
    import torch
    from torch_helion.hip import abi

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; this checks the GPU-less error path")
    d = _gemm_desc()
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_NOT_INIT
    assert "th_init" in abi.last_error(lib)


def test_product_raises_without_a_device():
    """The runtime refuses to bind a program to a non-HIP device (no host fallback)."""
    from torch_helion.hip import abi
    from torch_helion.hip.runtime import DeviceProgram
    from torch_helion.optimizer.opir import Program

    prog = Program("p", [], [], {}, [])
    with pytest.raises(abi.HipBackendError):
        DeviceProgram(prog, {}, device=__import__("torch").device("cpu"))


def test_fp8_gemm_validation(lib):
    """e4m3 weights: at most 128 rows, K a multiple of 32, per-column scales required."""
    from torch_helion.hip import abi

    for over, msg in (({"M": 129}, "at most 128 rows"), ({"K": 48}, "K % 32"), ({}, "rhs_scale")):
        d = _gemm_desc(in_dtype=abi.TH_F8E4M3, **over)
        assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_INVALID, over
        assert msg in abi.last_error(lib), (over, abi.last_error(lib))
    # e4m3 packs whole 32-K chunks
    assert lib.th_gemm_packed_bytes(256, 40, 1, abi.TH_F8E4M3) == 256 * 64  # K padded to 32-wide chunks
    assert lib.th_gemm_workspace_bytes(64, 4096, 4096, 1, abi.TH_BF16) == 0
    assert lib.th_gemm_workspace_bytes(64, 4096, 4096, 1, abi.TH_F8E4M3) > 0


def test_fp8_gemm_rope_outputs_on_two_accumulators(lib):
    """e4m3 weights: fused-RoPE outputs rotating two different accumulators over the same
    columns pass every check (the epilogues gather one rotation partner per accumulator; the
    GPU test rope_qk checks the values)."""
    from torch_helion.hip import abi

    d = _gemm_desc(in_dtype=abi.TH_F8E4M3, rhs_scale=16384, workspace=20480, workspace_bytes=1 << 30, n_acc=2, n_out=2,
                   rope_cos=24576, rope_sin=28672, rope_head_dim=32, rope_period=1)
    for o, a in ((0, 0), (1, 1)):
        d.out[o].op, d.out[o].a, d.out[o].b, d.out[o].e = abi.EPI_ROPE, a, -1, -1
        d.out[o].ptr, d.out[o].ld, d.out[o].dtype = 12288 + 4096 * o, 64, abi.TH_BF16
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_NOT_INIT, abi.last_error(lib)
    d.out[1].a = 0
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_NOT_INIT, abi.last_error(lib)


def test_lhs_gain_only_for_fp8(lib):
    """The activation-side gain is an e4m3-weight feature: a bf16 descriptor carrying one is
    unsupported, an e4m3 one passes the checks; the gain must be 16-byte aligned."""
    from torch_helion.hip import abi

    d = _gemm_desc(lhs_gain=32768)
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_UNSUPPORTED
    assert "lhs_gain" in abi.last_error(lib)
    d = _gemm_desc(in_dtype=abi.TH_F8E4M3, rhs_scale=16384, workspace=20480, workspace_bytes=1 << 30, lhs_gain=32772)
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_INVALID
    d.lhs_gain = 32768
    assert lib.th_gemm(C.byref(d), None) == abi.TH_ERR_NOT_INIT, abi.last_error(lib)


def test_gemm_noalloc_refuses_oversized_scratch(lib):
    """th_gemm_noalloc checks the fixed scratch size before anything else (here, before the
    missing device): 128 rows x 4096 e4m3 columns at K = 131072 need more than it holds."""
    from torch_helion.hip import abi

    d = _gemm_desc(in_dtype=abi.TH_F8E4M3, rhs_scale=16384, M=128, N=4096, K=131072, ld_lhs=131072)
    assert lib.th_gemm_workspace_bytes(128, 4096, 131072, 1, abi.TH_F8E4M3) > abi.GEMM_NOALLOC_SCRATCH_BYTES
    assert lib.th_gemm_noalloc(C.byref(d), None) == abi.TH_ERR_INVALID
    assert "scratch" in abi.last_error(lib), abi.last_error(lib)
    assert lib.th_gemm_noalloc(None, None) == abi.TH_ERR_INVALID


def test_embedding_validation(lib):
    """Token ids are int64 or int32; strides cover the row; an empty batch is a no-op."""
    from torch_helion.hip import abi

    def desc(**over):
        d = abi.EmbeddingDesc()
        d.tokens, d.dim, d.vocab, d.dtype, d.ids_dtype = 16, 64, 100, abi.TH_BF16, abi.TH_I64
        d.table, d.ld_table, d.ids, d.out, d.ld_out = 4096, 64, 8192, 12288, 64
        for k, v in over.items():
            setattr(d, k, v)
        return d

    for over, msg in (({"ids_dtype": abi.TH_F32}, "ids dtype"), ({"dtype": abi.TH_F16}, "dtype"),
                      ({"ld_out": 32}, "row stride"), ({"vocab": 0}, "bad sizes"), ({"table": 0}, "null operand"),
                      ({"out32": 4096, "ld_out32": 8}, "out32 row stride")):
        d = desc(**over)
        assert lib.th_embedding(C.byref(d), None) == abi.TH_ERR_INVALID, over
        assert msg in abi.last_error(lib), (over, abi.last_error(lib))
    d = desc(tokens=0, table=0, ids=0, out=0)
    assert lib.th_embedding(C.byref(d), None) == abi.TH_OK
