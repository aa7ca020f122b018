"""The C-ABI library loads on a machine without a GPU, exports every symbol
include/cmpext3_gemm.h declares, and rejects bad arguments before launching."""
import ctypes
import os
import re

import pytest

from cmp_ext_amd import cabi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "cmpext3_gemm.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cmpext3_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    for s in ["cmpext3_matmul_fp16", "cmpext3_matmul_bf16", "cmpext3_matmul_fp32", "cmpext3_gemm_f16",
              "cmpext3_gemm_bf16", "cmpext3_gemm_f32", "cmpext3_gemm_ex",
              "cmpext3_gemm_workspace_size", "cmpext3_gemm_plan", "cmpext3_status_string", "cmpext3_version"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(cabi.LIB_PATH)
    for s in declared_symbols():
        assert hasattr(lib, s), s
    assert set(declared_symbols()) == set(cabi.SIGNATURES), "ctypes table out of sync with the header"


def test_version_and_status_strings():
    assert b"gfx950" in cabi.lib().cmpext3_version()
    assert cabi.status_string(0) == "success"
    for st in (cabi.ERR_INVALID_ARG, cabi.ERR_UNSUPPORTED, cabi.ERR_TOO_LARGE):
        assert cabi.status_string(st) != "unknown status"
    assert cabi.status_string(-99) == "unknown status"


@pytest.mark.parametrize("kw,err", [
    (dict(M=-1), cabi.ERR_INVALID_ARG),
    (dict(dtype=9), cabi.ERR_UNSUPPORTED),
    (dict(layout=5), cabi.ERR_UNSUPPORTED),
    (dict(lda=1), cabi.ERR_INVALID_ARG),
    (dict(A=None), cabi.ERR_INVALID_ARG),     # null operand with work to do
    (dict(C=None), cabi.ERR_INVALID_ARG),
])
def test_gemm_ex_rejects_before_launch(kw, err):
    args = dict(dtype=cabi.F16, layout=cabi.B_KN, A=0x1000, lda=64, stride_a=0, B=0x2000, ldb=64, stride_b=0,
                C=0x3000, ldc=64, stride_c=0, bias=None, M=64, N=64, K=64, batch=1)
    args.update(kw)
    st = cabi.lib().cmpext3_gemm_ex(args["dtype"], args["layout"], args["A"], args["lda"], args["stride_a"],
                                    args["B"], args["ldb"], args["stride_b"], args["C"], args["ldc"],
                                    args["stride_c"], args["bias"], args["M"], args["N"], args["K"],
                                    args["batch"], None, 0, None)
    assert st == err


def test_empty_problems_launch_nothing():
    lib = cabi.lib()
    # M == 0, N == 0 or batch == 0: success without touching the (null) pointers or the GPU
    assert lib.cmpext3_gemm_ex(cabi.F16, cabi.B_KN, None, 8, 0, None, 8, 0, None, 8, 0, None, 0, 8, 8, 1, None, 0,
                               None) == 0
    assert lib.cmpext3_gemm_ex(cabi.F32, cabi.B_KN, None, 8, 0, None, 8, 0, None, 8, 0, None, 8, 0, 8, 1, None, 0,
                               None) == 0
    assert lib.cmpext3_gemm_ex(cabi.BF16, cabi.B_NK, None, 8, 0, None, 8, 0, None, 8, 0, None, 8, 8, 8, 0, None, 0,
                               None) == 0
    assert lib.cmpext3_matmul_fp16(None, None, None, 0, 0, 0, None) == 0
    assert lib.cmpext3_gemm_bf16(None, 8, None, 8, None, 8, 8, 0, 8, None) == 0
    # skinny-M shapes with no columns or no batch entries (the split-K planner divides by both)
    assert lib.cmpext3_gemm_ex(cabi.F16, cabi.B_KN, None, 8, 0, None, 8, 0, None, 8, 0, None, 8, 0, 8, 1, None, 0,
                               None) == 0
    assert lib.cmpext3_gemm_ex(cabi.F16, cabi.B_KN, None, 8, 0, None, 8, 0, None, 8, 0, None, 8, 8, 8, 0, None, 0,
                               None) == 0
    assert cabi.workspace_size(cabi.F16, cabi.B_KN, 16, 0, 8192) == 0
    assert cabi.workspace_size(cabi.BF16, cabi.B_KN, 16, 8192, 8192, batch=0) == 0


def test_strided_entry_points_check_pitches():
    lib = cabi.lib()
    # pitches below the row length are rejected before any launch
    assert lib.cmpext3_gemm_f16(0x1000, 63, 0x2000, 64, 0x3000, 64, 64, 64, 64, None) == cabi.ERR_INVALID_ARG
    assert lib.cmpext3_gemm_bf16(0x1000, 64, 0x2000, 32, 0x3000, 64, 64, 64, 64, None) == cabi.ERR_INVALID_ARG
    assert lib.cmpext3_gemm_f32(0x1000, 64, 0x2000, 64, 0x3000, 60, 64, 64, 64, None) == cabi.ERR_INVALID_ARG
    assert lib.cmpext3_gemm_f32(0x1000, 64, 0x2000, 64, None, 64, 64, 64, 64, None) == cabi.ERR_INVALID_ARG


def test_workspace_size_query():
    # decode shape: 128-column strips x 4 K splits of fp32 partials
    assert cabi.workspace_size(cabi.F16, cabi.B_KN, 16, 8192, 8192) == 4 * 16 * 8192 * 4
    assert cabi.workspace_size(cabi.F16, cabi.B_KN, 4096, 4096, 4096) == 0   # tiled kernel: none
    # fp32 has no skinny kernel: few tiles and a long K split K over the fp32 tiles
    kid, desc = cabi.plan(cabi.F32, cabi.B_KN, 16, 8192, 8192, workspace_bytes=1 << 30)
    splits = int(desc.split("splits=")[1].split()[0])
    assert splits > 1 and cabi.workspace_size(cabi.F32, cabi.B_KN, 16, 8192, 8192) == splits * 16 * 8192 * 4
    assert cabi.workspace_size(cabi.F16, cabi.B_KN, 16, 32768, 4096) == 0    # enough strips: no split
    assert cabi.workspace_size(7, cabi.B_KN, 16, 64, 64) == cabi.ERR_UNSUPPORTED


def test_conv2d_1x1_rejects_and_empty():
    lib = cabi.lib()
    # negative sizes and unknown dtypes are rejected before any launch
    assert lib.cmpext3_conv2d_1x1(cabi.F16, 0x1000, 0x2000, None, 0x3000, -1, 8, 8, 64, None, 0, None) == \
        cabi.ERR_INVALID_ARG
    assert lib.cmpext3_conv2d_1x1(cabi.F16, 0x1000, 0x2000, None, 0x3000, 1, 8, -8, 64, None, 0, None) == \
        cabi.ERR_INVALID_ARG
    assert lib.cmpext3_conv2d_1x1(5, 0x1000, 0x2000, None, 0x3000, 1, 8, 8, 64, None, 0, None) == \
        cabi.ERR_UNSUPPORTED
    assert lib.cmpext3_conv2d_1x1(cabi.F32, 0x1000, 0x2000, None, None, 1, 8, 8, 64, None, 0, None) == \
        cabi.ERR_INVALID_ARG                                         # null output with work to do
    # empty batch / no pixels / no output channels: success, nothing touched
    assert lib.cmpext3_conv2d_1x1(cabi.F16, None, None, None, None, 0, 8, 8, 64, None, 0, None) == cabi.OK
    assert lib.cmpext3_conv2d_1x1(cabi.BF16, None, None, None, None, 2, 8, 8, 0, None, 0, None) == cabi.OK
    assert lib.cmpext3_conv2d_1x1(cabi.F32, None, None, None, None, 2, 8, 0, 64, None, 0, None) == cabi.OK
