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


# ------------------------------------------------------------------ prepared calls (no GPU needed)
def _prep(dtype=cabi.F16, layout=cabi.B_KN, M=64, N=64, K=64, A=0x10000, B=0x20000, C=0x30000, bias=None,
          lda=None, ldb=None, ldc=None, batch=1, flags=0, limit=(1 << 63) - 1, strides=(0, 0, 0)):
    lda = max(K, 1) if lda is None else lda
    ldb = max(N if layout == cabi.B_KN else K, 1) if ldb is None else ldb
    ldc = max(N, 1) if ldc is None else ldc
    return cabi.prepare(dtype, layout, A, lda, strides[0], B, ldb, strides[1], C, ldc, strides[2], bias, M, N, K,
                        batch, flags, limit)


def test_prepared_call_matches_plan_query():
    for dtype, layout, M, N, K in [(cabi.F16, cabi.B_KN, 4096, 4096, 4096), (cabi.BF16, cabi.B_KN, 4096, 14336, 4096),
                                   (cabi.F16, cabi.B_KN, 16, 8192, 8192), (cabi.F32, cabi.B_KN, 4097, 3001, 2049),
                                   (cabi.F16, cabi.B_NK, 16, 4096, 14336), (cabi.F32, cabi.B_KN, 16, 8192, 8192)]:
        st, call = _prep(dtype, layout, M, N, K)
        assert st == cabi.OK
        kid, desc = cabi.describe(call)
        need = cabi.call_workspace_size(call)
        kid2, desc2 = cabi.plan(dtype, layout, M, N, K, workspace_bytes=need)
        assert (kid, desc) == (kid2, desc2)
        assert need == max(0, cabi.workspace_size(dtype, layout, M, N, K))


def test_prepared_call_limits_workspace():
    st, call = _prep(M=16, N=8192, K=8192, limit=0)
    assert st == cabi.OK and cabi.call_workspace_size(call) == 0 and "kernel=skinny " in cabi.describe(call)[1]
    st, call = _prep(M=16, N=8192, K=8192)
    assert "kernel=skinny_wide" in cabi.describe(call)[1] and cabi.call_workspace_size(call) == 4 * 16 * 8192 * 4


def test_linear_shape_gets_its_split_and_padding():
    # the workspace decisions linear takes through the bindings (weight as [N, K], bias per column)
    st, call = _prep(cabi.F16, cabi.B_NK, 512, 7168, 7168, bias=0x40000)
    kid, desc = cabi.describe(call)
    assert st == cabi.OK and "tile256x224" in desc and "splits=4" in desc, desc
    st, call = _prep(cabi.F16, cabi.B_NK, 512, 1999, 1001, bias=0x40000)
    kid, desc = cabi.describe(call)
    assert "padded=AB" in desc and "tile128x128" in desc, desc


def test_bias_alignment_does_not_steer_the_kernel():
    # a 2-byte aligned bias (e.g. bias[1:]) keeps the tiled kernel; only A, B and C count
    for bias in (0x40000, 0x40002, 0x40006):
        st, call = _prep(cabi.F16, cabi.B_NK, 4096, 4096, 4096, bias=bias)
        assert st == cabi.OK and "kernel=tile256x256" in cabi.describe(call)[1]
        st, call = _prep(cabi.BF16, cabi.B_KN, 16, 8192, 8192, bias=bias)
        assert "kernel=skinny_wide" in cabi.describe(call)[1]
    st, call = _prep(cabi.F16, cabi.B_NK, 4096, 4096, 4096, C=0x30002, bias=0x40000)
    assert "kernel=tile256x256" not in cabi.describe(call)[1]   # an unaligned C does


def test_fp32_output_pitch_bound():
    # fp32 kernels store C through 32-bit offsets from a tile base: 256 rows must fit
    st, _ = _prep(cabi.F32, cabi.B_KN, 64, 64, 64, ldc=(1 << 21))
    assert st == cabi.ERR_TOO_LARGE
    st, _ = _prep(cabi.F32, cabi.B_KN, 64, 64, 64, ldc=(1 << 21) - 1)
    assert st == cabi.OK
    st, _ = _prep(cabi.F16, cabi.B_KN, 64, 64, 64, ldc=(1 << 22))   # 16-bit epilogues use 64-bit pointers
    assert st == cabi.OK


def test_prepared_call_rejections():
    st, _ = _prep(flags=2)
    assert st == cabi.ERR_INVALID_ARG
    st, _ = _prep(M=-1)
    assert st == cabi.ERR_INVALID_ARG
    garbage = cabi.Call()
    assert cabi.call_workspace_size(garbage) == cabi.ERR_INVALID_ARG
    assert cabi.describe(garbage)[0] == cabi.ERR_INVALID_ARG
    assert cabi.run(garbage) == cabi.ERR_INVALID_ARG
    # a plan that needs workspace refuses to run without enough of it (before any launch)
    st, call = _prep(M=16, N=8192, K=8192)
    need = cabi.call_workspace_size(call)
    assert cabi.run(call, None, 0) == cabi.ERR_WORKSPACE
    assert cabi.run(call, 0x50000, need - 1) == cabi.ERR_WORKSPACE
    assert cabi.run(call, 0x50008, need) == cabi.ERR_WORKSPACE      # not 16-byte aligned
    assert cabi.status_string(cabi.ERR_WORKSPACE) != "unknown status"
    # empty problems run without touching anything
    st, call = _prep(M=0, A=None, B=None, C=None)
    assert st == cabi.OK and cabi.call_workspace_size(call) == 0 and cabi.run(call) == cabi.OK
    st, call = _prep(M=64, N=64, K=64, batch=0, A=None, B=None, C=None)
    assert st == cabi.OK and cabi.run(call) == cabi.OK
