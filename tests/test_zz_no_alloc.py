"""cmpext3_gemm_ex_noalloc: the same plan as cmpext3_gemm_ex with a workspace of
the size it asks for, run on the library's static scratch buffer instead.

Every case is called twice in a row, the second time with a smaller input (the
scratch keeps the first call's contents), and each output must equal, bit for
bit, cmpext3_gemm_ex's on a workspace allocated for it (the kernels are
deterministic and the plans are the same).  Cases cover each user of the
workspace: split-K fp32 partials of the skinny-M kernel, of the 16-bit tiles
and of the fp32 tiles, and zero-padded copies of unaligned 16-bit and fp32
operands; a call whose full plan needs more than the scratch holds runs the
plan cmpext3_gemm_ex runs with a workspace of the scratch's size.
"""
import numpy as np
import pytest
import torch

from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {cabi.F16: torch.float16, cabi.BF16: torch.bfloat16, cabi.F32: torch.float32}
TOL = {cabi.F16: O.TOLERANCE["fp16"], cabi.BF16: O.TOLERANCE["bf16"], cabi.F32: O.TOLERANCE["fp32"]}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


def operands(dtype, layout, M, N, K, batch, seed):
    g = torch.Generator().manual_seed(seed)
    bshape = (K, N) if layout == cabi.B_KN else (N, K)
    a = (torch.randn(batch, M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    b = (torch.randn(batch, *bshape, generator=g) / np.sqrt(K)).to(DT[dtype])
    bias = torch.randn(N, generator=g).to(DT[dtype])
    return a.cuda(), b.cuda(), bias.cuda()


def run_both(dtype, layout, M, N, K, batch, seed, with_bias):
    """(noalloc output, gemm_ex output with its own workspace, plan description)."""
    a, b, bias = operands(dtype, layout, M, N, K, batch, seed)
    ldb = N if layout == cabi.B_KN else K
    bias = bias if with_bias else None
    c_ref = torch.full((batch, M, N), float("nan"), dtype=DT[dtype], device="cuda")
    st, call = cabi.prepare(dtype, layout, a, K, M * K, b, ldb, K * N, c_ref, N, M * N, bias, M, N, K, batch)
    assert st == cabi.OK
    _, desc = cabi.describe(call)
    need = cabi.call_workspace_size(call)
    assert 0 < need <= cabi.SCRATCH_BYTES, (need, desc)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    st = cabi.gemm_ex(dtype, layout, a, K, M * K, b, ldb, K * N, c_ref, N, M * N, bias, M, N, K, batch, ws)
    assert st == cabi.OK, cabi.status_string(st)
    c = torch.full((batch, M, N), float("nan"), dtype=DT[dtype], device="cuda")
    st = cabi.gemm_ex_noalloc(dtype, layout, a, K, M * K, b, ldb, K * N, c, N, M * N, bias, M, N, K, batch)
    assert st == cabi.OK, cabi.status_string(st)
    torch.cuda.synchronize()
    # against the float64 oracle too (first batch entry)
    bt = O.to_f64(b[0].cpu()) if layout == cabi.B_KN else O.to_f64(b[0].cpu()).T
    ref = O.matmul_f64(O.to_f64(a[0].cpu()), bt)
    if bias is not None:
        ref = ref + O.to_f64(bias.cpu())[None, :]
    assert O.rel_frobenius(O.to_f64(c[0].cpu()), ref) <= TOL[dtype], desc
    return c, c_ref, desc


# (dtype, layout, first shape (M, N, K, batch), second smaller shape, bias, what the workspace holds)
CASES = [
    (cabi.F16, cabi.B_KN, (16, 8192, 8192, 1), (16, 2048, 4096, 1), False, "skinny split-K partials"),
    (cabi.BF16, cabi.B_KN, (16, 4096, 8192, 2), (8, 1024, 4096, 1), True, "skinny split-K, batched, bias"),
    (cabi.F16, cabi.B_NK, (256, 4096, 8192, 1), (256, 2048, 4096, 1), True, "tile split-K partials, bias"),
    (cabi.F32, cabi.B_KN, (16, 4096, 8192, 1), (16, 1024, 4096, 1), False, "fp32 split-K partials"),
    (cabi.F16, cabi.B_KN, (1000, 1000, 777, 1), (600, 520, 333, 1), False, "padded 16-bit copies"),
    (cabi.F32, cabi.B_KN, (2049, 2999, 3001, 1), (2500, 2501, 2502, 1), False, "padded fp32 copies"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[-1] for c in CASES])
def test_noalloc_matches_gemm_ex_twice(case):
    dtype, layout, first, second, with_bias, what = case
    descs = []
    for i, (M, N, K, batch) in enumerate((first, second)):
        c, c_ref, desc = run_both(dtype, layout, M, N, K, batch, seed=M + N + K + i, with_bias=with_bias)
        descs.append(desc)
        assert torch.equal(c, c_ref), (what, i, desc)
    keyword = "padded" if "padded" in what else "splits="
    assert all(keyword in d for d in descs), descs


def test_noalloc_plans_within_the_scratch_when_the_full_plan_needs_more():
    # fp16 6001^3 with odd rows: the zero-padded copies of A and B would take 2 x 72 MB, so
    # the call runs the plan cmpext3_gemm_ex runs with a 64 MiB workspace (here: no copies)
    M = N = K = 6001
    g = torch.Generator().manual_seed(11)
    a = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(torch.float16).cuda()
    b = (torch.randn(K, N, generator=g) / np.sqrt(K)).to(torch.float16).cuda()
    st, call = cabi.prepare(cabi.F16, cabi.B_KN, a, K, 0, b, N, 0, a, N, 0, None, M, N, K)
    assert st == cabi.OK and cabi.call_workspace_size(call) > cabi.SCRATCH_BYTES
    st, call = cabi.prepare(cabi.F16, cabi.B_KN, a, K, 0, b, N, 0, a, N, 0, None, M, N, K,
                            workspace_limit=cabi.SCRATCH_BYTES)
    assert st == cabi.OK
    need = cabi.call_workspace_size(call)
    assert 0 <= need <= cabi.SCRATCH_BYTES
    ws = torch.empty(cabi.SCRATCH_BYTES, dtype=torch.uint8, device="cuda")
    c_ref = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    st = cabi.gemm_ex(cabi.F16, cabi.B_KN, a, K, 0, b, N, 0, c_ref, N, 0, None, M, N, K, 1, ws)
    assert st == cabi.OK, cabi.status_string(st)
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    st = cabi.gemm_ex_noalloc(cabi.F16, cabi.B_KN, a, K, 0, b, N, 0, c, N, 0, None, M, N, K)
    assert st == cabi.OK, cabi.status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(c, c_ref)
    rows = [0, 1, 2999, M - 1]
    ref = O.matmul_f64(O.to_f64(a[rows].cpu()), O.to_f64(b.cpu()))
    assert O.rel_frobenius(O.to_f64(c[rows].cpu()), ref) <= TOL[cabi.F16]


def test_noalloc_on_a_side_stream():
    # the scratch is that of the stream's GPU; the call is queued on the stream given
    a, b, _ = operands(cabi.F16, cabi.B_KN, 16, 8192, 8192, 1, 9)
    c1 = torch.full((16, 8192), float("nan"), dtype=torch.float16, device="cuda")
    c2 = torch.full_like(c1, float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    assert cabi.gemm_ex_noalloc(cabi.F16, cabi.B_KN, a[0], 8192, 0, b[0], 8192, 0, c1, 8192, 0, None,
                                16, 8192, 8192, stream=side) == cabi.OK
    side.synchronize()
    ws = torch.empty(cabi.SCRATCH_BYTES, dtype=torch.uint8, device="cuda")
    assert cabi.gemm_ex(cabi.F16, cabi.B_KN, a[0], 8192, 0, b[0], 8192, 0, c2, 8192, 0, None,
                        16, 8192, 8192, 1, ws) == cabi.OK
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)


def test_noalloc_without_workspace_need_and_bad_arguments():
    # a plan that needs no workspace runs as cmpext3_gemm_ex does
    a, b, _ = operands(cabi.F16, cabi.B_KN, 512, 512, 512, 1, 5)
    c1 = torch.empty(512, 512, dtype=torch.float16, device="cuda")
    c2 = torch.empty_like(c1)
    assert cabi.gemm_ex_noalloc(cabi.F16, cabi.B_KN, a[0], 512, 0, b[0], 512, 0, c1, 512, 0, None,
                                512, 512, 512) == cabi.OK
    assert cabi.gemm_ex(cabi.F16, cabi.B_KN, a[0], 512, 0, b[0], 512, 0, c2, 512, 0, None, 512, 512, 512) == cabi.OK
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    # argument errors come back before any launch
    assert cabi.gemm_ex_noalloc(cabi.F16, cabi.B_KN, a[0], 100, 0, b[0], 512, 0, c1, 512, 0, None,
                                512, 512, 512) == cabi.ERR_INVALID_ARG
    assert cabi.gemm_ex_noalloc(9, cabi.B_KN, a[0], 512, 0, b[0], 512, 0, c1, 512, 0, None,
                                512, 512, 512) == cabi.ERR_UNSUPPORTED
