"""GPU parity of the gfx950 GEMM kernels against the float64 CPU oracle.

Every kernel family the selector can pick is exercised (the coverage test at
the end checks that), through the Python binding (`cmpext3`) and through the
C ABI (ctypes on libcmpext3_gemm.so).  Error bounds are the operator
contract's relative Frobenius bounds: fp32 1e-5, fp16 2e-3, bf16 1e-2.

The five benchmark configurations are checked at full size three ways:
sampled rows against the float64 oracle, every element against a PyTorch fp32
GEMM on the GPU (within the same bound), and the column/row sums of C against
the exact (1^T A) B and A (B 1) in float64.
"""
import numpy as np
import pytest
import torch

import cmpext3
from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
CODE = {"fp16": cabi.F16, "bf16": cabi.BF16, "fp32": cabi.F32}
MATMUL = {"fp16": cmpext3.fp16_matmul, "bf16": cmpext3.bf16_matmul, "fp32": cmpext3.fp32_matmul}
KERNEL_NAMES = ["tile256x256", "tile256x224", "tile128x128", "tile64x256", "skinny", "skinny_wide", "skinny_nk",
                "f32tile128x128",
                "f32tile64x64", "f32tile96x64", "f32tile64x64k4", "f32tile16x64k4", "generic64x64", "stream64x128",
                "stream128x128", "tall"]
SEEN_KERNELS = set()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


def kernel_of(desc):
    return desc.split()[0].split("=")[1]


def launched():
    """(kernel, description) of what the last operator call on this thread ran --
    its real plan, from the pointers, pitches and workspace of that call."""
    desc = cmpext3.last_plan()
    SEEN_KERNELS.add(kernel_of(desc))
    return kernel_of(desc), desc


def cabi_call(dtype, layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, M, N, K, batch=1,
              workspace=None):
    """cmpext3_gemm_prepare (with the workspace at hand) + cmpext3_gemm_run through the
    C ABI; returns (status, kernel, description) of the plan that ran."""
    limit = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st, call = cabi.prepare(dtype, layout, A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c, bias, M, N, K,
                            batch, 0, limit)
    if st != cabi.OK:
        return st, None, None
    _, desc = cabi.describe(call)
    SEEN_KERNELS.add(kernel_of(desc))
    return cabi.run(call, workspace), kernel_of(desc), desc


def err_vs_oracle(out, a, b, dtype, bias=None, layout="KN"):
    return O.reference_check(out.cpu(), a.cpu(), b.cpu(), dtype, bias.cpu() if bias is not None else None, layout)


def run_matmul(dtype, M, N, K, seed=0, dist="normal", scale=None):
    scale = scale if scale is not None else 1.0 / max(1.0, np.sqrt(K))
    a, b = O.make_inputs(dtype, M, N, K, dist, scale, seed)
    ag, bg = a.cuda(), b.cuda()
    out = MATMUL[dtype](ag, bg)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and out.dtype == DT[dtype]
    return a, b, out


# ---------------------------------------------------------------- edge shapes
GENERIC_SHAPES = [(1, 1, 1), (3, 5, 7), (65, 33, 17), (100, 7, 33), (129, 257, 65), (2, 300, 9)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K", GENERIC_SHAPES)
def test_generic_ragged(dtype, M, N, K):
    a, b, out = run_matmul(dtype, M, N, K, seed=M + N + K)
    assert launched()[0] in ("generic64x64", "skinny")
    assert err_vs_oracle(out, a, b, dtype) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K,kernel", [
    (512, 512, 512, "tile128x128"),
    (300, 200, 72, "tile128x128"),       # M, N and K tails
    (130, 8, 8, "tile128x128"),
    (2048, 4096, 1000, "tile128x128"),   # two workgroups per CU
    (1000, 1000, 776, "tile128x128"),    # ragged, K not a multiple of 64
    (64, 32768, 128, "tile128x128"),     # M <= 64 with 256 column tiles
    (16, 32768, 264, "tile128x128"),
    (256, 4096, 4096, "tile128x128"),    # few tiles, long K: split K (fp32 partials + reduce)
    (200, 1000, 3000, "tile128x128"),    # ... ragged, last split shorter
    (512, 7168, 7168, "tile256x224"),    # 256-row tiles with K split 4 ways
    (8192, 1024, 14336, "tile256x256"),  # ... and 2 ways
    (64, 65536, 512, "tile64x256"),      # M <= 64, short K, 256 tiles of 256 columns
    (40, 70000, 200, "tile64x256"),      # ragged rows, columns and K
    (4000, 4088, 1000, "tile256x256"),   # ragged 256x256 tiles
    (4000, 14000, 520, "tile256x224"),   # ragged 256x224 tiles
])
def test_tiled_shapes(dtype, M, N, K, kernel):
    a, b, out = run_matmul(dtype, M, N, K, seed=7)
    name, desc = launched()
    assert name == kernel, desc
    if M * N * K > 2e9:  # keep the float64 oracle cheap: sampled rows + fp32 GPU reference
        rows = torch.randperm(M, generator=torch.Generator().manual_seed(1))[:96].sort().values
        e = O.rel_frobenius(O.to_f64(out.cpu()[rows]), O.matmul_f64(O.to_f64(a[rows]), O.to_f64(b)))
        assert e <= O.TOLERANCE[dtype]
        ref = torch.matmul(a.cuda().float(), b.cuda().float())
        e2 = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
        assert e2 <= O.TOLERANCE[dtype]
    else:
        assert err_vs_oracle(out, a, b, dtype) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K", [(1, 8192, 1024), (16, 256, 8192), (17, 200, 72), (33, 96, 40),
                                   (64, 1024, 512), (5, 8, 8), (48, 8200, 2056)])
def test_skinny(dtype, M, N, K):
    """Binding (wide strips + split K when a workspace helps) and C ABI without
    workspace (narrow strips) both against the oracle."""
    a, b, out = run_matmul(dtype, M, N, K, seed=M)
    assert launched()[0] in ("skinny", "skinny_wide")
    assert err_vs_oracle(out, a, b, dtype) <= O.TOLERANCE[dtype]
    c = torch.empty(M, N, dtype=DT[dtype], device="cuda")
    st, name, desc = cabi_call(CODE[dtype], cabi.B_KN, a.cuda(), K, 0, b.cuda(), N, 0, c, N, 0, None, M, N, K)
    assert st == cabi.OK and name in ("skinny", "skinny_wide"), desc   # no workspace: wide only unsplit
    assert "splits=1 " in desc or name == "skinny", desc
    torch.cuda.synchronize()
    assert err_vs_oracle(c, a, b, dtype) <= O.TOLERANCE[dtype]


def test_skinny_split_k_repeated_and_concurrent():
    """Split-K skinny products (fp32 partials in the workspace, summed by a
    second launch): many calls in a row, batched calls, and calls on two
    streams at once, each with its own workspace, must all give the same bits
    as the first call, and match the oracle."""
    a, b = O.make_inputs("fp16", 16, 1024, 8192, "normal", 8192 ** -0.5, 3)
    ag, bg = a.cuda(), b.cuda()
    ref = cmpext3.fp16_matmul(ag, bg)
    name, desc = launched()
    assert name == "skinny_wide" and "splits=1 " not in desc, desc
    torch.cuda.synchronize()
    assert err_vs_oracle(ref, a, b, "fp16") <= O.TOLERANCE["fp16"]
    mismatches = torch.zeros((), dtype=torch.int64, device="cuda")
    for _ in range(2000):
        mismatches += (cmpext3.fp16_matmul(ag, bg) != ref).sum()
    assert mismatches.item() == 0
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        o1 = [cmpext3.fp16_matmul(ag, bg) for _ in range(50)]
    with torch.cuda.stream(s2):
        o2 = [cmpext3.fp16_matmul(ag, bg) for _ in range(50)]
    torch.cuda.synchronize()
    assert all(torch.equal(o, ref) for o in o1 + o2)
    # batched: every batch entry has its own block of partial sums
    a3 = torch.stack([ag, ag * 0.5, -ag])
    b3 = torch.stack([bg, bg, bg * 2])
    o3 = cmpext3.bmm(a3, b3)
    name, desc = launched()
    assert name == "skinny_wide" and "splits=1 " not in desc, desc
    torch.cuda.synchronize()
    for i in range(3):
        assert err_vs_oracle(o3[i], a3[i], b3[i], "fp16") <= O.TOLERANCE["fp16"]


# Split-K reductions into every store form: N % 8 == 4 (four columns per
# thread), C pitches and batch strides that do not keep 16-byte stores aligned
# (element stores), per-column bias, both B layouts and all three dtypes.
SPLIT_CASES = [
    # dtype, layout, M, N, K, ldc, batch, stride_c, bias
    ("fp16", "NK", 256, 1028, 8192, 1028, 1, 0, False),            # 128x128 tiles, 4 columns, 8-byte stores
    ("bf16", "KN", 16, 1024, 8192, 1027, 1, 0, True),              # skinny_wide, odd pitch
    ("bf16", "KN", 16, 8000, 8192, 8003, 1, 0, True),              # skinny_wide, half a strip, element stores
    ("fp16", "KN", 20, 8192, 8192, 8192, 1, 0, True),              # skinny_wide, 2 row blocks, 8-byte stores
    ("fp16", "KN", 16, 1024, 8192, 1024, 3, 16 * 1024 + 4, False),  # batch stride off the 16-byte grid
    ("fp16", "KN", 256, 4096, 4096, 4100, 1, 0, True),             # 128x128 tiles, pitch off the grid
    ("bf16", "NK", 256, 2052, 4096, 2052, 1, 0, True),             # W as [N, K], 4 columns per thread
    ("fp32", "KN", 16, 1028, 14336, 1028, 1, 0, False),            # fp32 16x64 tiles, 16-byte stores
    ("fp32", "NK", 130, 1000, 4100, 1001, 1, 0, True),             # fp32 tiles, element stores
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "-".join(str(x) for x in c))
def test_split_k_reduction_store_forms(case):
    """cmpext3_gemm_ex with a workspace on products that split K: the reduction of
    the fp32 partials writes C (plus bias) exactly where the pitches say, leaves the
    gaps between rows and batch entries untouched, and matches the float64 oracle."""
    dtype, layout, M, N, K, ldc, batch, stride_c, has_bias = case
    lay = cabi.B_KN if layout == "KN" else cabi.B_NK
    ldb = N if layout == "KN" else K
    ws_bytes = cabi.workspace_size(CODE[dtype], lay, M, N, K, batch)
    g = torch.Generator().manual_seed(M + N + K)
    bshape = (K, N) if layout == "KN" else (N, K)
    a = (torch.randn(batch, M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    b = (torch.randn(batch, *bshape, generator=g) / np.sqrt(K)).to(DT[dtype])
    bias = torch.randn(N, generator=g).to(DT[dtype]) if has_bias else None
    stride_c = stride_c or M * ldc
    sentinel = 7.0
    cbuf = torch.full((stride_c * (batch - 1) + M * ldc + 8,), sentinel, dtype=DT[dtype], device="cuda")
    ws = torch.empty(ws_bytes // 4 + 4, dtype=torch.float32, device="cuda")
    ag, bg = a.cuda(), b.cuda()
    st, name, desc = cabi_call(CODE[dtype], lay, ag, K, M * K, bg, ldb, K * N, cbuf, ldc, stride_c,
                               None if bias is None else bias.cuda(), M, N, K, batch, workspace=ws)
    assert st == cabi.OK, cabi.status_string(st)
    assert "splits=" in desc and "splits=1 " not in desc, desc
    torch.cuda.synchronize()
    cpu = cbuf.cpu()
    written = torch.zeros(cpu.numel(), dtype=torch.bool)
    for i in range(batch):
        rows = torch.arange(M).unsqueeze(1) * ldc + torch.arange(N).unsqueeze(0) + i * stride_c
        written[rows.reshape(-1)] = True
        out = cpu[rows]
        bt = O.to_f64(b[i]) if layout == "KN" else O.to_f64(b[i]).T
        ref = O.matmul_f64(O.to_f64(a[i]), bt)
        if bias is not None:
            ref = ref + O.to_f64(bias)[None, :]
        assert O.rel_frobenius(O.to_f64(out), ref) <= O.TOLERANCE[dtype], (i, desc)
    assert (cpu[~written] == sentinel).all(), "a store landed outside C's rows"


@pytest.mark.parametrize("M,N,K,kernel", [(512, 512, 512, "f32tile64x64k4"), (65, 47, 3, "f32tile64x64"),
                                          (1, 1, 1, "f32tile64x64"), (6144, 8192, 64, "f32tile128x128"),
                                          (257, 131, 129, "f32tile64x64k4"), (1023, 2001, 129, "f32tile64x64"),
                                          (301, 257, 777, "f32tile64x64k4"),
                                          (1440, 768, 200, "f32tile96x64"), (1439, 767, 201, "f32tile96x64")])
def test_fp32(M, N, K, kernel):
    a, b, out = run_matmul("fp32", M, N, K, seed=3, dist="uniform")
    name, desc = launched()
    assert name == kernel, desc
    assert err_vs_oracle(out, a, b, "fp32") <= O.TOLERANCE["fp32"]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_k_zero_and_empty(dtype):
    a = torch.zeros(5, 0, dtype=DT[dtype], device="cuda")
    b = torch.zeros(0, 8, dtype=DT[dtype], device="cuda")
    out = MATMUL[dtype](a, b)
    torch.cuda.synchronize()
    assert out.shape == (5, 8) and not out.any()
    out = MATMUL[dtype](torch.zeros(0, 4, dtype=DT[dtype], device="cuda"), torch.ones(4, 3, dtype=DT[dtype], device="cuda"))
    assert out.shape == (0, 3)
    w = torch.zeros(6, 0, dtype=DT[dtype], device="cuda")
    bias = torch.arange(6, dtype=DT[dtype], device="cuda")
    out = cmpext3.linear(torch.zeros(2, 3, 0, dtype=DT[dtype], device="cuda"), w, bias)
    torch.cuda.synchronize()
    assert out.shape == (2, 3, 6)
    assert torch.equal(out, bias.expand(2, 3, 6))


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_exact_small_integers(dtype):
    """Small-integer products are exact in every kernel: bit equality with the oracle."""
    g = torch.Generator().manual_seed(5)
    for M, N, K in [(300, 200, 72), (16, 64, 64), (7, 9, 11), (4096, 256, 64)]:
        a = torch.randint(-3, 4, (M, K), generator=g).to(DT[dtype])
        b = torch.randint(-3, 4, (K, N), generator=g).to(DT[dtype])
        out = MATMUL[dtype](a.cuda(), b.cuda()).cpu()
        ref = O.matmul_f64(O.to_f64(a), O.to_f64(b))
        assert np.array_equal(O.to_f64(out), ref)


def test_fp16_overflow_matches_rounding():
    a = torch.full((4, 1), 300.0, dtype=torch.float16, device="cuda")
    b = torch.full((1, 8), 300.0, dtype=torch.float16, device="cuda")
    out = cmpext3.fp16_matmul(a, b).cpu()
    assert torch.isinf(out).all()   # 90000 is beyond fp16's range, as in O.round_fp16


# ------------------------------------------------------- layouts, views, bias
@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("shape", [(2, 150, 72, 200), (1, 4096, 4096, 4096), (3, 7, 40, 12), (1, 16, 64, 64),
                                   (1, 2048, 512, 1004), (1, 4096, 512, 3588), (2, 2048, 1024, 3588),
                                   (1, 16, 14336, 4096), (1, 1, 4096, 4096), (2, 16, 520, 1000),
                                   (1, 64, 2048, 256),   # the four above: decode shapes, skinny kernel on W [N,K]
                                   (1, 512, 7168, 7168)])  # split K on 256x224 tiles, bias in the reduction
def test_linear_with_bias(dtype, shape):
    Bt, S, K, N = shape
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(Bt, S, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    w = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    bias = torch.randn(N, generator=g).to(DT[dtype])
    out = cmpext3.linear(x.cuda(), w.cuda(), bias.cuda())
    torch.cuda.synchronize()
    assert out.shape == (Bt, S, N)
    name, desc = launched()
    if shape == (1, 512, 7168, 7168) and dtype != "fp32":  # the binding's workspace: 256x224 tiles split K
        assert name == "tile256x224" and "splits=4" in desc, desc
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w), O.to_f64(bias))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    out_nb = cmpext3.linear(x.cuda(), w.cuda())
    assert O.rel_frobenius(O.to_f64(out_nb.cpu()), O.linear_f64(O.to_f64(x), O.to_f64(w))) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_skinny_linear_weight_binding_and_c_abi(dtype):
    """Decode-shaped Linear: W [N, K] through the skinny kernel for that layout, from
    the binding and from the C ABI (same kernel, same bits), against the oracle."""
    M, N, K = 16, 4096, 4096
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    w = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w))
    out = cmpext3.linear(x.cuda(), w.cuda())
    assert launched()[0] == "skinny_nk"
    c = torch.empty(M, N, dtype=DT[dtype], device="cuda")
    st, name, _ = cabi_call(CODE[dtype], cabi.B_NK, x.cuda(), K, 0, w.cuda(), K, 0, c, N, 0, None, M, N, K)
    assert st == cabi.OK and name == "skinny_nk"
    torch.cuda.synchronize()
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    assert torch.equal(out, c)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K,bias", [(24, 14336, 4096, True), (33, 12800, 2056, False), (64, 14336, 4096, True)])
def test_skinny_nk_wide_strips(dtype, M, N, K, bias):
    """Decode-shaped Linear with 17..64 rows of x and a tall W: 64-row W strips (two to
    four 16-row blocks of x, 128- or 256-k stages), ragged M and K, with and without a
    column bias, against the oracle; deterministic."""
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    w = torch.randn(N, K, generator=g).to(DT[dtype])
    b = torch.randn(N, generator=g).to(DT[dtype]) if bias else None
    print(f"skinny_nk {dtype} M={M} N={N} K={K} bias={bias}", flush=True)
    out = cmpext3.linear(x.cuda(), w.cuda(), None if b is None else b.cuda())
    name, desc = launched()
    assert name == "skinny_nk" and "x64 " in desc, desc
    torch.cuda.synchronize()
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w), None if b is None else O.to_f64(b))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    again = cmpext3.linear(x.cuda(), w.cuda(), None if b is None else b.cuda())
    assert torch.equal(out, again)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K,splits", [(1, 1024, 14336, 4), (24, 512, 14336, 8), (64, 1000, 8200, 4),
                                          (64, 2048, 14336, 2), (40, 4096, 10248, 4)])
def test_skinny_nk_split_k(dtype, M, N, K, splits):
    """Decode-shaped Linear with few strips of W and long rows: K split over workgroups
    (fp32 partials, then the reduction adds the column bias and rounds), against the
    oracle; repeated calls bit-identical."""
    g = torch.Generator().manual_seed(M + N + K)
    x = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype]).cuda()
    w = torch.randn(N, K, generator=g).to(DT[dtype]).cuda()
    b = torch.randn(N, generator=g).to(DT[dtype]).cuda()
    print(f"skinny_nk split {dtype} M={M} N={N} K={K}", flush=True)
    out = cmpext3.linear(x, w, b)
    name, desc = launched()
    assert name == "skinny_nk" and f"splits={splits} " in desc, desc
    torch.cuda.synchronize()
    ref = O.linear_f64(O.to_f64(x.cpu()), O.to_f64(w.cpu()), O.to_f64(b.cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    for _ in range(3):
        assert torch.equal(out, cmpext3.linear(x, w, b))


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_skinny_nk_split_k_batched_c_abi(dtype):
    """The split over a batch through the C ABI (grid.z = batch x splits, partials per
    split and entry), C rows 8 apart wider than N, each entry against the oracle."""
    g = torch.Generator().manual_seed(5)
    Bn, M, N, K = 3, 16, 256, 14336
    a = (torch.randn(Bn, M, K, generator=g) / np.sqrt(K)).to(DT[dtype]).cuda()
    w = torch.randn(Bn, N, K, generator=g).to(DT[dtype]).cuda()
    c = torch.full((Bn, M, N + 8), float("nan"), dtype=DT[dtype], device="cuda")
    ws = torch.empty(1 << 24, dtype=torch.uint8, device="cuda")
    print(f"skinny_nk split C ABI {dtype} {Bn}x{M}x{N}x{K}", flush=True)
    st, name, desc = cabi_call(CODE[dtype], cabi.B_NK, a, K, M * K, w, K, N * K, c, N + 8, M * (N + 8), None,
                               M, N, K, Bn, workspace=ws)
    assert st == cabi.OK and name == "skinny_nk" and "splits=" in desc, desc
    torch.cuda.synchronize()
    got = c.cpu()
    assert torch.isnan(got[:, :, N:].float()).all()
    for i in range(Bn):
        ref = O.linear_f64(O.to_f64(a[i].cpu()), O.to_f64(w[i].cpu()))
        assert O.rel_frobenius(O.to_f64(got[i, :, :N]), ref) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_tall_split_k(dtype):
    """Narrow B with long K over few strips: the tall kernel with K split (fp32 partials,
    the reduction adds the bias and rounds) -- a router-shaped Linear with a column bias
    (B as [N, K], 8 ways) and a batched bmm with B as [K, N] (4 ways) -- against the
    oracle; repeated calls bit-identical."""
    g = torch.Generator().manual_seed(31)
    dt = DT[dtype]
    x = (torch.randn(1024, 14336, generator=g) / np.sqrt(14336)).to(dt).cuda()
    w = torch.randn(16, 14336, generator=g).to(dt).cuda()
    b = torch.randn(16, generator=g).to(dt).cuda()
    print(f"tall split linear {dtype} 1024x16x14336", flush=True)
    out = cmpext3.linear(x, w, b)
    name, desc = launched()
    assert name == "tall" and "splits=8 " in desc, desc
    torch.cuda.synchronize()
    ref = O.linear_f64(O.to_f64(x.cpu()), O.to_f64(w.cpu()), O.to_f64(b.cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    assert torch.equal(out, cmpext3.linear(x, w, b))
    p = (torch.randn(2, 1024, 8200, generator=g) / np.sqrt(8200)).to(dt).cuda()
    v = torch.randn(2, 8200, 64, generator=g).to(dt).cuda()
    print(f"tall split bmm {dtype} 2x1024x64x8200", flush=True)
    out = cmpext3.bmm(p, v)
    name, desc = launched()
    assert name == "tall" and "splits=4 " in desc, desc
    torch.cuda.synchronize()
    ref = O.bmm_f64(O.to_f64(p.cpu()), O.to_f64(v.cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    assert torch.equal(out, cmpext3.bmm(p, v))


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_tall_narrow_b_through_the_operators(dtype):
    """A narrow B under few 128-row tiles runs on strips of A's rows (the tall kernel):
    attention's P V through bmm (B as [K, N], 64-row strips over a batch), a router-shaped
    Linear with a column bias (B as [N, K], 32-row strips) and a matmul with 16 columns
    written into a column slice of a wider C; against the oracle, deterministic."""
    g = torch.Generator().manual_seed(23)
    dt = DT[dtype]
    p = (torch.randn(8, 2048, 2048, generator=g) / np.sqrt(2048)).to(dt)
    v = torch.randn(8, 2048, 64, generator=g).to(dt)
    print(f"tall bmm {dtype} 8x2048x64x2048", flush=True)
    out = cmpext3.bmm(p.cuda(), v.cuda())
    name, desc = launched()
    assert name == "tall" and "tile=64x64" in desc, desc
    torch.cuda.synchronize()
    ref = O.bmm_f64(O.to_f64(p), O.to_f64(v))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    assert torch.equal(out, cmpext3.bmm(p.cuda(), v.cuda()))

    x = (torch.randn(3000, 1032, generator=g) / np.sqrt(1032)).to(dt)
    w = torch.randn(40, 1032, generator=g).to(dt)
    b = torch.randn(40, generator=g).to(dt)
    print(f"tall linear {dtype} 3000x40x1032", flush=True)
    out = cmpext3.linear(x.cuda(), w.cuda(), b.cuda())
    name, desc = launched()
    assert name == "tall" and "tile=32x64" in desc and "layout=NK" in desc, desc
    torch.cuda.synchronize()
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w), O.to_f64(b))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]

    a = (torch.randn(4096, 2048, generator=g) / np.sqrt(2048)).to(dt).cuda()
    bm = torch.randn(2048, 16, generator=g).to(dt).cuda()
    cw = torch.full((4096, 24), float("nan"), dtype=dt, device="cuda")
    print(f"tall C ABI {dtype} 4096x16x2048 into C[:, 3:19]", flush=True)
    st, name, desc = cabi_call(CODE[dtype], cabi.B_KN, a, 2048, 0, bm, 16, 0, cw[:, 3:19], 24, 0, None, 4096, 16, 2048)
    assert st == cabi.OK and name == "tall", desc
    torch.cuda.synchronize()
    got = cw.cpu()
    assert torch.isnan(got[:, :3].float()).all() and torch.isnan(got[:, 19:].float()).all()
    ref = O.matmul_f64(O.to_f64(a.cpu()), O.to_f64(bm.cpu()))
    assert O.rel_frobenius(O.to_f64(got[:, 3:19]), ref) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_weight_layout_batched_and_bias_c_abi(dtype):
    """[N, K] B through the C ABI: a batch of decode-shaped products (skinny_nk, one
    launch over grid.z) equal per entry to the single products, and a short-K product
    with many columns and a column bias (tile64x256), both against the oracle."""
    g = torch.Generator().manual_seed(11)
    Bn, M, N, K = 3, 16, 1000, 520
    a = (torch.randn(Bn, M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    w = (torch.randn(Bn, N, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    ag, wg = a.cuda(), w.cuda()
    c = torch.empty(Bn, M, N, dtype=DT[dtype], device="cuda")
    st, name, _ = cabi_call(CODE[dtype], cabi.B_NK, ag, K, M * K, wg, K, N * K, c, N, M * N, None, M, N, K, Bn)
    assert st == cabi.OK and name == "skinny_nk"
    for i in range(Bn):
        ci = torch.empty(M, N, dtype=DT[dtype], device="cuda")
        assert cabi.gemm_ex(CODE[dtype], cabi.B_NK, ag[i], K, 0, wg[i], K, 0, ci, N, 0, None, M, N, K) == cabi.OK
        torch.cuda.synchronize()
        assert torch.equal(ci, c[i])
        ref = O.linear_f64(O.to_f64(a[i]), O.to_f64(w[i]))
        assert O.rel_frobenius(O.to_f64(c[i].cpu()), ref) <= O.TOLERANCE[dtype]
    M, N, K = 48, 65536 + 40, 200
    x = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    w2 = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    bias = torch.randn(N, generator=g).to(DT[dtype])
    out = cmpext3.linear(x.cuda(), w2.cuda(), bias.cuda())
    assert launched()[0] == "tile64x256"
    torch.cuda.synchronize()
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w2), O.to_f64(bias))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_unaligned_operands_padded(dtype):
    """16-bit operands whose rows are not 16-byte aligned (odd K, odd N, offset views):
    the bindings pass a workspace, so A and/or B are copied zero-padded and a tiled
    kernel runs; the C ABI without a workspace runs the generic kernel.  Both against
    the oracle; C's odd row pitch is written element by element."""
    g = torch.Generator().manual_seed(21)
    for M, N, K in [(1023, 1025, 1027), (1024, 1031, 1024), (640, 1024, 1001)]:
        a = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
        b = (torch.randn(K, N, generator=g)).to(DT[dtype])
        out = MATMUL[dtype](a.cuda(), b.cuda())
        name, desc = launched()
        assert "padded=" in desc and name != "generic64x64", desc
        c = torch.empty(M, N, dtype=DT[dtype], device="cuda")
        st, name, _ = cabi_call(CODE[dtype], cabi.B_KN, a.cuda(), K, 0, b.cuda(), N, 0, c, N, 0, None, M, N, K)
        assert st == cabi.OK and name == "generic64x64"   # no workspace: element loads
        torch.cuda.synchronize()
        ref = O.matmul_f64(O.to_f64(a), O.to_f64(b))
        assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
        assert O.rel_frobenius(O.to_f64(c.cpu()), ref) <= O.TOLERANCE[dtype]
    # Linear with odd K and bias (W [N, K] padded), an offset view of A, a batch with odd K
    x = (torch.randn(512, 1001, generator=g) / 32).to(DT[dtype])
    w = (torch.randn(1999, 1001, generator=g) / 32).to(DT[dtype])
    bias = torch.randn(1999, generator=g).to(DT[dtype])
    out = cmpext3.linear(x.cuda(), w.cuda(), bias.cuda())
    name, desc = launched()
    assert name == "tile128x128" and "padded=AB" in desc, desc
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w), O.to_f64(bias))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    base = (torch.randn(1025, 1025, generator=g) / 32).to(DT[dtype])
    b2 = (torch.randn(1024, 768, generator=g) / 32).to(DT[dtype])
    view = base.cuda()[1:, 1:]  # rows start 2 bytes off 16-byte alignment: A is copied zero-padded
    out = MATMUL[dtype](view, b2.cuda())
    name, desc = launched()
    assert "padded=A" in desc and name != "generic64x64", desc
    ref = O.matmul_f64(O.to_f64(base[1:, 1:]), O.to_f64(b2))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    a3 = (torch.randn(3, 300, 257, generator=g) / 16).to(DT[dtype])
    b3 = (torch.randn(3, 257, 301, generator=g) / 16).to(DT[dtype])
    out = cmpext3.bmm(a3.cuda(), b3.cuda())
    assert "padded=AB" in launched()[1]
    torch.cuda.synchronize()
    for i in range(3):
        ref = O.matmul_f64(O.to_f64(a3[i]), O.to_f64(b3[i]))
        assert O.rel_frobenius(O.to_f64(out[i].cpu()), ref) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("M,N,K,kernel", [(4100, 3000, 2048, "f32tile96x64"), (3000, 2000, 1000, "f32tile64x64"),
                                          (2000, 2000, 1000, "f32tile128x128"), (2000, 2000, 260, "f32tile128x128"),
                                          (1000, 1000, 1028, "f32tile64x64k4"), (520, 516, 1028, "f32tile64x64k4")])
@pytest.mark.parametrize("layout", ["KN", "NK"])
def test_fp32_dma16(M, N, K, kernel, layout):
    """fp32 operands with 16-byte aligned rows and K, N multiples of 4 load through
    16-byte LDS-DMA: every tile, both B layouts, M/N tails, K % 16 != 0 and K splits
    (520 x 516 x 1028 on 64x64k4)."""
    g = torch.Generator().manual_seed(M + K)
    a = torch.rand(M, K, generator=g) * 2 - 1
    b = torch.rand(K, N, generator=g) * 2 - 1 if layout == "KN" else torch.rand(N, K, generator=g) * 2 - 1
    out = cmpext3.fp32_matmul(a.cuda(), b.cuda()) if layout == "KN" else cmpext3.linear(a.cuda(), b.cuda())
    name, desc = launched()
    assert "dma16" in desc and name == kernel, desc
    torch.cuda.synchronize()
    assert err_vs_oracle(out, a, b, "fp32", layout=layout) <= O.TOLERANCE["fp32"]
    if layout == "KN":  # a view whose rows start 4 bytes in takes the 4-byte path
        a2 = torch.zeros(M, K + 4)
        a2[:, 1:K + 1] = a
        av = a2.cuda()[:, 1:K + 1]
        out2 = cmpext3.fp32_matmul(av, b.cuda())
        torch.cuda.synchronize()
        assert err_vs_oracle(out2, a, b, "fp32") <= O.TOLERANCE["fp32"]


def test_fp32_unaligned_padded():
    """fp32 operands whose rows are not 16-byte aligned (odd K and N): with the bindings'
    workspace, large products on the 64x64 tile copy A and B zero-padded (K and N rounded
    up to 4) and run on the 16-byte DMA path; the C ABI without a workspace runs the
    4-byte path on its own tile, and the two agree bit for bit: the padded K columns add
    exact zeros in the positions the 4-byte path zero-fills, and every tile of
    gemm_f32_kernel sums an output's products in the same order (16-k stages, then the
    MFMA's fixed k order), so the tile does not matter (64x64k4, whose waves sum partial
    tiles, is not used by either here).  Linear (W as [N, K], padded) with bias, and a batch of
    odd-K products (kept on the 4-byte path: on the 128x128 and 96x64 tiles it loses less
    than the copies cost), against the oracle."""
    g = torch.Generator().manual_seed(41)
    for M, N, K in [(2049, 2999, 3001), (2500, 2501, 2502)]:
        a = torch.rand(M, K, generator=g) * 2 - 1
        b = torch.rand(K, N, generator=g) * 2 - 1
        out = cmpext3.fp32_matmul(a.cuda(), b.cuda())
        name, desc = launched()
        assert "padded=AB" in desc and "dma16" in desc, desc
        c = torch.empty(M, N, device="cuda")
        st, name, desc = cabi_call(cabi.F32, cabi.B_KN, a.cuda(), K, 0, b.cuda(), N, 0, c, N, 0, None, M, N, K)
        assert st == cabi.OK and "padded" not in desc, desc
        torch.cuda.synchronize()
        assert err_vs_oracle(out, a, b, "fp32") <= O.TOLERANCE["fp32"]
        assert torch.equal(out, c)
    x = torch.rand(2049, 3001, generator=g) * 2 - 1
    w = torch.rand(2999, 3001, generator=g) * 2 - 1
    bias = torch.rand(2999, generator=g)
    out = cmpext3.linear(x.cuda(), w.cuda(), bias.cuda())
    assert "padded=AB" in launched()[1]
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w), O.to_f64(bias))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE["fp32"]
    a3 = torch.rand(2, 1537, 2003, generator=g) * 2 - 1
    b3 = torch.rand(2, 2003, 2001, generator=g) * 2 - 1
    out = cmpext3.bmm(a3.cuda(), b3.cuda())
    torch.cuda.synchronize()
    for i in range(2):
        assert err_vs_oracle(out[i], a3[i], b3[i], "fp32") <= O.TOLERANCE["fp32"]


def test_fp32_m16_tile():
    """fp32 products with M <= 16 run on 16x64 tiles with K split over each workgroup's
    waves: ragged M, N and K (4-byte DMA), aligned (16-byte DMA), a K split across
    workgroups, Linear (W as [N, K]) with bias, and a batch, against the oracle."""
    g = torch.Generator().manual_seed(61)
    for M, N, K in [(13, 1001, 333), (7, 3000, 777), (16, 1000, 100), (16, 4096, 4096)]:
        a = torch.rand(M, K, generator=g) * 2 - 1
        b = torch.rand(K, N, generator=g) * 2 - 1
        out = cmpext3.fp32_matmul(a.cuda(), b.cuda())
        name, desc = launched()
        assert name == "f32tile16x64k4", desc
        if (M, N, K) == (16, 4096, 4096):
            assert "splits=" in desc, desc
        torch.cuda.synchronize()
        assert err_vs_oracle(out, a, b, "fp32") <= O.TOLERANCE["fp32"]
    for M, N, K in [(5, 1000, 1000), (16, 4096, 4096)]:
        x = torch.rand(M, K, generator=g) * 2 - 1
        w = torch.rand(N, K, generator=g) * 2 - 1
        bias = torch.rand(N, generator=g)
        out = cmpext3.linear(x.cuda(), w.cuda(), bias.cuda())
        assert launched()[0] == "f32tile16x64k4"
        ref = O.linear_f64(O.to_f64(x), O.to_f64(w), O.to_f64(bias))
        assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE["fp32"]
    a3 = torch.rand(4, 16, 1000, generator=g) * 2 - 1
    b3 = torch.rand(4, 1000, 512, generator=g) * 2 - 1
    out = cmpext3.bmm(a3.cuda(), b3.cuda())
    assert launched()[0] == "f32tile16x64k4"
    torch.cuda.synchronize()
    for i in range(4):
        assert err_vs_oracle(out[i], a3[i], b3[i], "fp32") <= O.TOLERANCE["fp32"]


def test_fp32_split_k():
    """fp32 products with few tiles and a long K split K over the fp32 tiles (fp32
    partials, summed with the bias by a second launch): matmul, ragged, Linear with bias
    and a batch, against the oracle at fp32's 1e-5."""
    g = torch.Generator().manual_seed(31)
    for M, N, K in [(16, 1024, 14336), (130, 1000, 4100)]:
        a = torch.rand(M, K, generator=g) * 2 - 1
        b = torch.rand(K, N, generator=g) * 2 - 1
        out = cmpext3.fp32_matmul(a.cuda(), b.cuda())
        assert "splits=" in launched()[1]
        torch.cuda.synchronize()
        assert err_vs_oracle(out, a, b, "fp32") <= O.TOLERANCE["fp32"]
    x = torch.rand(64, 8192, generator=g) * 2 - 1
    w = torch.rand(512, 8192, generator=g) * 2 - 1
    bias = torch.rand(512, generator=g)
    out = cmpext3.linear(x.cuda(), w.cuda(), bias.cuda())
    assert "splits=" in launched()[1]                 # linear passes its workspace: K splits
    ref = O.linear_f64(O.to_f64(x), O.to_f64(w), O.to_f64(bias))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE["fp32"]
    a3 = torch.rand(3, 64, 4096, generator=g) * 2 - 1
    b3 = torch.rand(3, 4096, 256, generator=g) * 2 - 1
    out = cmpext3.bmm(a3.cuda(), b3.cuda())
    assert "splits=" in launched()[1]
    torch.cuda.synchronize()
    for i in range(3):
        assert err_vs_oracle(out[i], a3[i], b3[i], "fp32") <= O.TOLERANCE["fp32"]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_views_and_layouts(dtype):
    g = torch.Generator().manual_seed(9)
    base = torch.randn(130, 97, generator=g).to(DT[dtype]).cuda()
    w = torch.randn(64, 96, generator=g).to(DT[dtype]).cuda()
    a = base[1:, 1:]                # offset view: misaligned rows and base pointer
    bt = w.t()                      # [96, 64] transposed view -> consumed as NK
    out = MATMUL[dtype](a, bt)
    ref = O.matmul_f64(O.to_f64(a.cpu()), O.to_f64(bt.cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    a2 = base[:, ::2][:, :48]       # non-unit inner stride -> copied
    b2 = torch.randn(48, 33, generator=g).to(DT[dtype]).cuda()
    out2 = MATMUL[dtype](a2, b2)
    ref2 = O.matmul_f64(O.to_f64(a2.cpu()), O.to_f64(b2.cpu()))
    assert O.rel_frobenius(O.to_f64(out2.cpu()), ref2) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("Bn,M,N,K", [(3, 64, 96, 40), (4, 512, 512, 512), (2, 16, 256, 128), (5, 7, 9, 11)])
def test_bmm(dtype, Bn, M, N, K):
    g = torch.Generator().manual_seed(Bn * M)
    a = (torch.randn(Bn, M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    b = (torch.randn(Bn, K, N, generator=g) / np.sqrt(K)).to(DT[dtype])
    out = cmpext3.bmm(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    _, desc_b = launched()
    ref = O.bmm_f64(O.to_f64(a), O.to_f64(b))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    for i in range(Bn):  # each batch entry equals the 2-D op on its slice, bit for bit, on the same plan
        single = MATMUL[dtype](a[i].cuda(), b[i].cuda())
        if launched()[1] == desc_b.replace(f"x{Bn} ", "x1 "):
            assert torch.equal(single, out[i])


# ------------------------------------------------------------ C ABI, streams
@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_c_abi_matches_binding(dtype):
    for M, N, K in [(300, 200, 72), (16, 512, 256), (33, 41, 17)]:
        a, b = O.make_inputs(dtype, M, N, K, "normal", 0.1, M)
        ag, bg = a.cuda(), b.cuda()
        c = torch.empty(M, N, dtype=DT[dtype], device="cuda")
        assert cabi.matmul(CODE[dtype], ag, bg, c, M, N, K) == cabi.OK
        c2 = torch.empty_like(c)
        st = cabi.gemm_ex(CODE[dtype], cabi.B_KN, ag, K, 0, bg, N, 0, c2, N, 0, None, M, N, K)
        assert st == cabi.OK
        torch.cuda.synchronize()
        assert torch.equal(c, c2)
        if cabi.workspace_size(CODE[dtype], cabi.B_KN, M, N, K) == 0:
            assert torch.equal(c, MATMUL[dtype](ag, bg))
        assert err_vs_oracle(c, a, b, dtype) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_c_abi_strided_views(dtype):
    """cmpext3_gemm_{f16,bf16,f32} on row-pitched views: A and B are column slices of
    wider matrices and C is written into a slice of a wider buffer, whose other
    columns must stay untouched; same bits as the binding on contiguous copies."""
    for M, N, K in [(300, 200, 72), (16, 512, 256), (33, 41, 17), (520, 1000, 264)]:
        a, b = O.make_inputs(dtype, M, N, K, "normal", 0.1, M + N)
        pad = 8 if K % 8 == 0 and N % 8 == 0 else 5  # odd pitches go to the generic kernel
        A = torch.zeros(M, K + pad, dtype=DT[dtype], device="cuda")
        B = torch.zeros(K, N + pad, dtype=DT[dtype], device="cuda")
        A[:, :K] = a.cuda()
        B[:, :N] = b.cuda()
        C = torch.full((M, N + 3 * pad), 7.0, dtype=DT[dtype], device="cuda")
        st = cabi.gemm_strided(CODE[dtype], A, K + pad, B, N + pad, C, N + 3 * pad, M, N, K)
        assert st == cabi.OK
        torch.cuda.synchronize()
        assert torch.all(C[:, N:] == 7.0)
        out = C[:, :N]
        assert err_vs_oracle(out, a, b, dtype) <= O.TOLERANCE[dtype]
        if pad == 8 and cabi.workspace_size(CODE[dtype], cabi.B_KN, M, N, K) == 0:
            assert torch.equal(out, MATMUL[dtype](a.cuda(), b.cuda()))


def test_runs_on_current_stream_and_is_deterministic():
    a, b = O.make_inputs("fp16", 1024, 1024, 1024, "normal", 1 / 32, 0)
    ag, bg = a.cuda(), b.cuda()
    ref = cmpext3.fp16_matmul(ag, bg)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        outs = [cmpext3.fp16_matmul(ag, bg) for _ in range(3)]
    s.synchronize()
    for o in outs:
        assert torch.equal(o, ref)


# --------------------------------------------------------- benchmark configs
def _full_config_check(name, via_cabi=False):
    c = O.CONFIGS[name]
    dtype, M, N, K = c["dtype"], c["M"], c["N"], c["K"]
    a, b = O.make_inputs(dtype, M, N, K, c["dist"], c.get("scale", 1.0), 0)
    ag, bg = a.cuda(), b.cuda()
    out = MATMUL[dtype](ag, bg)
    _, desc = launched()
    if via_cabi:
        # same kernel through the C ABI (with the workspace the binding uses): bit-identical
        c2 = torch.empty_like(out)
        ws_bytes = cabi.workspace_size(CODE[dtype], cabi.B_KN, M, N, K)
        ws = torch.empty(max(ws_bytes, 0), dtype=torch.uint8, device="cuda") if ws_bytes > 0 else None
        st, _, desc2 = cabi_call(CODE[dtype], cabi.B_KN, ag, K, 0, bg, N, 0, c2, N, 0, None, M, N, K, 1, ws)
        assert st == cabi.OK and desc2 == desc, (desc, desc2)
        torch.cuda.synchronize()
        assert torch.equal(out, c2)
        # the reference-shaped entry point (no workspace) within tolerance
        c3 = torch.empty_like(out)
        assert cabi.matmul(CODE[dtype], ag, bg, c3, M, N, K) == cabi.OK
        torch.cuda.synchronize()
        e3 = ((c3.double() - out.double()).norm() / out.double().norm()).item()
        assert e3 <= O.TOLERANCE[dtype], e3
    torch.cuda.synchronize()
    tol = O.TOLERANCE[dtype]
    out_c = out.cpu()
    af, bf = O.to_f64(a), O.to_f64(b)
    # (1) sampled rows (always the first and last) against the float64 oracle
    gen = torch.Generator().manual_seed(2)
    rows = sorted(set([0, M - 1] + torch.randint(0, M, (min(M, 64),), generator=gen).tolist()))
    e_rows = O.rel_frobenius(O.to_f64(out_c[rows]), O.matmul_f64(af[rows], bf))
    assert e_rows <= tol, e_rows
    # (2) every element against a PyTorch fp32 GEMM on the GPU
    ref = torch.matmul(ag.float(), bg.float())
    e_full = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
    assert e_full <= tol, e_full
    # (3) column and row sums against the exact (1^T A) B and A (B 1)
    of = O.to_f64(out_c)
    e_col = O.rel_frobenius(of.sum(axis=0), af.sum(axis=0) @ bf)
    e_row = O.rel_frobenius(of.sum(axis=1), af @ bf.sum(axis=1))
    assert e_col <= tol and e_row <= tol, (e_col, e_row)
    return e_rows, e_full


def test_cfg1_fp32_512_full_oracle():
    c = O.CONFIGS["cfg1_fp32_512"]
    a, b = O.make_inputs("fp32", 512, 512, 512, c["dist"], 1.0, 0)
    out = cmpext3.fp32_matmul(a.cuda(), b.cuda())
    assert err_vs_oracle(out, a, b, "fp32") <= O.TOLERANCE["fp32"]
    _full_config_check("cfg1_fp32_512")


def test_cfg2_fp16_4096():
    _full_config_check("cfg2_fp16_4096", via_cabi=True)


def test_cfg3_bf16_mlp():
    _full_config_check("cfg3_bf16_mlp")


def test_cfg4_fp16_skinny():
    _full_config_check("cfg4_fp16_skinny", via_cabi=True)
    c = O.CONFIGS["cfg4_fp16_skinny"]
    a, b = O.make_inputs("fp16", 16, 8192, 8192, c["dist"], c["scale"], 0)
    out = cmpext3.fp16_matmul(a.cuda(), b.cuda())
    assert err_vs_oracle(out, a, b, "fp16") <= O.TOLERANCE["fp16"]   # full float64 oracle


def test_cfg5_fp32_ragged():
    _full_config_check("cfg5_fp32_ragged", via_cabi=True)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_linear_misaligned_bias_stays_tiled(dtype):
    """A bias view that is only 2-byte aligned (bias[1:]) is read element by element
    in the epilogue; the product stays on the tiled kernel and gives the same bits as
    an aligned copy of the same bias.  Against the float64 oracle on sampled rows."""
    M = N = K = 4096
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(M, K, generator=g) / 8).to(DT[dtype]).cuda()
    w = (torch.randn(N, K, generator=g) / 8).to(DT[dtype]).cuda()
    bias_full = torch.randn(N + 1, generator=g).to(DT[dtype]).cuda()
    bias_view = bias_full[1:]
    assert bias_view.data_ptr() % 8 == 2
    out = cmpext3.linear(x, w, bias_view)
    name, desc = launched()
    assert name == "tile256x256", desc
    out_aligned = cmpext3.linear(x, w, bias_view.clone())
    torch.cuda.synchronize()
    assert torch.equal(out, out_aligned)
    rows = [0, 1, 1000, 4095]
    ref = O.linear_f64(O.to_f64(x[rows].cpu()), O.to_f64(w.cpu()), O.to_f64(bias_view.cpu()))
    assert O.rel_frobenius(O.to_f64(out[rows].cpu()), ref) <= O.TOLERANCE[dtype]
    # the ragged tail (N % 4 != 0) with a misaligned bias, 128x128 tiles
    x2, w2 = x[:1000, :1000].contiguous(), w[:1002, :1000].contiguous()
    b2 = bias_full[1:1003]
    out2 = cmpext3.linear(x2, w2, b2)
    torch.cuda.synchronize()
    assert launched()[0] != "generic64x64"
    ref2 = O.linear_f64(O.to_f64(x2.cpu()), O.to_f64(w2.cpu()), O.to_f64(b2.cpu()))
    assert O.rel_frobenius(O.to_f64(out2.cpu()), ref2) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_tiled_split_k_batched(dtype):
    """16-bit tiled products that split K inside a batch (grid.z = batch * splits):
    bmm of 3 x 256x2048x8192 (5 ways, the last K range shorter), every batch entry
    against the float64 oracle, and equal bit for bit to the same entry computed alone
    (same tile and split)."""
    Bn, M, N, K = 3, 256, 2048, 8192
    g = torch.Generator().manual_seed(88)
    a = (torch.randn(Bn, M, K, generator=g) / 64).to(DT[dtype])
    b = (torch.randn(Bn, K, N, generator=g) / 64).to(DT[dtype])
    out = cmpext3.bmm(a.cuda(), b.cuda())
    name, desc = launched()
    assert name.startswith("tile") and "splits=" in desc and "splits=1 " not in desc, desc
    torch.cuda.synchronize()
    for i in range(Bn):
        ref = O.matmul_f64(O.to_f64(a[i]), O.to_f64(b[i]))
        assert O.rel_frobenius(O.to_f64(out[i].cpu()), ref) <= O.TOLERANCE[dtype], i
    single = cmpext3.bmm(a[1:2].cuda(), b[1:2].cuda())
    _, desc1 = launched()
    if desc1.split()[0] == desc.split()[0] and desc1.split("splits=")[1].split()[0] == desc.split("splits=")[1].split()[0]:
        assert torch.equal(single[0], out[1])


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K,batch,bias", [
    (64, 8200, 128, 64, False),   # 65 column tiles per entry, the last one 8 columns wide
    (40, 16384, 72, 32, True),    # ragged M and K, bias per row (4096 tiles: 16 per CU)
    (1, 524288, 8, 1, False),     # one row, K = 8, one product of 4096 tiles
    (128, 16384, 128, 32, True),  # 128-row tiles
    (96, 8200, 64, 64, False),    # 128-row tiles, M and N ragged
    (64, 16384, 256, 32, True),   # K = 256: two chunks of 128 k per tile
    (48, 8200, 200, 64, False),   # second chunk ragged (72 k), M and N ragged
    (8, 131072, 136, 4, True),    # second chunk of 8 k
    (128, 16384, 256, 32, True),  # 128 rows in two groups of 4 waves, K = 256
    (96, 8200, 200, 64, False),   # ... M, N and the second chunk ragged
    (72, 131072, 136, 4, True),   # ... second chunk of 8 k
    (256, 16384, 64, 32, True),   # two row blocks of 128
    (200, 8200, 136, 64, False),  # ... the second of 72 rows, N and K ragged
    (512, 16384, 256, 32, True),  # four row blocks, K = 256
    (1000, 16384, 128, 16, True),  # eight row blocks, the last of 104 rows
])
def test_stream_kernel(dtype, M, N, K, batch, bias):
    """Short-K products over many columns with one A for the whole batch (the 1x1
    convolution shape) through the C ABI: the streaming kernel, against the float64
    oracle on sampled batch entries and an fp32 GPU product on all, deterministic."""
    g = torch.Generator().manual_seed(M + K + batch)
    a = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    b = torch.randn(batch, K, N, generator=g).to(DT[dtype])
    bvec = torch.randn(M, generator=g).to(DT[dtype]) if bias else None
    ag, bg = a.cuda(), b.cuda()
    bvg = bvec.cuda() if bias else None
    c = torch.full((batch, M, N), float("nan"), dtype=DT[dtype], device="cuda")
    print(f"stream {dtype} M={M} N={N} K={K} batch={batch} bias={bias}", flush=True)
    st, call = cabi.prepare(CODE[dtype], cabi.B_KN, ag, K, 0, bg, N, K * N, c, N, M * N, bvg, M, N, K, batch,
                            cabi.BIAS_PER_ROW if bias else 0, 0)
    assert st == cabi.OK
    _, desc = cabi.describe(call)
    SEEN_KERNELS.add(kernel_of(desc))
    assert kernel_of(desc) == ("stream64x128" if M <= 64 else "stream128x128"), desc
    assert cabi.run(call) == cabi.OK
    torch.cuda.synchronize()
    assert not torch.isnan(c).any()
    ref = torch.matmul(ag.float(), bg.float())
    if bias:
        ref = ref + bvg.float()[:, None]
    e2 = ((c.double() - ref.double()).norm() / ref.double().norm()).item()
    assert e2 <= O.TOLERANCE[dtype]
    for i in sorted({0, batch // 2, batch - 1}):
        r = O.matmul_f64(O.to_f64(a), O.to_f64(b[i]))
        if bias:
            r = r + O.to_f64(bvec)[:, None]
        assert O.rel_frobenius(O.to_f64(c[i].cpu()), r) <= O.TOLERANCE[dtype], i
    c2 = torch.empty_like(c)
    st, call2 = cabi.prepare(CODE[dtype], cabi.B_KN, ag, K, 0, bg, N, K * N, c2, N, M * N, bvg, M, N, K, batch,
                             cabi.BIAS_PER_ROW if bias else 0, 0)
    assert st == cabi.OK
    # repeated back-to-back launches (the ring's waits rely on the order in which a wave's
    # loads and stores complete): every one bit-identical to the first
    for _ in range(20):
        c2.fill_(float("nan"))
        assert cabi.run(call2) == cabi.OK
        torch.cuda.synchronize()
        assert torch.equal(c, c2)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("M,N,K,batch,bias", [
    (64, 16384, 128, 32, True),    # NHWC images of 128 x 128 pixels, 128 -> 64 channels
    (40, 8200, 72, 64, False),     # ragged M, N (last tile 8 pixels) and K
    (1, 524288, 8, 1, False),      # one row; 16-byte rows of B
    (128, 16384, 256, 32, True),   # 128-row tiles, two K chunks
    (300, 8200, 136, 32, False),   # three row blocks, the second chunk of 8 k
])
def test_stream_kernel_b_nk(dtype, M, N, K, batch, bias):
    """The streaming kernel with B given as [N, K] (a 1x1 convolution over NHWC images:
    pixels x input channels) through the C ABI, against the float64 oracle on sampled
    batch entries and an fp32 GPU product on all, deterministic."""
    g = torch.Generator().manual_seed(M + K + batch + 1)
    a = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    b = torch.randn(batch, N, K, generator=g).to(DT[dtype])
    bvec = torch.randn(M, generator=g).to(DT[dtype]) if bias else None
    ag, bg = a.cuda(), b.cuda()
    bvg = bvec.cuda() if bias else None
    c = torch.full((batch, M, N), float("nan"), dtype=DT[dtype], device="cuda")
    print(f"stream NK {dtype} M={M} N={N} K={K} batch={batch} bias={bias}", flush=True)
    st, call = cabi.prepare(CODE[dtype], cabi.B_NK, ag, K, 0, bg, K, N * K, c, N, M * N, bvg, M, N, K, batch,
                            cabi.BIAS_PER_ROW if bias else 0, 0)
    assert st == cabi.OK
    _, desc = cabi.describe(call)
    SEEN_KERNELS.add(kernel_of(desc))
    assert kernel_of(desc) == ("stream64x128" if M <= 64 else "stream128x128") and "layout=NK" in desc, desc
    assert cabi.run(call) == cabi.OK
    torch.cuda.synchronize()
    assert not torch.isnan(c).any()
    ref = torch.matmul(ag.float(), bg.float().transpose(1, 2))
    if bias:
        ref = ref + bvg.float()[:, None]
    e2 = ((c.double() - ref.double()).norm() / ref.double().norm()).item()
    assert e2 <= O.TOLERANCE[dtype]
    for i in sorted({0, batch // 2, batch - 1}):
        r = O.matmul_f64(O.to_f64(a), O.to_f64(b[i]).T)
        if bias:
            r = r + O.to_f64(bvec)[:, None]
        assert O.rel_frobenius(O.to_f64(c[i].cpu()), r) <= O.TOLERANCE[dtype], i
    c2 = torch.full_like(c, float("nan"))
    assert cabi.run(call) == cabi.OK
    torch.cuda.synchronize()
    c2.copy_(c)
    assert cabi.run(call) == cabi.OK
    torch.cuda.synchronize()
    assert torch.equal(c, c2)


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_views_read_in_place(dtype):
    """bmm and linear read row-pitched views, batch slices and transposed operands in
    place (the plan shows the layout and pitch they ran with) and match the oracle."""
    g = torch.Generator().manual_seed(21)
    dt = DT[dtype]
    # bmm(q, k^T): the keys as a transposed view -> B given as [N, K]
    q = (torch.randn(4, 96, 64, generator=g) / 8).to(dt).cuda()
    k = torch.randn(4, 200, 64, generator=g).to(dt).cuda()
    out = cmpext3.bmm(q, k.transpose(1, 2))
    plan = cmpext3.last_plan()
    assert "layout=NK" in plan, plan
    ref = O.bmm_f64(O.to_f64(q.cpu()), O.to_f64(k.cpu()).transpose(0, 2, 1))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    # bmm on column slices of wider tensors (row pitch above the width) and a batch slice
    big_a = (torch.randn(5, 96, 80, generator=g) / 8).to(dt).cuda()
    big_b = torch.randn(5, 64, 136, generator=g).to(dt).cuda()
    a, b = big_a[1:, :, 8:72], big_b[1:, :, :128]
    out = cmpext3.bmm(a, b)
    assert "layout=KN" in cmpext3.last_plan()
    ref = O.bmm_f64(O.to_f64(a.cpu()), O.to_f64(b.cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    # linear: the weight as a transposed view of a [K, N] tensor -> B given as [K, N]; a
    # row-pitched 2-D input
    w_kn = (torch.randn(64, 120, generator=g) / 8).to(dt).cuda()
    x = torch.randn(50, 72, generator=g).to(dt).cuda()[:, :64]
    bias = torch.randn(120, generator=g).to(dt).cuda()
    out = cmpext3.linear(x, w_kn.t(), bias)
    assert "layout=KN" in cmpext3.last_plan()
    ref = O.linear_f64(O.to_f64(x.cpu()), O.to_f64(w_kn.t().cpu()), O.to_f64(bias.cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]
    # linear with a row slice of a larger weight ([N, K] rows, B given as [N, K], offset base)
    w_big = (torch.randn(130, 64, generator=g) / 8).to(dt).cuda()
    out = cmpext3.linear(x, w_big[3:123])
    assert "layout=NK" in cmpext3.last_plan()
    ref = O.linear_f64(O.to_f64(x.cpu()), O.to_f64(w_big[3:123].cpu()))
    assert O.rel_frobenius(O.to_f64(out.cpu()), ref) <= O.TOLERANCE[dtype]


def test_every_kernel_family_was_exercised():
    missing = set(KERNEL_NAMES) - SEEN_KERNELS
    assert not missing, f"kernels never selected by these tests: {missing}"
