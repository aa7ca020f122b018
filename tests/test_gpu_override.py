"""Plans forced with the CMPEXT3_GEMM_CONFIG tuning override, against the float64 oracle.

The override reaches kernel configurations the selector does not choose by itself,
which this file checks for parity: the streaming kernel with only one to a few
128-column tiles per workgroup (its ring filling and draining within a tile or two,
chunks past the end loaded through empty descriptors), over one or several row
blocks, with one or two K chunks; the 256x256 tile with a K split and a batch; the
generic kernel on aligned operands; an fp32 tile with a K split; the tall kernel (strips
of A's rows, B of at most 128 columns as [K, N] or [N, K]) with both strip heights.
"""
import pytest
import torch

from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
CODE = {"fp16": cabi.F16, "bf16": cabi.BF16, "fp32": cabi.F32}


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _run(dtype, M, N, K, batch, shared_a, bias, workspace, seed, nk=False, ldc=None):
    """C[b] = A[b] B[b] (+ bias per row if bias == "row", per column if "col") through a
    prepared call, B given as [K, N] (or [N, K] if nk), C rows `ldc` apart (default N);
    returns (kernel description, max relative error over the batch)."""
    g = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    ldc = ldc or N
    a = (torch.randn(1 if shared_a else batch, M, K, generator=g) / max(K, 1) ** 0.5).to(dt)
    b = torch.randn(batch, K, N, generator=g).to(dt)
    bv = torch.randn(M if bias == "row" else N, generator=g).to(dt) if bias else None
    cfull = torch.full((batch, M, ldc), float("nan"), dtype=dt, device="cuda")
    c = cfull[:, :, :N]
    ag = a.cuda()
    bg = b.transpose(1, 2).contiguous().cuda() if nk else b.cuda()
    bvg = None if bv is None else bv.cuda()  # held until the call has run (prepare keeps the pointer)
    st, call = cabi.prepare(CODE[dtype], cabi.B_NK if nk else cabi.B_KN, ag, K, 0 if shared_a else M * K,
                            bg, K if nk else N, K * N, c, ldc, M * ldc,
                            bvg, M, N, K, batch,
                            cabi.BIAS_PER_ROW if bias == "row" else 0, (1 << 40) if workspace else 0)
    assert st == cabi.OK
    _, desc = cabi.describe(call)
    print(f"{dtype} M={M} N={N} K={K} batch={batch} bias={bias}: {desc}", flush=True)
    ws_bytes = cabi.call_workspace_size(call)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") if ws_bytes > 0 else None
    assert cabi.run(call, ws) == cabi.OK
    torch.cuda.synchronize()
    out = c.cpu()
    err = 0.0
    if ldc > N:  # the columns past N are untouched
        assert torch.isnan(cfull[:, :, N:].float()).all()
    for i in range(batch):
        r = O.matmul_f64(O.to_f64(a[0 if shared_a else i]), O.to_f64(b[i]))
        if bias == "row":
            r = r + O.to_f64(bv)[:, None]
        elif bias == "col":
            r = r + O.to_f64(bv)[None, :]
        err = max(err, O.rel_frobenius(O.to_f64(out[i]), r))
    return desc, err


@pytest.mark.parametrize("dtype,M,N,K,batch,bias", [
    ("fp16", 64, 128, 128, 1, "row"),    # one tile: one workgroup, one tile
    ("bf16", 1, 8, 8, 1, None),          # one row, one 8-column tile
    ("fp16", 40, 296, 72, 3, "row"),     # 3 tiles per entry, the last ragged; 9 tiles, 8 workgroups
    ("fp16", 64, 1000, 200, 2, None),    # two K chunks, 16 tiles
    ("bf16", 128, 640, 128, 1, "row"),   # 128-row tiles, 5 tiles
    ("fp16", 96, 136, 256, 2, None),     # 128-row tiles, two chunks, 2 tiles per entry
    ("fp16", 300, 1024, 64, 1, "row"),   # three row blocks over 8 tiles
    ("bf16", 1000, 256, 136, 2, None),   # eight row blocks, two chunks, 4 tiles
])
def test_forced_stream_kernel_few_tiles(monkeypatch, dtype, M, N, K, batch, bias):
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=stream64x128")
    desc, err = _run(dtype, M, N, K, batch, True, bias, False, M + N + K)
    assert desc.startswith("kernel=stream64x128" if M <= 64 else "kernel=stream128x128"), desc
    assert err <= O.TOLERANCE[dtype], err


def test_forced_tile_split_batched(monkeypatch):
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tile256x256,splits=3")
    desc, err = _run("fp16", 512, 384, 1600, 2, False, "col", True, 7)
    assert desc.startswith("kernel=tile256x256") and "splits=3" in desc, desc
    assert err <= O.TOLERANCE["fp16"], err


def test_forced_generic_on_aligned_operands(monkeypatch):
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=generic64x64")
    desc, err = _run("bf16", 200, 264, 512, 2, False, "row", True, 8)
    assert desc.startswith("kernel=generic64x64"), desc
    assert err <= O.TOLERANCE["bf16"], err


def test_forced_fp32_tile_split(monkeypatch):
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=f32tile128x128,splits=4")
    desc, err = _run("fp32", 300, 260, 2100, 1, False, "col", True, 9)
    assert desc.startswith("kernel=f32tile128x128") and "splits=4" in desc, desc
    assert err <= O.TOLERANCE["fp32"], err


@pytest.mark.parametrize("dtype,M,N,K,batch,bias,nk,strip,ldc", [
    ("fp16", 2048, 64, 2048, 2, None, False, 64, None),    # B as [K, N], 64 columns, whole stages
    ("bf16", 1000, 64, 200, 3, "col", False, 32, None),    # ragged strips and last stage
    ("fp16", 300, 8, 136, 1, "row", False, 64, 24),        # one column block, C rows 24 apart
    ("fp16", 777, 72, 264, 2, "col", False, 64, None),     # 72 columns: the 128-column form
    ("bf16", 513, 128, 1032, 1, "row", False, 32, 136),    # 128 columns, 32-row strips
    ("fp16", 2048, 64, 2048, 2, "col", True, 64, None),    # B as [N, K] (a router's weight)
    ("bf16", 1000, 40, 72, 2, None, True, 32, None),       # [N, K], 40 rows, short K
    ("fp16", 700, 8, 520, 2, "col", True, 64, None),       # [N, K], 8 rows: one 16-row block
    ("bf16", 1500, 24, 1032, 1, "row", True, 32, 40),      # [N, K], 24 rows: two 16-row blocks
    ("fp16", 129, 128, 520, 3, "row", True, 64, 130),      # [N, K], 128 rows, odd C pitch
])
def test_forced_tall(monkeypatch, dtype, M, N, K, batch, bias, nk, strip, ldc):
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", f"kernel=tall,strip={strip}")
    desc, err = _run(dtype, M, N, K, batch, False, bias, False, M + N + K, nk=nk, ldc=ldc)
    assert desc.startswith("kernel=tall") and f"tile={strip}x" in desc, desc
    assert err <= O.TOLERANCE[dtype], err


def test_forced_skinny_nk_split(monkeypatch):
    """skinny_nk with a forced 3-way split of a ragged K (ranges of 1536, 1536, 1032) and a
    bias per row (added by the reduction), over a batch."""
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=skinny_nk,splits=3")
    desc, err = _run("bf16", 40, 296, 4104, 2, False, "row", True, 12, nk=True)
    assert desc.startswith("kernel=skinny_nk") and "splits=3 ksplit=1536" in desc, desc
    assert err <= O.TOLERANCE["bf16"], err


def test_forced_tall_split(monkeypatch):
    """The tall kernel with a forced 3-way split of a ragged K (B as [K, N], 64-row strips,
    a bias per row added by the reduction) over a batch."""
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tall,strip=64,splits=3")
    desc, err = _run("fp16", 700, 40, 2056, 2, False, "row", True, 13)
    assert desc.startswith("kernel=tall") and "splits=3 ksplit=768" in desc, desc
    assert err <= O.TOLERANCE["fp16"], err
