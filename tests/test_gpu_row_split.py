"""16-bit products whose last round of tiles would run mostly empty run as two
launches over their rows (rows that whole rounds of 256-row tiles cover, then the
rest): through the C ABI, with B as [K,N] and as [N,K], batches, a bias per column
or per row and with or without a workspace, every row of C meets the float64 oracle
(sampled rows, all rows next to the split) and an fp32 GPU product (all rows), and
nothing is written between C's rows."""
import numpy as np
import pytest
import torch

from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
CODE = {"fp16": cabi.F16, "bf16": cabi.BF16}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


# dtype, layout, M, N, K, batch, bias ("col", "row" or None), workspace
CASES = [
    ("bf16", "KN", 4100, 4096, 4096, 1, None, True),     # + 4 rows: skinny_wide (split K)
    ("bf16", "KN", 4100, 4096, 4096, 1, None, False),    # no workspace: narrow skinny rows
    ("fp16", "NK", 4100, 4096, 4096, 1, "col", True),    # Linear: + 4 rows of skinny_nk
    ("bf16", "NK", 5000, 4096, 4096, 1, "col", True),    # + 904 rows of 128x128 tiles
    ("fp16", "KN", 2060, 4096, 1024, 2, None, True),     # batched
    ("fp16", "KN", 4100, 1024, 2048, 4, "row", True),    # bias per row, batched
]


def _random_split_cases(n, seed=11):
    """Seeded random shapes (multiples of 8 in N and K) whose plan splits the rows."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dtype = ["fp16", "bf16"][rng.integers(2)]
        layout = ["KN", "NK"][rng.integers(2)]
        batch = int(rng.choice([1, 1, 2]))
        M, N, K = int(rng.integers(257, 7000)), int(rng.integers(1, 769)) * 8, int(rng.integers(1, 385)) * 8
        if M * N * K * batch > 1.2e11:
            continue
        bias = [None, "col", "row"][rng.integers(3)]
        ws = bool(rng.integers(2))
        _, d = cabi.plan(CODE[dtype], cabi.B_KN if layout == "KN" else cabi.B_NK, M, N, K, ldc=N + 8,
                         has_bias=bias is not None, batch=batch, workspace_bytes=(1 << 62) if ws else 0)
        if " rows=" in d:
            out.append((dtype, layout, M, N, K, batch, bias, ws))
    return out


CASES += _random_split_cases(8)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(x) for x in c))
def test_row_split(case):
    dtype, layout, M, N, K, batch, bias_mode, with_ws = case
    lay = cabi.B_KN if layout == "KN" else cabi.B_NK
    g = torch.Generator().manual_seed(M + N + K + batch)
    a = (torch.randn(batch, M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    bshape = (K, N) if layout == "KN" else (N, K)
    b = (torch.randn(batch, *bshape, generator=g)).to(DT[dtype])
    nbias = {"col": N, "row": M, None: 0}[bias_mode]
    bias = torch.randn(nbias, generator=g).to(DT[dtype]) if bias_mode else None
    ldc = N + 8
    sentinel = 3.0
    cg = torch.full((batch, M, ldc), sentinel, dtype=DT[dtype], device="cuda")
    ag, bg = a.cuda(), b.cuda()
    biasg = bias.cuda() if bias is not None else None
    flags = 1 if bias_mode == "row" else 0
    st, call = cabi.prepare(CODE[dtype], lay, ag, K, M * K, bg, bshape[1], bshape[0] * bshape[1], cg, ldc, M * ldc,
                            biasg, M, N, K, batch, flags, (1 << 62) if with_ws else 0)
    assert st == cabi.OK, cabi.status_string(st)
    _, desc = cabi.describe(call)
    assert " rows=" in desc, desc  # two launches over the rows
    m_main = int(desc.split(" rows=")[1].split()[0])
    assert 0 < m_main < M and m_main % 256 == 0, desc
    ws_bytes = cabi.call_workspace_size(call)
    assert with_ws or ws_bytes == 0, desc
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda") if ws_bytes > 0 else None
    assert cabi.run(call, ws) == cabi.OK
    torch.cuda.synchronize()
    out = cg.cpu()
    assert (out[:, :, N:] == sentinel).all(), "a store landed between C's rows"
    out = out[:, :, :N]
    # every row against an fp32 product on the GPU
    bt = bg.float() if layout == "KN" else bg.float().transpose(1, 2).contiguous()
    ref32 = torch.bmm(ag.float(), bt)
    if bias_mode == "col":
        ref32 += biasg.float()[None, None, :]
    elif bias_mode == "row":
        ref32 += biasg.float()[None, :, None]
    for i in range(batch):
        assert O.rel_frobenius(O.to_f64(out[i]), O.to_f64(ref32[i].cpu())) <= O.TOLERANCE[dtype], (i, desc)
    # sampled rows, and every row from 8 before the split to the end, against the float64 oracle
    gen = torch.Generator().manual_seed(7)
    rows = sorted(set(torch.randint(0, m_main, (24,), generator=gen).tolist()) | set(range(m_main - 8, M)))
    for i in {0, batch - 1}:
        bf = O.to_f64(b[i]) if layout == "KN" else O.to_f64(b[i]).T
        ref = O.matmul_f64(O.to_f64(a[i][rows]), bf)
        if bias_mode == "col":
            ref = ref + O.to_f64(bias)[None, :]
        elif bias_mode == "row":
            ref = ref + O.to_f64(bias)[rows][:, None]
        assert O.rel_frobenius(O.to_f64(out[i][rows]), ref) <= O.TOLERANCE[dtype], (i, desc)


def test_row_split_under_graph_capture():
    # the two launches captured in a graph (the skinny tail then sums its split-K partials in
    # a second launch instead of in-kernel): every replay equals the eager result bit for bit
    import cmpext3

    g = torch.Generator().manual_seed(41)
    a = (torch.randn(4100, 4096, generator=g) / 64).to(torch.bfloat16).cuda()
    b = torch.randn(4096, 4096, generator=g).to(torch.bfloat16).cuda()
    eager = cmpext3.bf16_matmul(a, b)
    desc = cmpext3.last_plan()
    assert " rows=4096 | rows 4096..4099: kernel=skinny_wide" in desc, desc
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        cmpext3.bf16_matmul(a, b)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = cmpext3.bf16_matmul(a, b)
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(cmpext3.bf16_matmul(a, b), eager)
