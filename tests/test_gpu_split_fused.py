"""Split-K skinny products whose partial sums are added up inside the splitting
kernel: the last workgroup of each column strip to finish sums the strip's
partials (counters of the calling stream, zero between kernels).  Under graph
capture, and on streams beyond the counters' slots, the sum runs in a second
launch instead; both forms do the same arithmetic, so their results must be
bit-identical.  Each case also meets the float64 oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

import cmpext3
from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


def operands(dtype, M, N, K, batch, seed):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(batch, M, K, generator=g) / np.sqrt(K)).to(DT[dtype])
    b = (torch.randn(batch, K, N, generator=g) / np.sqrt(K)).to(DT[dtype])
    return a.cuda(), b.cuda()


# dtype, M, N, K, batch: strips of 128 columns (one partly filled at N % 128 != 0),
# 1..4 blocks of 16 rows, batches of several entries
CASES = [
    ("fp16", 16, 8192, 8192, 1),
    ("bf16", 1, 4096, 8192, 1),
    ("fp16", 40, 2056, 6144, 1),
    ("bf16", 64, 1024, 16384, 2),
    ("fp16", 8, 3000, 8192, 3),
    ("fp16", 32, 8000, 8192, 1),
    ("bf16", 16, 4096, 4352, 2),
    ("bf16", 3, 8192, 8192, 1),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(x) for x in c))
def test_in_kernel_sum_matches_second_launch(case):
    dtype, M, N, K, batch = case
    a, b = operands(dtype, M, N, K, batch, seed=M + N + K)
    mm = cmpext3.fp16_matmul if dtype == "fp16" else cmpext3.bf16_matmul
    f = (lambda: cmpext3.bmm(a, b)) if batch > 1 else (lambda: mm(a[0], b[0]))
    eager = f()
    desc = cmpext3.last_plan()
    assert desc.startswith("kernel=skinny_wide") and "splits=1 " not in desc, desc
    torch.cuda.synchronize()
    # captured: the counters are not used, the reduction is a second launch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        f()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f()
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), desc
        assert torch.equal(f(), eager)
    for i in range(batch):
        ref = O.matmul_f64(O.to_f64(a[i].cpu()), O.to_f64(b[i].cpu()))
        got = O.to_f64((eager[i] if batch > 1 else eager).cpu())
        assert O.rel_frobenius(got, ref) <= O.TOLERANCE[dtype]


def test_counters_reset_between_shapes():
    # products with different strip counts and splits, interleaved on one stream: each
    # must leave its counters at zero for the next
    shapes = [(16, 8192, 8192), (16, 1024, 8192), (32, 4096, 4096), (4, 8192, 16384)]
    ins = [operands("fp16", M, N, K, 1, seed=i) for i, (M, N, K) in enumerate(shapes)]
    refs = [cmpext3.fp16_matmul(a[0], b[0]) for a, b in ins]
    torch.cuda.synchronize()
    bad = torch.zeros((), dtype=torch.int64, device="cuda")
    for _ in range(100):
        for (a, b), r in zip(ins, refs):
            bad += (cmpext3.fp16_matmul(a[0], b[0]) != r).sum()
    assert bad.item() == 0
    for (a, b), r in zip(ins, refs):
        ref = O.matmul_f64(O.to_f64(a[0].cpu()), O.to_f64(b[0].cpu()))
        assert O.rel_frobenius(O.to_f64(r.cpu()), ref) <= O.TOLERANCE["fp16"]


def test_more_streams_than_counter_slots():
    # 72 streams of the runtime's own (more than the 64 counter slots of a GPU): the
    # streams past the slots reduce in a second launch; every stream's result is exact
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    a, b = operands("fp16", 16, 2048, 8192, 1, seed=7)
    ref = cmpext3.fp16_matmul(a[0], b[0])
    torch.cuda.synchronize()
    M, N, K = 16, 2048, 8192
    need = cabi.lib().cmpext3_gemm_workspace_size(cabi.F16, cabi.B_KN, M, N, K, 1)
    assert need > 0
    streams, outs, wss = [], [], []
    try:
        for _ in range(72):
            h = ctypes.c_void_p()
            assert hip.hipStreamCreate(ctypes.byref(h)) == 0
            streams.append(h)
        for h in streams:
            c = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
            ws = torch.empty(need, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            st = cabi.lib().cmpext3_gemm_ex(cabi.F16, cabi.B_KN, a[0].data_ptr(), K, 0, b[0].data_ptr(), N, 0,
                                            c.data_ptr(), N, 0, None, M, N, K, 1, ws.data_ptr(), need, h.value)
            assert st == cabi.OK, cabi.status_string(st)
            outs.append(c)
            wss.append(ws)
        for h in streams:
            assert hip.hipStreamSynchronize(h) == 0
        for c in outs:
            assert torch.equal(c, ref)
    finally:
        for h in streams:
            hip.hipStreamSynchronize(h)
            hip.hipStreamDestroy(h)


def test_per_thread_default_stream_from_two_threads():
    # hipStreamPerThread is one handle for a different stream on every host thread, so it
    # gets no counters (second launch); two threads calling on it at once are both exact
    import threading

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    M, N, K = 16, 4096, 8192
    a, b = operands("fp16", M, N, K, 1, seed=11)
    ref = cmpext3.fp16_matmul(a[0], b[0])
    need = cabi.lib().cmpext3_gemm_workspace_size(cabi.F16, cabi.B_KN, M, N, K, 1)
    outs = [torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda") for _ in range(2)]
    wss = [torch.empty(need, dtype=torch.uint8, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    status = [None, None]

    def work(i):
        torch.cuda.set_device(0)
        st = 0
        for _ in range(20):
            st = st or cabi.lib().cmpext3_gemm_ex(cabi.F16, cabi.B_KN, a[0].data_ptr(), K, 0, b[0].data_ptr(), N, 0,
                                                  outs[i].data_ptr(), N, 0, None, M, N, K, 1, wss[i].data_ptr(),
                                                  need, 2)  # hipStreamPerThread
        status[i] = st or hip.hipStreamSynchronize(2)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert status == [0, 0]
    for c in outs:
        assert torch.equal(c, ref)
