"""The GEMM path under HIP graph capture (torch.cuda.CUDAGraph).

The library launches only kernels on the caller's stream (no memsets, copies,
synchronizations or allocations of its own; the bindings take their output and
workspace from PyTorch's caching allocator, which under capture is the graph's
private pool), so every path can be captured: tiled products, split-K skinny
products (second launch summing the partials), padded fp32 copies, the fp32
tiles with K split over their waves, bmm and the 1x1 convolution.  The test
replays the captured graph several times, with eager calls of the same
operators and synchronizations in between, and checks every replay bit for
bit against the eager results (all kernels are deterministic).
"""
import pytest
import torch

import cmpext3

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


def _inputs():
    g = torch.Generator(device="cuda").manual_seed(5)

    def rn(*shape, dtype=torch.float16, scale=1.0):
        return (torch.randn(*shape, generator=g, device="cuda") * scale).to(dtype)

    return {
        "a16": rn(1024, 1024, scale=1 / 32), "b16": rn(1024, 2048, scale=1 / 32),
        "xs": rn(16, 8192, scale=1 / 64), "bs": rn(8192, 1024, scale=1 / 64),
        "a32": rn(2049, 3001, dtype=torch.float32), "b32": rn(3001, 2999, dtype=torch.float32),
        "x32": rn(300, 1000, dtype=torch.float32), "w32": rn(1000, 1000, dtype=torch.float32),
        "bias32": rn(1000, dtype=torch.float32),
        "p": rn(4, 256, 512, dtype=torch.bfloat16), "q": rn(4, 512, 384, dtype=torch.bfloat16),
        "img": rn(2, 64, 16, 16), "wc": rn(32, 64, 1, 1, scale=1 / 8), "bc": rn(32),
    }


def _calls(t):
    return [
        lambda: cmpext3.fp16_matmul(t["a16"], t["b16"]),            # tile kernel
        lambda: cmpext3.fp16_matmul(t["xs"], t["bs"]),              # skinny, K split + reduce
        lambda: cmpext3.fp32_matmul(t["a32"], t["b32"]),            # padded copies + 16-byte DMA
        lambda: cmpext3.linear(t["x32"], t["w32"], t["bias32"]),    # fp32, K split over waves, bias
        lambda: cmpext3.bmm(t["p"], t["q"]),
        lambda: cmpext3.conv2d(t["img"], t["wc"], t["bc"]),
    ]


def test_calls_cover_the_paths():
    t = _inputs()
    ran = []
    for f in _calls(t):
        f()
        ran.append(cmpext3.last_plan())
    torch.cuda.synchronize()
    assert "splits=" in ran[1] and "splits=1 " not in ran[1], ran[1]
    assert "padded=" in ran[2], ran[2]
    assert "k4" in ran[3], ran[3]


def test_graph_replays_match_eager():
    t = _inputs()
    calls = _calls(t)
    eager = [f() for f in calls]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream before capture
        for f in calls:
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [f() for f in calls]
    for rep in range(4):
        again = [f() for f in calls]  # eager work between the replays
        torch.cuda.synchronize()
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e, a) in enumerate(zip(outs, eager, again)):
            assert torch.equal(a, e), f"eager call {i} changed"
            assert torch.equal(o, e), f"replay {rep}: call {i} differs from the eager result"
