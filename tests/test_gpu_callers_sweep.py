"""Seeded random sweep of the Python operators (cmpext3.fp16/bf16/fp32_matmul,
linear, bmm, conv2d) on views and shapes a caller of the reference's module
passes: row slices and column slices of larger tensors (row pitch above the
width, misaligned base pointers), transposed operands (the matmul's B consumed
in place as [N, K]; the others copied), stepped views, 2- to 4-D linear
inputs, offset batch slices, channels-last convolution inputs and misaligned
bias views.  Every result is checked against the float64 oracle
(oracle.gemm_oracle: matmul_f64 / linear_f64 / bmm_f64 / conv2d_1x1_f64; the
reference's semantics, src/main.cpp:155-424) within the operator contract's
bound, with the output's shape, dtype, device and contiguity; the inputs must
come back unchanged.
"""
import numpy as np
import pytest
import torch

import cmpext3
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
MATMUL = {"fp16": cmpext3.fp16_matmul, "bf16": cmpext3.bf16_matmul, "fp32": cmpext3.fp32_matmul}
N_EACH = 30


def _dim(rng, lo, hi):
    x = int(rng.integers(lo, hi))
    return (x + 7) // 8 * 8 if rng.random() < 0.5 else x


def _matrix(rng, gen, rows, cols, dt, how, scale=1.0):
    """A [rows, cols] GPU operand made `how`: plain, a row/column slice of a larger
    tensor, a transposed view, or a stepped view."""
    def rnd(*shape):
        return (torch.randn(*shape, generator=gen) * scale).to(dt).cuda()
    if how == "plain":
        return rnd(rows, cols)
    if how == "rows":      # rows r0 .. r0+rows of a taller tensor: misaligned base when r0*cols is odd
        r0 = int(rng.integers(1, 4))
        return rnd(rows + r0 + 1, cols)[r0:r0 + rows]
    if how == "cols":      # columns c0 .. c0+cols of a wider tensor: row pitch > cols
        c0 = int(rng.integers(0, 9))
        return rnd(rows, cols + c0 + int(rng.integers(0, 9)))[:, c0:c0 + cols]
    if how == "t":         # transposed view of a contiguous [cols, rows] tensor
        return rnd(cols, rows).t()
    if how == "step":      # every other column of a tensor twice as wide
        return rnd(rows, 2 * cols)[:, ::2]
    raise ValueError(how)


def matmul_cases():
    rng = np.random.default_rng(11)
    out = []
    for i in range(N_EACH):
        dtype = ["fp16", "bf16", "fp32"][i % 3]
        M, N, K = _dim(rng, 1, 300), _dim(rng, 1, 300), _dim(rng, 1, 300)
        out.append(dict(i=i, dtype=dtype, M=M, N=N, K=K,
                        a=str(rng.choice(["plain", "rows", "cols", "t", "step"])),
                        b=str(rng.choice(["plain", "rows", "cols", "t", "step"]))))
    return out


def linear_cases():
    rng = np.random.default_rng(12)
    out = []
    for i in range(N_EACH):
        dtype = ["fp16", "bf16", "fp32"][i % 3]
        lead = [int(x) for x in rng.integers(1, 9, size=int(rng.integers(1, 4)))]
        if rng.random() < 0.1:
            lead[0] = 0
        out.append(dict(i=i, dtype=dtype, lead=lead, N=_dim(rng, 1, 400), K=_dim(rng, 1, 400),
                        x=str(rng.choice(["plain", "t", "step"])), w=str(rng.choice(["plain", "rows", "cols"])),
                        bias=str(rng.choice(["none", "plain", "offset"]))))
    return out


def bmm_cases():
    rng = np.random.default_rng(13)
    out = []
    for i in range(N_EACH):
        dtype = ["fp16", "bf16", "fp32"][i % 3]
        out.append(dict(i=i, dtype=dtype, B=int(rng.integers(1, 6)), M=_dim(rng, 1, 200), N=_dim(rng, 1, 200),
                        K=_dim(rng, 1, 200), a=str(rng.choice(["plain", "t", "offset"])),
                        b=str(rng.choice(["plain", "t", "offset"]))))
    return out


def conv_cases():
    rng = np.random.default_rng(14)
    out = []
    for i in range(N_EACH):
        dtype = ["fp16", "bf16", "fp32"][i % 3]
        out.append(dict(i=i, dtype=dtype, B=int(rng.integers(1, 4)), C=_dim(rng, 1, 160), H=int(rng.integers(1, 24)),
                        W=int(rng.integers(1, 24)), Co=_dim(rng, 1, 160),
                        x=str(rng.choice(["plain", "channels_last", "offset"])),
                        bias=str(rng.choice(["none", "plain", "offset"])),
                        args=int(rng.integers(3))))
    return out


def _close(out, ref, dtype, what):
    err = O.rel_frobenius(O.to_f64(out.cpu()), ref)
    assert err <= O.TOLERANCE[dtype], f"{what}: rel err {err:.3e}"


def _unchanged(t, before):
    assert torch.equal(t.cpu(), before), "an input was modified"


@pytest.mark.parametrize("c", matmul_cases(), ids=lambda c: f"m{c['i']}")
def test_matmul_views(c):
    rng = np.random.default_rng(100 + c["i"])
    gen = torch.Generator().manual_seed(100 + c["i"])
    dt = DT[c["dtype"]]
    a = _matrix(rng, gen, c["M"], c["K"], dt, c["a"], 1.0 / max(c["K"], 1) ** 0.5)
    b = _matrix(rng, gen, c["K"], c["N"], dt, c["b"])
    a0, b0 = a.cpu(), b.cpu()
    print(f"matmul {c}", flush=True)
    out = MATMUL[c["dtype"]](a, b)
    torch.cuda.synchronize()
    assert out.shape == (c["M"], c["N"]) and out.dtype == dt and out.is_cuda and out.is_contiguous()
    _close(out, O.matmul_f64(O.to_f64(a0), O.to_f64(b0)), c["dtype"], str(c))
    _unchanged(a, a0)
    _unchanged(b, b0)


@pytest.mark.parametrize("c", linear_cases(), ids=lambda c: f"l{c['i']}")
def test_linear_views(c):
    rng = np.random.default_rng(200 + c["i"])
    gen = torch.Generator().manual_seed(200 + c["i"])
    dt = DT[c["dtype"]]
    N, K, lead = c["N"], c["K"], c["lead"]
    scale = 1.0 / max(K, 1) ** 0.5
    if c["x"] == "plain":
        x = (torch.randn(*lead, K, generator=gen) * scale).to(dt).cuda()
    elif c["x"] == "step":    # every other element of a last dimension twice as long
        x = (torch.randn(*lead, 2 * K, generator=gen) * scale).to(dt).cuda()[..., ::2]
    elif len(lead) == 1:      # transposed view of a contiguous [K, rows] tensor
        x = (torch.randn(K, lead[0], generator=gen) * scale).to(dt).cuda().t()
    else:                     # the last two leading dimensions swapped
        x = (torch.randn(*lead[:-2], lead[-1], lead[-2], K, generator=gen) * scale).to(dt).cuda().transpose(-2, -3)
    w = _matrix(rng, gen, N, K, dt, c["w"])
    bias = None
    if c["bias"] == "plain":
        bias = torch.randn(N, generator=gen).to(dt).cuda()
    elif c["bias"] == "offset":  # a view starting one element in: 2-byte aligned for 16-bit dtypes
        bias = torch.randn(N + 1, generator=gen).to(dt).cuda()[1:]
    x0, w0 = x.cpu(), w.cpu()
    print(f"linear {c}", flush=True)
    out = cmpext3.linear(x, w, bias)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (*lead, N) and out.dtype == dt and out.is_cuda and out.is_contiguous()
    ref = O.linear_f64(O.to_f64(x0), O.to_f64(w0), None if bias is None else O.to_f64(bias.cpu()))
    _close(out, ref, c["dtype"], str(c))
    _unchanged(x, x0)
    _unchanged(w, w0)


def _batched(rng, gen, B, rows, cols, dt, how, scale=1.0):
    def rnd(*shape):
        return (torch.randn(*shape, generator=gen) * scale).to(dt).cuda()
    if how == "plain":
        return rnd(B, rows, cols)
    if how == "t":       # last two dimensions transposed
        return rnd(B, cols, rows).transpose(1, 2)
    if how == "offset":  # batch entries 1 .. B of a larger batch
        return rnd(B + 1, rows, cols)[1:]
    raise ValueError(how)


@pytest.mark.parametrize("c", bmm_cases(), ids=lambda c: f"b{c['i']}")
def test_bmm_views(c):
    rng = np.random.default_rng(300 + c["i"])
    gen = torch.Generator().manual_seed(300 + c["i"])
    dt = DT[c["dtype"]]
    a = _batched(rng, gen, c["B"], c["M"], c["K"], dt, c["a"], 1.0 / max(c["K"], 1) ** 0.5)
    b = _batched(rng, gen, c["B"], c["K"], c["N"], dt, c["b"])
    a0, b0 = a.cpu(), b.cpu()
    print(f"bmm {c}", flush=True)
    out = cmpext3.bmm(a, b)
    torch.cuda.synchronize()
    assert out.shape == (c["B"], c["M"], c["N"]) and out.dtype == dt and out.is_contiguous()
    _close(out, O.bmm_f64(O.to_f64(a0), O.to_f64(b0)), c["dtype"], str(c))
    _unchanged(a, a0)
    _unchanged(b, b0)


@pytest.mark.parametrize("c", conv_cases(), ids=lambda c: f"c{c['i']}")
def test_conv2d_views(c):
    gen = torch.Generator().manual_seed(400 + c["i"])
    dt = DT[c["dtype"]]
    B, C, H, W, Co = c["B"], c["C"], c["H"], c["W"], c["Co"]
    x = torch.randn(B + (c["x"] == "offset"), C, H, W, generator=gen).to(dt).cuda()
    if c["x"] == "offset":
        x = x[1:]
    elif c["x"] == "channels_last":
        x = x.to(memory_format=torch.channels_last)
    w = (torch.randn(Co, C, 1, 1, generator=gen) / max(C, 1) ** 0.5).to(dt).cuda()
    bias = None
    if c["bias"] == "plain":
        bias = torch.randn(Co, generator=gen).to(dt).cuda()
    elif c["bias"] == "offset":
        bias = torch.randn(Co + 1, generator=gen).to(dt).cuda()[1:]
    x0 = x.cpu()
    print(f"conv2d {c}", flush=True)
    if c["args"] == 0:
        out = cmpext3.conv2d(x, w, bias)
    elif c["args"] == 1:
        out = cmpext3.conv2d(x, w, bias, 1, 0)
    else:
        out = cmpext3.conv2d(x, w, bias, (1, 1), (0, 0), (1, 1), 1)
    torch.cuda.synchronize()
    assert out.shape == (B, Co, H, W) and out.dtype == dt and out.is_contiguous()
    ref = O.conv2d_1x1_f64(O.to_f64(x0), O.to_f64(w.cpu()), None if bias is None else O.to_f64(bias.cpu()))
    _close(out, ref, c["dtype"], str(c))
    _unchanged(x, x0)
