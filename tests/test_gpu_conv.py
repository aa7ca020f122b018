"""GPU parity of cmpext3.conv2d (1x1, stride 1, padding 0: one GEMM per image
on the NCHW data, bias per output channel) against the float64 CPU oracle
oracle.gemm_oracle.conv2d_1x1_f64 (the reference's 1x1 branch,
src/main.cpp:402-424), through the Python binding and the C ABI
(cmpext3_conv2d_1x1).  Bounds: relative Frobenius fp32 1e-5, fp16 2e-3,
bf16 1e-2."""
import numpy as np
import pytest
import torch

import cmpext3
from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
CODE = {"fp16": cabi.F16, "bf16": cabi.BF16, "fp32": cabi.F32}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


def make(dtype, B, C, H, W, Co, seed, with_bias=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, C, H, W, generator=g) / np.sqrt(max(C, 1))).to(DT[dtype])
    w = (torch.randn(Co, C, 1, 1, generator=g)).to(DT[dtype])
    bias = torch.randn(Co, generator=g).to(DT[dtype]) if with_bias else None
    return x, w, bias


def oracle(x, w, bias):
    return O.conv2d_1x1_f64(O.to_f64(x), O.to_f64(w), None if bias is None else O.to_f64(bias))


def kernel_for(dtype, B, C, H, W, Co):
    """Kernel the selector picks for this shape with aligned operands (a prediction)."""
    return cmpext3.plan(dtype, Co, H * W, C, batch=B, has_bias=True).split()[0].split("=")[1]


# (B, C_in, H, W, C_out): tiled kernels, skinny (C_out <= 64) with and without
# the K split, ragged H*W (generic path for 16-bit), a Stable-Diffusion-like
# 320-channel block, and C_out = 1.
SHAPES = [(2, 256, 32, 32, 512), (2, 512, 64, 64, 16), (1, 64, 7, 7, 96), (3, 40, 5, 9, 24),
          (1, 320, 64, 64, 320), (4, 128, 16, 16, 1), (1, 1, 8, 8, 8),
          (16, 128, 64, 64, 64), (64, 128, 32, 32, 40),  # few output channels, many pixels: tiled
          (4, 129, 31, 33, 200),  # odd channels and pixels: weight and images copied zero-padded
          (8, 64, 256, 256, 48),  # 4096 column tiles of 128 pixels: the streaming kernel
          (8, 96, 256, 256, 128),  # ... with 128-row tiles
          (16, 200, 128, 256, 56),  # ... K = 200 in two chunks of 128 input channels
          (16, 192, 128, 256, 96),  # ... 128-row tiles in two groups of 4 waves
          (16, 96, 128, 256, 320)]  # ... three row blocks of 128 output channels


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("shape", SHAPES)
def test_conv2d_1x1_matches_oracle(dtype, shape):
    B, C, H, W, Co = shape
    x, w, bias = make(dtype, B, C, H, W, Co, seed=sum(shape))
    print(f"conv2d {dtype} {shape} kernel={kernel_for(dtype, B, C, H, W, Co)}", flush=True)
    out = cmpext3.conv2d(x.cuda(), w.cuda(), bias.cuda())
    print(f"  ran: {cmpext3.last_plan()}", flush=True)
    torch.cuda.synchronize()
    assert out.shape == (B, Co, H, W) and out.dtype == DT[dtype] and out.is_contiguous()
    assert O.rel_frobenius(O.to_f64(out.cpu()), oracle(x, w, bias)) <= O.TOLERANCE[dtype]
    out_nb = cmpext3.conv2d(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    assert O.rel_frobenius(O.to_f64(out_nb.cpu()), oracle(x, w, None)) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("shape", [(8, 64, 256, 256, 48), (16, 192, 128, 256, 96), (16, 96, 128, 256, 320),
                                   (2, 40, 5, 9, 24)])
def test_conv2d_1x1_channels_last(dtype, shape):
    """NHWC (channels-last) inputs are read in place (B given as [H*W, C_in] per image; the
    streaming kernel for the large shapes): same result as the NCHW input, NCHW output."""
    B, C, H, W, Co = shape
    x, w, bias = make(dtype, B, C, H, W, Co, seed=sum(shape) + 1)
    xg = x.cuda().to(memory_format=torch.channels_last)
    assert not xg.is_contiguous() and xg.is_contiguous(memory_format=torch.channels_last)
    print(f"conv2d channels-last {dtype} {shape}", flush=True)
    out = cmpext3.conv2d(xg, w.cuda(), bias.cuda())
    print(f"  ran: {cmpext3.last_plan()}", flush=True)
    torch.cuda.synchronize()
    assert out.shape == (B, Co, H, W) and out.is_contiguous()
    if dtype != "fp32":
        assert "layout=NK" in cmpext3.last_plan()
    assert O.rel_frobenius(O.to_f64(out.cpu()), oracle(x, w, bias)) <= O.TOLERANCE[dtype]


@pytest.mark.parametrize("name", ["conv_f16_2x5x3x4_o6_bias", "conv_bf16_3x24x2x5_o7",
                                  "conv_f32_1x9x4x4_o3_bias"])
def test_conv2d_golden_fixtures(golden, name):
    dt = {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}[name.split("_")[1]]
    exp = golden[name + "/expected"]
    B, Co, H, W = exp.shape
    tdt, view = DT[dt], (torch.int32 if dt == "fp32" else torch.int16)
    x = torch.from_numpy(golden[name + "/x"].astype(np.int64)).to(view).view(tdt).reshape(B, -1, H, W)
    w = torch.from_numpy(golden[name + "/w"].astype(np.int64)).to(view).view(tdt).reshape(Co, -1, 1, 1)
    bias = None
    if name + "/bias" in golden:
        bias = torch.from_numpy(golden[name + "/bias"].astype(np.int64)).to(view).view(tdt).cuda()
    out = cmpext3.conv2d(x.cuda(), w.cuda(), bias)
    torch.cuda.synchronize()
    assert O.rel_frobenius(O.to_f64(out.cpu()), exp) <= O.TOLERANCE[dt]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_conv2d_exact_small_integers(dtype):
    """Integer inputs whose sums stay exact in fp32 and in the output dtype:
    the result equals the oracle bit for bit."""
    g = torch.Generator().manual_seed(5)
    x = torch.randint(-2, 3, (2, 96, 16, 16), generator=g).to(DT[dtype])
    w = torch.randint(-2, 3, (80, 96, 1, 1), generator=g).to(DT[dtype])
    bias = torch.randint(-4, 5, (80,), generator=g).to(DT[dtype])
    out = cmpext3.conv2d(x.cuda(), w.cuda(), bias.cuda())
    torch.cuda.synchronize()
    assert np.array_equal(O.to_f64(out.cpu()), oracle(x, w, bias))


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_conv2d_c_abi_matches_binding(dtype):
    for (B, C, H, W, Co) in [(2, 256, 32, 32, 512), (2, 512, 64, 64, 16), (1, 64, 7, 7, 96)]:
        x, w, bias = make(dtype, B, C, H, W, Co, seed=B + C)
        xg, wg, bg = x.cuda(), w.cuda(), bias.cuda()
        ref = cmpext3.conv2d(xg, wg, bg)
        out = torch.empty_like(ref)
        ws_bytes = cabi.workspace_size(CODE[dtype], cabi.B_KN, Co, H * W, C, B)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") if ws_bytes > 0 else None
        assert cabi.conv2d_1x1(CODE[dtype], xg, wg, bg, out, B, C, Co, H * W, ws) == cabi.OK
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        # without a workspace (skinny shapes then run unsplit): within tolerance
        out2 = torch.empty_like(ref)
        assert cabi.conv2d_1x1(CODE[dtype], xg, wg, bg, out2, B, C, Co, H * W) == cabi.OK
        torch.cuda.synchronize()
        assert O.rel_frobenius(O.to_f64(out2.cpu()), oracle(x, w, bias)) <= O.TOLERANCE[dtype]


def test_conv2d_each_image_equals_its_gemm():
    """Image b of the batched launch is W @ X_b (+ bias per row): bit-identical
    to the single-image call (same kernel), and equal to linear on the NHWC
    view within tolerance (the reference's own route)."""
    x, w, bias = make("bf16", 3, 128, 16, 16, 192, seed=7)
    xg, wg, bg = x.cuda(), w.cuda(), bias.cuda()
    out = cmpext3.conv2d(xg, wg, bg)
    for b in range(3):
        single = cmpext3.conv2d(xg[b:b + 1], wg, bg)
        if kernel_for("bf16", 1, 128, 16, 16, 192) == kernel_for("bf16", 3, 128, 16, 16, 192):
            assert torch.equal(single[0], out[b])
    via_linear = cmpext3.linear(xg.permute(0, 2, 3, 1), wg.view(192, 128), bg).permute(0, 3, 1, 2)
    torch.cuda.synchronize()
    assert O.rel_frobenius(O.to_f64(via_linear.cpu()), O.to_f64(out.cpu())) <= O.TOLERANCE["bf16"]


def test_conv2d_empty_and_noncontiguous():
    x, w, bias = make("fp16", 2, 32, 8, 8, 16, seed=3)
    # zero batch and zero pixels: empty outputs, nothing launched
    assert cmpext3.conv2d(x[:0].cuda(), w.cuda(), bias.cuda()).shape == (0, 16, 8, 8)
    assert cmpext3.conv2d(x[:, :, :0].cuda(), w.cuda(), bias.cuda()).shape == (2, 16, 0, 8)
    # a channels-last input is made contiguous first
    xcl = x.cuda().to(memory_format=torch.channels_last)
    out = cmpext3.conv2d(xcl, w.cuda(), bias.cuda())
    torch.cuda.synchronize()
    assert O.rel_frobenius(O.to_f64(out.cpu()), oracle(x, w, bias)) <= O.TOLERANCE["fp16"]
