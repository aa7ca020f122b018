"""Python surface of the extension: import, signatures and argument checks
that fail before any GPU work (no GPU needed)."""
import pytest
import torch

import cmpext3


def test_module_surface():
    for name in ["fp16_matmul", "bf16_matmul", "fp32_matmul", "linear", "bmm", "conv2d", "plan", "version"]:
        assert callable(getattr(cmpext3, name))
    assert "gfx950" in cmpext3.version()
    assert cmpext3.extension_path.endswith(".so")


def test_plan_strings():
    assert "tile256x256" in cmpext3.plan("f16", 4096, 4096, 4096)
    assert "skinny" in cmpext3.plan("fp16", 16, 8192, 8192)
    assert "layout=NK" in cmpext3.plan("bf16", 100, 200, 64, layout="NK", has_bias=True)
    with pytest.raises(RuntimeError):
        cmpext3.plan("int8", 4, 4, 4)


@pytest.mark.parametrize("fn,dt", [(cmpext3.fp16_matmul, torch.float16), (cmpext3.bf16_matmul, torch.bfloat16),
                                   (cmpext3.fp32_matmul, torch.float32)])
def test_matmul_argument_checks(fn, dt):
    a = torch.zeros(4, 8, dtype=dt)
    b = torch.zeros(8, 3, dtype=dt)
    with pytest.raises(RuntimeError, match="on a GPU"):
        fn(a, b)                                  # CPU tensors are rejected (the reference does not check)
    with pytest.raises(RuntimeError, match="2-D"):
        fn(a[None], b)
    with pytest.raises(RuntimeError, match="expected"):
        fn(a.double(), b.double())
    with pytest.raises(RuntimeError, match="mismatch"):
        fn(a, torch.zeros(7, 3, dtype=dt))


def test_linear_and_bmm_argument_checks():
    x = torch.zeros(2, 4, 8, dtype=torch.float16)
    w = torch.zeros(5, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Input dim >= 2"):
        cmpext3.linear(torch.zeros(8, dtype=torch.float16), w)
    with pytest.raises(RuntimeError, match="Weight dim == 2"):
        cmpext3.linear(x, w[None])
    with pytest.raises(RuntimeError, match="Input shape mismatch"):
        cmpext3.linear(x, torch.zeros(5, 7, dtype=torch.float16))
    with pytest.raises(RuntimeError):
        cmpext3.linear(x, w)                      # CPU
    with pytest.raises(RuntimeError, match="3D"):
        cmpext3.bmm(x[0], x)
    with pytest.raises(RuntimeError, match="Batch size mismatch"):
        cmpext3.bmm(x, torch.zeros(3, 8, 2, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="Contracting dimension"):
        cmpext3.bmm(x, torch.zeros(2, 7, 2, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="Dtype mismatch"):
        cmpext3.bmm(x, torch.zeros(2, 8, 2, dtype=torch.float32))


def test_conv2d_argument_checks():
    """The reference's conv2d checks (src/main.cpp:372-388) in the same order,
    then the 1x1 / stride 1 / padding 0 / dilation 1 restriction of this
    library, all before any GPU work."""
    x = torch.zeros(2, 8, 5, 5, dtype=torch.float16)
    w = torch.zeros(4, 8, 1, 1, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Input must be 4D"):
        cmpext3.conv2d(x[0], w)
    with pytest.raises(RuntimeError, match="Weight must be 4D"):
        cmpext3.conv2d(x, w[:, :, 0, 0])
    with pytest.raises(RuntimeError, match="only groups=1"):
        cmpext3.conv2d(x, w, groups=2)
    with pytest.raises(RuntimeError, match="Input channels mismatch"):
        cmpext3.conv2d(x, torch.zeros(4, 7, 1, 1, dtype=torch.float16))
    for kw in (dict(stride=2), dict(stride=(1, 2)), dict(padding=1), dict(padding=[0, 1]), dict(dilation=2)):
        with pytest.raises(RuntimeError, match="only the 1x1 kernel"):
            cmpext3.conv2d(x, w, **kw)
    with pytest.raises(RuntimeError, match="only the 1x1 kernel"):
        cmpext3.conv2d(x, torch.zeros(4, 8, 3, 3, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="Dtype mismatch"):
        cmpext3.conv2d(x, w.float())
    with pytest.raises(RuntimeError, match="Unsupported dtype"):
        cmpext3.conv2d(x.double(), w.double())
    with pytest.raises(RuntimeError, match="on a GPU"):
        cmpext3.conv2d(x, w, stride=(1, 1), padding=(0, 0), dilation=[1])   # sequences accepted; CPU rejected
