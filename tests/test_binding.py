"""Python surface of the extension: import, signatures and argument checks
that fail before any GPU work (no GPU needed)."""
import pytest
import torch

import cmpext3


def test_module_surface():
    for name in ["fp16_matmul", "bf16_matmul", "fp32_matmul", "linear", "bmm", "plan", "version"]:
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
