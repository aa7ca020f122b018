"""cmpext3 dense GEMM operators for AMD Instinct MI355X (gfx950).

Python surface (same names and argument meaning as the reference extension's
GEMM entry points, src/main.cpp:1594-1602, plus the dtype-specific matmuls):

    fp16_matmul(a, b), bf16_matmul(a, b), fp32_matmul(a, b)   C = A @ B
    linear(input, weight, bias=None)                          input @ weight.T + bias
    bmm(input, mat2)                                           batched A @ B
    conv2d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1)
                                                               1x1 NCHW convolution as a GEMM
    plan(dtype, M, N, K, layout="KN", batch=1, has_bias=False) kernel the selector picks
    last_plan()                                                kernel(s) this thread's last call ran

Every call runs the hand-written gfx950 kernels of lib/libcmpext3_gemm.so on
PyTorch's current stream.  There is no fallback: if the compiled extension is
missing, every operator access (and `import cmpext3`) raises ImportError; only
the `build` submodule stays usable.
"""
import torch  # noqa: F401  (loads PyTorch's HIP runtime before the extension binds to it)

__all__ = ["fp16_matmul", "bf16_matmul", "fp32_matmul", "linear", "bmm", "conv2d", "plan", "last_plan",
           "version"]

try:
    from . import _cmpext3 as _ext

    _missing = [n for n in __all__ if not hasattr(_ext, n)]
    if _missing:  # built from older sources
        raise ImportError(f"{_ext.__file__} is stale (lacks {', '.join(_missing)}); rebuild it")
except ImportError as _e:  # a tree that was not built: every operator access raises
    _ext = None
    _ext_error = _e

if _ext is not None:
    fp16_matmul = _ext.fp16_matmul
    bf16_matmul = _ext.bf16_matmul
    fp32_matmul = _ext.fp32_matmul
    linear = _ext.linear
    bmm = _ext.bmm
    conv2d = _ext.conv2d
    plan = _ext.plan
    last_plan = _ext.last_plan
    version = _ext.version
    extension_path = _ext.__file__
else:

    def __getattr__(name):
        # The submodule `cmp_ext_amd.build` stays importable so that an unbuilt tree can be
        # built; any operator (and `from cmp_ext_amd import *`, hence `import cmpext3`) fails.
        if name not in __all__ and name != "extension_path":
            raise AttributeError(name)
        raise ImportError(
            "cmp_ext_amd: the compiled extension is missing; run `python -m cmp_ext_amd.build` "
            f"(or __graft_entry__.build()) first ({_ext_error})"
        ) from _ext_error
