"""ctypes view of the C ABI in include/cmpext3_gemm.h (libcmpext3_gemm.so).

Used by the tests and the benchmark to drive the kernels through the same
boundary a non-Python caller would bind.  PyTorch is imported first so that
the library binds to PyTorch's HIP runtime (a second runtime in the process
would not understand PyTorch's stream handles).
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libcmpext3_gemm.so")

F16, BF16, F32 = 0, 1, 2
B_KN, B_NK = 0, 1
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_TOO_LARGE, ERR_WORKSPACE, ERR_SCRATCH = 0, -1, -2, -3, -4, -5
SCRATCH_BYTES = 64 << 20
BIAS_PER_ROW = 1

# Exported symbols and their C signatures, as declared in include/cmpext3_gemm.h.
_i, _i64, _p, _cp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_char_p
SIGNATURES = {
    "cmpext3_matmul_fp16": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "cmpext3_matmul_bf16": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "cmpext3_matmul_fp32": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "cmpext3_gemm_f16": (_i, [_p, _i64, _p, _i64, _p, _i64, _i, _i, _i, _p]),
    "cmpext3_gemm_bf16": (_i, [_p, _i64, _p, _i64, _p, _i64, _i, _i, _i, _p]),
    "cmpext3_gemm_f32": (_i, [_p, _i64, _p, _i64, _p, _i64, _i, _i, _i, _p]),
    "cmpext3_gemm_ex": (_i, [_i, _i, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p,
                             _i, _i, _i, _i, _p, _i64, _p]),
    "cmpext3_conv2d_1x1": (_i, [_i, _p, _p, _p, _p, _i, _i, _i, _i, _p, _i64, _p]),
    "cmpext3_gemm_workspace_size": (_i64, [_i, _i, _i, _i, _i, _i]),
    "cmpext3_gemm_plan": (_i, [_i, _i, _i, _i, _i, _i64, _i64, _i64, _i, _i, _i, _i64, _cp, _i]),
    "cmpext3_gemm_prepare": (_i, [_p, _i, _i, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i,
                                  _i, _i, _i, _i, _i64]),
    "cmpext3_gemm_call_workspace_size": (_i64, [_p]),
    "cmpext3_gemm_call_describe": (_i, [_p, _cp, _i]),
    "cmpext3_gemm_run": (_i, [_p, _p, _i64, _p]),
    "cmpext3_gemm_ex_noalloc": (_i, [_i, _i, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p,
                                     _i, _i, _i, _i, _p]),
    "cmpext3_status_string": (_cp, [_i]),
    "cmpext3_version": (_cp, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} not built; run `python -m cmp_ext_amd.build`")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def status_string(st: int) -> str:
    return lib().cmpext3_status_string(st).decode()


def plan(dtype: int, layout: int, M: int, N: int, K: int, lda: int | None = None,
         ldb: int | None = None, ldc: int | None = None, align: int = 16, has_bias: bool = False,
         batch: int = 1, workspace_bytes: int = 0) -> tuple[int, str]:
    lda = max(K, 1) if lda is None else lda
    ldb = max(N if layout == B_KN else K, 1) if ldb is None else ldb
    ldc = max(N, 1) if ldc is None else ldc
    buf = ctypes.create_string_buffer(640)
    kid = lib().cmpext3_gemm_plan(dtype, layout, M, N, K, lda, ldb, ldc, align, int(has_bias), batch,
                                  workspace_bytes, buf, 640)
    return kid, buf.value.decode()


def workspace_size(dtype: int, layout: int, M: int, N: int, K: int, batch: int = 1) -> int:
    return lib().cmpext3_gemm_workspace_size(dtype, layout, M, N, K, batch)


def _stream_handle(stream) -> int | None:
    if stream is None:
        if not torch.cuda.is_available():  # argument checks on a machine without a GPU
            return None
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def gemm_ex(dtype: int, layout: int, A, lda: int, stride_a: int, B, ldb: int, stride_b: int, C,
            ldc: int, stride_c: int, bias, M: int, N: int, K: int, batch: int = 1, workspace=None,
            stream=None) -> int:
    """Call cmpext3_gemm_ex with raw device pointers (ints) or tensors.
    `workspace` is None or a device tensor (its byte size is passed)."""
    def ptr(x):
        if x is None:
            return None
        return x.data_ptr() if hasattr(x, "data_ptr") else int(x)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return lib().cmpext3_gemm_ex(dtype, layout, ptr(A), lda, stride_a, ptr(B), ldb, stride_b, ptr(C),
                                 ldc, stride_c, ptr(bias), M, N, K, batch, ptr(workspace), ws_bytes,
                                 _stream_handle(stream))


class Call(ctypes.Structure):
    """cmpext3_gemm_call: one prepared GEMM (opaque, 512 bytes)."""
    _fields_ = [("opaque", ctypes.c_int64 * 64)]


def _ptr(x):
    if x is None:
        return None
    return x.data_ptr() if hasattr(x, "data_ptr") else int(x)


def prepare(dtype: int, layout: int, A, lda: int, stride_a: int, B, ldb: int, stride_b: int, C,
            ldc: int, stride_c: int, bias, M: int, N: int, K: int, batch: int = 1, flags: int = 0,
            workspace_limit: int = (1 << 63) - 1) -> tuple[int, Call]:
    """cmpext3_gemm_prepare: returns (status, call)."""
    call = Call()
    st = lib().cmpext3_gemm_prepare(ctypes.byref(call), dtype, layout, _ptr(A), lda, stride_a, _ptr(B), ldb,
                                    stride_b, _ptr(C), ldc, stride_c, _ptr(bias), flags, M, N, K, batch,
                                    workspace_limit)
    return st, call


def call_workspace_size(call: Call) -> int:
    return lib().cmpext3_gemm_call_workspace_size(ctypes.byref(call))


def describe(call: Call) -> tuple[int, str]:
    buf = ctypes.create_string_buffer(640)
    kid = lib().cmpext3_gemm_call_describe(ctypes.byref(call), buf, 640)
    return kid, buf.value.decode()


def run(call: Call, workspace=None, workspace_bytes: int | None = None, stream=None) -> int:
    """cmpext3_gemm_run; `workspace` is None or a device tensor (its byte size is passed
    unless `workspace_bytes` says otherwise)."""
    if workspace_bytes is None:
        workspace_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return lib().cmpext3_gemm_run(ctypes.byref(call), _ptr(workspace), workspace_bytes, _stream_handle(stream))


def gemm_ex_noalloc(dtype: int, layout: int, A, lda: int, stride_a: int, B, ldb: int, stride_b: int, C,
                    ldc: int, stride_c: int, bias, M: int, N: int, K: int, batch: int = 1, stream=None) -> int:
    """Call cmpext3_gemm_ex_noalloc (the library's static scratch buffer as workspace)."""
    return lib().cmpext3_gemm_ex_noalloc(dtype, layout, _ptr(A), lda, stride_a, _ptr(B), ldb, stride_b, _ptr(C),
                                         ldc, stride_c, _ptr(bias), M, N, K, batch, _stream_handle(stream))


def conv2d_1x1(dtype: int, inp, weight, bias, out, batch: int, c_in: int, c_out: int, hw: int,
               workspace=None, stream=None) -> int:
    """Call cmpext3_conv2d_1x1 (contiguous NCHW input/output, [c_out, c_in] weight)."""
    def ptr(x):
        if x is None:
            return None
        return x.data_ptr() if hasattr(x, "data_ptr") else int(x)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return lib().cmpext3_conv2d_1x1(dtype, ptr(inp), ptr(weight), ptr(bias), ptr(out), batch, c_in, c_out,
                                    hw, ptr(workspace), ws_bytes, _stream_handle(stream))


def gemm_strided(dtype: int, A, lda: int, B, ldb: int, C, ldc: int, M: int, N: int, K: int, stream=None) -> int:
    """Call cmpext3_gemm_{f16,bf16,f32} (row pitches in elements; A, B, C may be views)."""
    fn = {F16: lib().cmpext3_gemm_f16, BF16: lib().cmpext3_gemm_bf16, F32: lib().cmpext3_gemm_f32}[dtype]
    return fn(A.data_ptr(), lda, B.data_ptr(), ldb, C.data_ptr(), ldc, M, N, K, _stream_handle(stream))


def matmul(dtype: int, A, B, C, M: int, N: int, K: int, stream=None) -> int:
    """Call cmpext3_matmul_{fp16,bf16,fp32} (packed row-major operands)."""
    fn = {F16: lib().cmpext3_matmul_fp16, BF16: lib().cmpext3_matmul_bf16,
          F32: lib().cmpext3_matmul_fp32}[dtype]
    return fn(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, _stream_handle(stream))
