import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402,F401  (PyTorch's HIP runtime must be loaded before libcmpext3_gemm.so)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def has_gpu() -> bool:
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def oracle_c():
    """ctypes handle to the plain-C brute-force oracle (built here if missing)."""
    import ctypes

    so = os.path.join(ROOT, "oracle", "liboracle_gemm.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(so)
    d, i, i64, p = ctypes.c_double, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
    lib.oracle_gemm_f64.argtypes = [i, p, i64, p, i64, p, i64, i, i, i]
    lib.oracle_gemm_f64.restype = None
    lib.oracle_f16_bits_to_f64.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_bits_to_f64.restype = d
    lib.oracle_bf16_bits_to_f64.argtypes = [ctypes.c_uint16]
    lib.oracle_bf16_bits_to_f64.restype = d
    lib.oracle_f32_to_bf16_bits.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_bf16_bits.restype = ctypes.c_uint16
    return lib


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(os.path.join(ROOT, "tests", "golden", "gemm_golden.npz"))
