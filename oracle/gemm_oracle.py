"""CPU restatement of the reference GEMM operators -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module.

What it restates (eastmoe/cmp_ext, read as text, never run):
  * matmul: C[m, n] = sum_k A[m*lda + k] * B[k*ldb + n] with lda = K,
    ldb = N, ldc = N -- launch_matmul_fp16 (src/cuda/fp16_matmul.cu:301-321),
    launch_matmul_bf16 (src/cuda/bf16_matmul.cu:232-247) and
    launch_matmul_fp32 (src/cuda/fp32_matmul.cu:236-254).
  * linear(input[..., K], weight[N, K], bias[N]) = input @ weight^T + bias,
    output shaped [..., N] -- custom_linear_forward (src/main.cpp:155-256).
  * bmm(input[B, M, K], mat2[B, K, N]) = per-batch matmul --
    custom_bmm_forward (src/main.cpp:273-357).
  * conv2d with a 1x1 kernel, stride 1, padding 0, dilation 1, groups 1:
    NCHW -> NHWC, linear with the [C_out, C_in] view of the weight (+ bias),
    NHWC -> NCHW -- the 1x1 branch of custom_conv2d_forward
    (src/main.cpp:402-424).
The reference accumulates fp16/bf16 products in half precision
(fp16_matmul.cu:86-98, bf16_matmul.cu:65-77); the operator contract this
build implements (fp32 accumulation, one final rounding to the input dtype)
is checked against the exact value of the sum instead: a float64 product of
the dtype-rounded inputs, with the relative-Frobenius bounds below.

Pinning (tests/test_oracle.py): matmul_f64 is checked against an exactly
rounded dot product per element (math.fsum of exact float64 products, via the
committed golden fixtures and directly), against the plain-C triple loop in
oracle/gemm_ref.c, and against closed forms (identity, permutation, zero,
rank-1 integer, K = 1, transpose and linearity identities).  conv2d_1x1_f64
is checked against exactly rounded golden values, against
torch.nn.functional.conv2d in float64 and against matmul_f64 per image.  The dtype
rounding functions are checked against IEEE bit-level decoding in C and
against exhaustive/boundary cases.  make_inputs (the seeded benchmark inputs)
is checked against the distributions BASELINE.json names -- Kolmogorov-Smirnov
against scipy's uniform[-1, 1] and normal(0, scale) CDFs, range, mean and
spread within a few standard errors -- and for the order of its draws (A
first, then B from the same generator) and the independence of A and B;
planted mistakes (rand for randn, a wrong scale, a [0, 1) range, B equal to A)
each fail those checks.
"""
from __future__ import annotations

import numpy as np

# Relative Frobenius error bounds of the operator contract.
TOLERANCE = {"fp32": 1e-5, "fp16": 2e-3, "bf16": 1e-2}

# The five benchmark/parity configurations (BASELINE.json "configs").
CONFIGS = {
    "cfg1_fp32_512": dict(dtype="fp32", M=512, N=512, K=512, dist="uniform"),
    "cfg2_fp16_4096": dict(dtype="fp16", M=4096, N=4096, K=4096, dist="normal", scale=1.0 / 64.0),
    "cfg3_bf16_mlp": dict(dtype="bf16", M=4096, N=14336, K=4096, dist="normal", scale=0.02),
    "cfg4_fp16_skinny": dict(dtype="fp16", M=16, N=8192, K=8192, dist="normal",
                             scale=1.0 / float(np.sqrt(8192.0))),
    "cfg5_fp32_ragged": dict(dtype="fp32", M=4097, N=3001, K=2049, dist="uniform"),
}


def round_fp16(x: np.ndarray) -> np.ndarray:
    """Round to IEEE binary16 (round to nearest even) and widen to float64."""
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float64)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest even; NaN stays NaN)
    and widen to float64.  bf16 is the top 16 bits of an IEEE binary32."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    nan = np.isnan(f)
    r = np.where(nan, (u | 0x400000) & 0xFFFF0000, r)
    return (r.astype(np.uint32)).view(np.float32).astype(np.float64)


def matmul_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = A @ B in float64 (row-major semantics of fp16_matmul.cu:311-313)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"shape mismatch {a.shape} x {b.shape}")
    if a.shape[1] == 0:
        return np.zeros((a.shape[0], b.shape[1]), dtype=np.float64)
    return a @ b


def linear_f64(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """input @ weight^T + bias, leading dims kept (src/main.cpp:155-256)."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    if x.ndim < 2 or w.ndim != 2 or x.shape[-1] != w.shape[1]:
        raise ValueError("linear: bad shapes")
    out = matmul_f64(x.reshape(-1, x.shape[-1]), w.T)
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None, :]
    return out.reshape(*x.shape[:-1], w.shape[0])


def bmm_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Per-batch matmul (src/main.cpp:273-357)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.ndim != 3 or b.ndim != 3 or a.shape[0] != b.shape[0] or a.shape[2] != b.shape[1]:
        raise ValueError("bmm: bad shapes")
    return np.stack([matmul_f64(a[i], b[i]) for i in range(a.shape[0])]) if a.shape[0] else \
        np.zeros((0, a.shape[1], b.shape[2]))


def conv2d_1x1_f64(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """1x1 convolution as the reference computes it (src/main.cpp:402-424):
    input [B, C_in, H, W] permuted to NHWC (:407), linear against the weight
    viewed as [C_out, C_in] (:410, :418), result permuted back to
    [B, C_out, H, W] (:423)."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    if x.ndim != 4 or w.ndim != 4 or w.shape[2:] != (1, 1) or x.shape[1] != w.shape[1]:
        raise ValueError("conv2d_1x1: bad shapes")
    nhwc = np.transpose(x, (0, 2, 3, 1))
    out = linear_f64(nhwc, w.reshape(w.shape[0], w.shape[1]), bias) if x.shape[1] else \
        np.zeros(nhwc.shape[:3] + (w.shape[0],)) + (0 if bias is None else np.asarray(bias, np.float64))
    return np.ascontiguousarray(np.transpose(out, (0, 3, 1, 2)))


def rel_frobenius(out: np.ndarray, ref: np.ndarray) -> float:
    """||out - ref||_F / ||ref||_F (0 when both are zero)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = float(np.linalg.norm((out - ref).ravel()))
    den = float(np.linalg.norm(ref.ravel()))
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


def make_inputs(dtype: str, M: int, N: int, K: int, dist: str, scale: float = 1.0, seed: int = 0,
                b_layout: str = "KN"):
    """Seeded inputs of the benchmark configurations: a CPU torch.Generator seeded
    with `seed` draws A first, then B, both in float32 (uniform[-1, 1] or
    normal(0, 1) * scale), and each is then cast to `dtype`.  Returns torch
    CPU tensors in `dtype` (B as [K, N], or [N, K] for b_layout "NK")."""
    import torch

    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dtype]
    g = torch.Generator().manual_seed(seed)
    bshape = (K, N) if b_layout == "KN" else (N, K)
    if dist == "uniform":
        a = torch.rand((M, K), generator=g, dtype=torch.float32) * 2 - 1
        b = torch.rand(bshape, generator=g, dtype=torch.float32) * 2 - 1
    elif dist == "normal":
        a = torch.randn((M, K), generator=g, dtype=torch.float32) * scale
        b = torch.randn(bshape, generator=g, dtype=torch.float32) * scale
    else:
        raise ValueError(dist)
    return a.to(tdt), b.to(tdt)


def to_f64(t) -> np.ndarray:
    """A torch tensor of any of the three dtypes as exact float64 values."""
    import torch

    return t.detach().to("cpu", torch.float64).numpy()


def reference_check(out, a, b, dtype: str, bias=None, layout: str = "KN") -> float:
    """Relative Frobenius error of a GEMM result against the float64 oracle."""
    af, bf = to_f64(a), to_f64(b)
    if layout == "NK":
        bf = bf.T
    ref = matmul_f64(af, bf)
    if bias is not None:
        ref = ref + to_f64(bias)[None, :]
    return rel_frobenius(to_f64(out), ref)


def cpu_matmul(a, b):
    """The reference CPU path that BASELINE.json names: the same op via
    torch.matmul on CPU tensors in the operands' dtype (timed as the CPU
    baseline; never used by the product)."""
    import torch

    return torch.matmul(a, b)
