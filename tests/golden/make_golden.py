"""Write tests/golden/gemm_golden.npz: small GEMM cases with exactly rounded
expected outputs, plus fingerprints of the seeded benchmark inputs.

Expected values are computed element by element as math.fsum of the exact
float64 products of the dtype-rounded inputs (a product of two fp16, bf16 or
fp32 values is exact in float64), i.e. the correctly rounded float64 value of
the true sum -- independently of numpy/BLAS and of the oracle module's
matmul.  Inputs come from oracle.gemm_oracle.make_inputs (seeded CPU torch
generator, A drawn before B), and are stored as raw bit patterns.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.gemm_oracle import CONFIGS, make_inputs, to_f64  # noqa: E402

# name: (dtype, M, N, K, layout, with_bias, dist, scale, seed)
CASES = {
    "f16_3x5x7_kn": ("fp16", 3, 5, 7, "KN", False, "normal", 1.0, 11),
    "f16_17x9x33_kn": ("fp16", 17, 9, 33, "KN", False, "normal", 0.25, 12),
    "bf16_17x9x33_kn": ("bf16", 17, 9, 33, "KN", False, "normal", 0.25, 13),
    "bf16_6x40x72_nk_bias": ("bf16", 6, 40, 72, "NK", True, "uniform", 1.0, 14),
    "f16_4x24x16_nk_bias": ("fp16", 4, 24, 16, "NK", True, "uniform", 1.0, 15),
    "f32_5x3x65_kn": ("fp32", 5, 3, 65, "KN", False, "uniform", 1.0, 16),
    "f32_2x3x1_kn": ("fp32", 2, 3, 1, "KN", False, "uniform", 1.0, 17),
    "f32_33x31x129_kn": ("fp32", 33, 31, 129, "KN", False, "uniform", 1.0, 18),
}


# 1x1 convolutions: name: (dtype, batch, c_in, H, W, c_out, with_bias, seed)
CONV_CASES = {
    "conv_f16_2x5x3x4_o6_bias": ("fp16", 2, 5, 3, 4, 6, True, 21),
    "conv_bf16_3x24x2x5_o7": ("bf16", 3, 24, 2, 5, 7, False, 22),
    "conv_f32_1x9x4x4_o3_bias": ("fp32", 1, 9, 4, 4, 3, True, 23),
}


def bits(t) -> np.ndarray:
    import torch

    if t.dtype == torch.float32:
        return t.contiguous().view(torch.int32).numpy().view(np.uint32).copy()
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def exact_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    M, K = a.shape
    N = b.shape[1]
    out = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            out[m, n] = math.fsum(float(a[m, k]) * float(b[k, n]) for k in range(K))
    return out


def main() -> None:
    import torch

    data = {}
    for name, (dt, M, N, K, lay, with_bias, dist, scale, seed) in CASES.items():
        a, b = make_inputs(dt, M, N, K, dist, scale, seed, b_layout=lay)
        af, bf = to_f64(a), to_f64(b)
        bkn = bf if lay == "KN" else bf.T
        exp = exact_matmul(af, bkn)
        if with_bias:
            g = torch.Generator().manual_seed(seed + 1000)
            bias = (torch.rand((N,), generator=g) * 2 - 1).to(a.dtype)
            data[name + "/bias"] = bits(bias)
            bb = to_f64(bias)
            exp = np.array([[math.fsum([exp[m, n], bb[n]]) for n in range(N)] for m in range(M)])
        data[name + "/a"] = bits(a)
        data[name + "/b"] = bits(b)
        data[name + "/expected"] = exp
    for name, (dt, B, C, H, W, O, with_bias, seed) in CONV_CASES.items():
        tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dt]
        g = torch.Generator().manual_seed(seed)
        x = (torch.rand((B, C, H, W), generator=g) * 2 - 1).to(tdt)
        w = (torch.rand((O, C, 1, 1), generator=g) * 2 - 1).to(tdt)
        bias = (torch.rand((O,), generator=g) * 2 - 1).to(tdt) if with_bias else None
        xf, wf = to_f64(x), to_f64(w)
        bf = to_f64(bias) if with_bias else np.zeros(O)
        exp = np.zeros((B, O, H, W))
        for b_ in range(B):
            for o in range(O):
                for h in range(H):
                    for w_ in range(W):
                        terms = [float(xf[b_, c, h, w_]) * float(wf[o, c, 0, 0]) for c in range(C)]
                        exp[b_, o, h, w_] = math.fsum(terms + ([float(bf[o])] if with_bias else []))
        data[name + "/x"] = bits(x)
        data[name + "/w"] = bits(w)
        if with_bias:
            data[name + "/bias"] = bits(bias)
        data[name + "/expected"] = exp
    # fingerprints of the benchmark inputs (seed 0): first 8 elements of A and
    # of B, and float64 sums of each, as produced by the seeded generator
    for cname, c in CONFIGS.items():
        a, b = make_inputs(c["dtype"], c["M"], c["N"], c["K"], c["dist"], c.get("scale", 1.0), 0)
        data[cname + "/a_head"] = bits(a.reshape(-1)[:8])
        data[cname + "/b_head"] = bits(b.reshape(-1)[:8])
        data[cname + "/sums"] = np.array([to_f64(a).sum(), to_f64(b).sum()])
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_golden.npz")
    np.savez_compressed(out, **data)
    print(f"wrote {out} ({os.path.getsize(out)} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
