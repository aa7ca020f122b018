"""Pins the CPU oracle (oracle/gemm_oracle.py, oracle/gemm_ref.c) against
exactly rounded golden values, brute force, closed forms and invariants, and
shows that plausible mistakes in it would be caught."""
import math

import numpy as np
import pytest
import torch

from oracle import gemm_oracle as O

GOLDEN_CASES = ["f16_3x5x7_kn", "f16_17x9x33_kn", "bf16_17x9x33_kn", "bf16_6x40x72_nk_bias",
                "f16_4x24x16_nk_bias", "f32_5x3x65_kn", "f32_2x3x1_kn", "f32_33x31x129_kn"]


def decode(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "fp32":
        return bits.view(np.float32).astype(np.float64)
    if dtype == "fp16":
        return bits.view(np.float16).astype(np.float64)
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def golden_operands(golden, name):
    dt = {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}[name.split("_")[0]]
    a = decode(golden[name + "/a"], dt)
    b = decode(golden[name + "/b"], dt)
    bias = decode(golden[name + "/bias"], dt) if name + "/bias" in golden else None
    return dt, a, b, bias


def oracle_for(name, a, b, bias, matmul=O.matmul_f64):
    if "_nk" in name:
        out = O.linear_f64(a, b.reshape(-1, a.shape[1]), bias) if bias is not None else matmul(a, b.T)
    else:
        out = matmul(a, b)
    return out


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_oracle_matches_exactly_rounded_golden(golden, name):
    dt, a, b, bias = golden_operands(golden, name)
    exp = golden[name + "/expected"]
    M, N = exp.shape
    a = a.reshape(M, -1)
    b = b.reshape(-1, N) if "_kn" in name else b.reshape(N, -1)
    out = oracle_for(name, a, b, bias)
    # BLAS float64 vs correctly rounded sums: a few ulps of the largest term
    scale = np.abs(a) @ np.abs(b if "_kn" in name else b.T) + (np.abs(bias) if bias is not None else 0)
    assert np.all(np.abs(out - exp) <= 1e-14 * scale + 1e-300)


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_c_bruteforce_matches_golden(golden, oracle_c, name):
    dt, a, b, bias = golden_operands(golden, name)
    exp = golden[name + "/expected"]
    M, N = exp.shape
    K = a.size // M
    a = np.ascontiguousarray(a.reshape(M, K))
    layout = 0 if "_kn" in name else 1
    b = np.ascontiguousarray(b.reshape((K, N) if layout == 0 else (N, K)))
    c = np.zeros((M, N))
    oracle_c.oracle_gemm_f64(layout, a.ctypes.data, K, b.ctypes.data, b.shape[1], c.ctypes.data, N, M, N, K)
    if bias is not None:
        c = c + bias[None, :]
    scale = np.abs(a) @ np.abs(b if layout == 0 else b.T) + (np.abs(bias) if bias is not None else 0)
    assert np.all(np.abs(c - exp) <= 1e-14 * scale + 1e-300)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 17, 65), (17, 3, 129), (65, 129, 3), (129, 65, 17)])
@pytest.mark.parametrize("layout", [0, 1])
def test_numpy_oracle_matches_c_bruteforce(oracle_c, M, N, K, layout):
    rng = np.random.default_rng(M * 1000 + N * 10 + K + layout)
    a = rng.standard_normal((M, K))
    b = rng.standard_normal((K, N) if layout == 0 else (N, K))
    c = np.zeros((M, N))
    oracle_c.oracle_gemm_f64(layout, a.ctypes.data, K, b.ctypes.data, b.shape[1], c.ctypes.data, N, M, N, K)
    ref = O.matmul_f64(a, b if layout == 0 else b.T)
    np.testing.assert_allclose(ref, c, rtol=1e-12, atol=1e-12 * K)


def test_closed_forms():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((7, 5))
    assert np.array_equal(O.matmul_f64(a, np.eye(5)), a)           # identity
    perm = np.eye(5)[[3, 0, 4, 1, 2]]
    assert np.array_equal(O.matmul_f64(a, perm), a[:, [1, 3, 4, 0, 2]])  # permutation of columns
    assert not O.matmul_f64(a, np.zeros((5, 4))).any()             # zero
    u = rng.integers(-8, 8, size=(6, 1)).astype(float)
    v = rng.integers(-8, 8, size=(1, 9)).astype(float)
    assert np.array_equal(O.matmul_f64(u, v), u * v)               # K = 1 / rank-1 outer product
    ai = rng.integers(-3, 4, size=(12, 40)).astype(float)
    bi = rng.integers(-3, 4, size=(40, 10)).astype(float)
    exact = np.array([[sum(int(ai[m, k]) * int(bi[k, n]) for k in range(40)) for n in range(10)]
                      for m in range(12)], dtype=float)
    assert np.array_equal(O.matmul_f64(ai, bi), exact)              # small integers are exact
    assert O.matmul_f64(np.zeros((3, 0)), np.zeros((0, 4))).shape == (3, 4)  # K = 0 -> zeros


def test_invariants():
    rng = np.random.default_rng(1)
    a, b = rng.standard_normal((9, 13)), rng.standard_normal((13, 6))
    a2 = rng.standard_normal((9, 13))
    np.testing.assert_allclose(O.matmul_f64(a, b).T, O.matmul_f64(b.T, a.T), rtol=1e-13)
    np.testing.assert_allclose(O.matmul_f64(2 * a + a2, b), 2 * O.matmul_f64(a, b) + O.matmul_f64(a2, b),
                               rtol=1e-12, atol=1e-12)
    x = rng.standard_normal((2, 3, 13))
    w = rng.standard_normal((6, 13))
    bias = rng.standard_normal(6)
    lin = O.linear_f64(x, w, bias)
    assert lin.shape == (2, 3, 6)
    np.testing.assert_allclose(lin.reshape(6, 6), x.reshape(6, 13) @ w.T + bias, rtol=1e-13)
    bb = rng.standard_normal((4, 13, 5))
    aa = rng.standard_normal((4, 9, 13))
    out = O.bmm_f64(aa, bb)
    for i in range(4):
        np.testing.assert_array_equal(out[i], O.matmul_f64(aa[i], bb[i]))


def test_round_fp16_all_bit_patterns(oracle_c):
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = pats.view(np.float16).astype(np.float64)
    dec = np.array([oracle_c.oracle_f16_bits_to_f64(int(p)) for p in pats])
    finite = np.isfinite(vals)
    assert np.array_equal(vals[finite], dec[finite])
    assert np.array_equal(np.isnan(vals), np.isnan(dec))
    # round_fp16 is idempotent on every representable value
    assert np.array_equal(O.round_fp16(vals[finite]), vals[finite])


def test_round_fp16_ties_and_overflow():
    # 1 + 2^-11 is a tie between 1 and 1 + 2^-10: nearest even is 1
    assert O.round_fp16(np.array([1 + 2.0 ** -11]))[0] == 1.0
    assert O.round_fp16(np.array([1 + 3 * 2.0 ** -11]))[0] == 1 + 2 * 2.0 ** -10
    assert O.round_fp16(np.array([65520.0]))[0] == np.inf   # halfway to 2^16 rounds up to inf
    assert O.round_fp16(np.array([65519.0]))[0] == 65504.0


def test_round_bf16_matches_c_and_torch(oracle_c):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4000),
                        np.array([0.0, -0.0, 1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 3.3895314e38, np.inf, -np.inf],
                                 dtype=np.float32)]).astype(np.float32)
    ours = O.round_bf16(x)
    c_bits = np.array([oracle_c.oracle_f32_to_bf16_bits(float(v)) for v in x], dtype=np.uint16)
    c_vals = np.array([oracle_c.oracle_bf16_bits_to_f64(int(bb)) for bb in c_bits])
    assert np.array_equal(ours, c_vals)
    t = torch.from_numpy(x).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.array_equal(ours, t)
    assert O.round_bf16(np.array([1 + 2 ** -8], dtype=np.float32))[0] == 1.0       # tie -> even
    assert O.round_bf16(np.array([1 + 3 * 2 ** -8], dtype=np.float32))[0] == 1 + 2 ** -6
    assert np.isnan(O.round_bf16(np.array([np.nan], dtype=np.float32))[0])


def test_rel_frobenius():
    ref = np.array([[3.0, 4.0]])
    assert O.rel_frobenius(ref, ref) == 0.0
    assert math.isclose(O.rel_frobenius(ref * 1.001, ref), 1e-3, rel_tol=1e-9)
    assert O.rel_frobenius(np.array([[0.0, 1e-3]]), np.array([[0.0, 0.0]])) == float("inf")
    assert O.rel_frobenius(np.zeros((2, 2)), np.zeros((2, 2))) == 0.0


def test_seeded_inputs_fingerprint(golden):
    """The benchmark input generator is pinned: first elements and sums of A and B."""
    for cname in ["cfg1_fp32_512", "cfg4_fp16_skinny"]:
        c = O.CONFIGS[cname]
        a, b = O.make_inputs(c["dtype"], c["M"], c["N"], c["K"], c["dist"], c.get("scale", 1.0), 0)
        ab = a.reshape(-1)[:8].contiguous()
        bb = b.reshape(-1)[:8].contiguous()
        view = torch.int32 if c["dtype"] == "fp32" else torch.int16
        npdt = np.uint32 if c["dtype"] == "fp32" else np.uint16
        assert np.array_equal(ab.view(view).numpy().view(npdt), golden[cname + "/a_head"])
        assert np.array_equal(bb.view(view).numpy().view(npdt), golden[cname + "/b_head"])
        np.testing.assert_allclose([O.to_f64(a).sum(), O.to_f64(b).sum()], golden[cname + "/sums"], rtol=1e-12)
    a, b = O.make_inputs("fp16", 4, 5, 6, "normal", 1.0, 0)
    assert a.dtype == torch.float16 and a.shape == (4, 6) and b.shape == (6, 5)
    a2, b2 = O.make_inputs("fp16", 4, 5, 6, "normal", 1.0, 0)
    assert torch.equal(a, a2) and torch.equal(b, b2)


# ---- planted mistakes: each mutated oracle must fail the golden check ----

def _dropped_last_term(a, b):
    return O.matmul_f64(a[:, :-1], b[:-1, :])


def _transposed_operand(a, b):
    if b.shape[0] == b.shape[1]:
        return O.matmul_f64(a, b.T)
    return O.matmul_f64(a, b[::-1])


def _sign_error(a, b):
    out = O.matmul_f64(a, b)
    out[-1, -1] = -out[-1, -1]
    return out


def _index_shift(a, b):
    return O.matmul_f64(a, np.roll(b, 1, axis=1))


@pytest.mark.parametrize("mutant", [_dropped_last_term, _transposed_operand, _sign_error, _index_shift])
def test_planted_mistakes_are_caught(golden, mutant):
    name = "f16_17x9x33_kn"
    dt, a, b, bias = golden_operands(golden, name)
    exp = golden[name + "/expected"]
    M, N = exp.shape
    a, b = a.reshape(M, -1), b.reshape(-1, N)
    out = mutant(a, b)
    assert out.shape != exp.shape or O.rel_frobenius(out, exp) > O.TOLERANCE["fp16"]


def test_cfg1_cpu_reference_path_within_fp32_bound():
    """Config 1 of the benchmark contract: the reference CPU path (torch.matmul
    on CPU) on the seeded 512^3 fp32 inputs, against the float64 oracle."""
    c = O.CONFIGS["cfg1_fp32_512"]
    a, b = O.make_inputs(c["dtype"], c["M"], c["N"], c["K"], c["dist"], c.get("scale", 1.0), 0)
    out = O.cpu_matmul(a, b)
    assert out.dtype == torch.float32 and out.shape == (512, 512)
    err = O.reference_check(out, a, b, "fp32")
    assert 0.0 < err <= O.TOLERANCE["fp32"]
    # A planted mistake (operand transposed) is far outside the bound.
    assert O.reference_check(O.cpu_matmul(a, b.T.contiguous()), a, b, "fp32") > 0.5


# ---- conv2d 1x1 (the reference runs it through linear, src/main.cpp:402-424) ----

CONV_CASES = ["conv_f16_2x5x3x4_o6_bias", "conv_bf16_3x24x2x5_o7", "conv_f32_1x9x4x4_o3_bias"]


def conv_operands(golden, name):
    dt = {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}[name.split("_")[1]]
    exp = golden[name + "/expected"]
    B, O_, H, W = exp.shape
    x = decode(golden[name + "/x"], dt).reshape(B, -1, H, W)
    w = decode(golden[name + "/w"], dt).reshape(O_, -1, 1, 1)
    bias = decode(golden[name + "/bias"], dt) if name + "/bias" in golden else None
    return x, w, bias, exp


@pytest.mark.parametrize("name", CONV_CASES)
def test_conv_oracle_matches_exactly_rounded_golden(golden, name):
    x, w, bias, exp = conv_operands(golden, name)
    out = O.conv2d_1x1_f64(x, w, bias)
    assert out.shape == exp.shape
    scale = np.einsum("bchw,oc->bohw", np.abs(x), np.abs(w[:, :, 0, 0])) + \
        (np.abs(bias)[None, :, None, None] if bias is not None else 0)
    assert np.all(np.abs(out - exp) <= 1e-14 * scale + 1e-300)


@pytest.mark.parametrize("B,C,H,W,Co", [(1, 1, 1, 1, 1), (2, 3, 5, 7, 4), (3, 16, 4, 1, 9), (1, 0, 2, 2, 3)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv_oracle_matches_torch_conv2d_and_per_image_matmul(B, C, H, W, Co, with_bias):
    rng = np.random.default_rng(B * 1000 + C * 100 + H * 10 + W + Co)
    x = rng.standard_normal((B, C, H, W))
    w = rng.standard_normal((Co, C, 1, 1))
    bias = rng.standard_normal(Co) if with_bias else None
    out = O.conv2d_1x1_f64(x, w, bias)
    if C > 0:   # (torch returns no output channels at all for C_in = 0; the empty sum is 0 + bias)
        ref = torch.nn.functional.conv2d(torch.from_numpy(x), torch.from_numpy(w),
                                         None if bias is None else torch.from_numpy(bias)).numpy()
        np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12 * max(C, 1))
    else:
        np.testing.assert_array_equal(out, np.zeros((B, Co, H, W)) + (0 if bias is None else bias[None, :, None, None]))
    for b in range(B):   # each image is the GEMM W[Co, C] @ X_b[C, H*W] (+ bias per row)
        mm = O.matmul_f64(w[:, :, 0, 0], x[b].reshape(C, H * W))
        if bias is not None:
            mm = mm + bias[:, None]
        np.testing.assert_allclose(out[b].reshape(Co, H * W), mm, rtol=1e-12, atol=1e-12 * max(C, 1))


def _conv_wrong_permute(x, w, bias):   # NHWC built as N,W,H,C and not undone
    out = O.linear_f64(np.transpose(x, (0, 3, 2, 1)), w[:, :, 0, 0], bias)
    return np.transpose(out, (0, 3, 1, 2))


def _conv_bias_per_column(x, w, bias):  # bias indexed by pixel instead of channel
    out = O.conv2d_1x1_f64(x, w, None)
    flat = out.reshape(out.shape[0], out.shape[1], -1)
    n = flat.shape[2]
    flat = flat + np.resize(bias, n)[None, None, :]
    return flat.reshape(out.shape)


def _conv_dropped_channel(x, w, bias):
    return O.conv2d_1x1_f64(x[:, 1:], w[:, 1:], bias)


@pytest.mark.parametrize("mutant", [_conv_wrong_permute, _conv_bias_per_column, _conv_dropped_channel])
def test_conv_planted_mistakes_are_caught(golden, mutant):
    x, w, bias, exp = conv_operands(golden, "conv_f16_2x5x3x4_o6_bias")
    out = mutant(x, w, bias)
    assert out.shape != exp.shape or O.rel_frobenius(out, exp) > O.TOLERANCE["fp16"]


# ---- the seeded input generator against the distributions BASELINE.json names ----

def _sample(t, n=200_000):
    """Up to n values of a tensor as float64 (a fixed stride through it)."""
    v = O.to_f64(t).reshape(-1)
    return v[:: max(1, v.size // n)][:n]


def distribution_ok(t, dist, scale=1.0, alpha=1e-4):
    """True when the values of t look like iid draws of the named distribution:
    Kolmogorov-Smirnov against scipy's CDF, plus range (uniform), mean and spread
    within a few standard errors of the distribution's own."""
    from scipy import stats

    v = _sample(t)
    n = v.size
    if dist == "uniform":
        if v.min() < -1.0 or v.max() > 1.0:
            return False
        sd = math.sqrt(1.0 / 3.0)
        if stats.kstest(v, "uniform", args=(-1.0, 2.0)).pvalue < alpha:
            return False
    else:
        sd = scale
        if stats.kstest(v, "norm", args=(0.0, scale)).pvalue < alpha:
            return False
    if abs(v.mean()) > 5 * sd / math.sqrt(n):
        return False
    # the sample variance of n iid draws has a relative standard error of about sqrt(2/n)
    # (normal; smaller for uniform)
    return abs(v.var() / sd ** 2 - 1.0) < 6 * math.sqrt(2.0 / n)


def independent(a, b):
    """A and B are distinct draws: not equal and uncorrelated (|r| < 5 / sqrt(n))."""
    x, y = _sample(a), _sample(b)
    n = min(x.size, y.size)
    x, y = x[:n], y[:n]
    if np.array_equal(x, y):
        return False
    return abs(np.corrcoef(x, y)[0, 1]) < 5 / math.sqrt(n)


@pytest.mark.parametrize("cname", sorted(O.CONFIGS))
def test_make_inputs_follows_the_config_distributions(cname):
    c = O.CONFIGS[cname]
    # the full shapes, but small M keeps it quick: B is drawn whole
    M = min(c["M"], 64)
    a, b = O.make_inputs(c["dtype"], M, c["N"], c["K"], c["dist"], c.get("scale", 1.0), 0)
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[c["dtype"]]
    assert a.dtype == tdt and b.dtype == tdt and a.shape == (M, c["K"]) and b.shape == (c["K"], c["N"])
    assert distribution_ok(a, c["dist"], c.get("scale", 1.0)), cname
    assert distribution_ok(b, c["dist"], c.get("scale", 1.0)), cname
    assert independent(a, b)


def test_make_inputs_scales_are_the_configs():
    # N(0,1)/sqrt(4096), N(0,0.02), N(0,1)/sqrt(8192), U[-1,1] for fp32
    assert O.CONFIGS["cfg2_fp16_4096"]["scale"] == 1 / 64
    assert O.CONFIGS["cfg3_bf16_mlp"]["scale"] == 0.02
    assert math.isclose(O.CONFIGS["cfg4_fp16_skinny"]["scale"], 1 / math.sqrt(8192), rel_tol=1e-15)
    assert O.CONFIGS["cfg1_fp32_512"]["dist"] == O.CONFIGS["cfg5_fp32_ragged"]["dist"] == "uniform"


def test_make_inputs_draw_order_and_seeding():
    # A is drawn first: it does not depend on N (nor on B's layout); B continues the same
    # stream, so it moves with the size of A; another seed moves both; same seed, same bits
    a1, b1 = O.make_inputs("fp32", 8, 40, 16, "uniform", 1.0, 3)
    a2, b2 = O.make_inputs("fp32", 8, 24, 16, "uniform", 1.0, 3)
    a3, b3 = O.make_inputs("fp32", 9, 40, 16, "uniform", 1.0, 3)
    a4, b4 = O.make_inputs("fp32", 8, 40, 16, "uniform", 1.0, 4)
    a5, b5 = O.make_inputs("fp32", 8, 40, 16, "uniform", 1.0, 3, b_layout="NK")
    assert torch.equal(a1, a2) and torch.equal(a1, a5) and torch.equal(a1, a3[:8])
    # B starts where A ends in the stream, whatever N is: the smaller B is a prefix
    assert torch.equal(b1.reshape(-1)[:16 * 24], b2.reshape(-1))
    assert not torch.equal(b1, b3) and not torch.equal(a1, a4) and not torch.equal(b1, b4)
    assert b5.shape == (40, 16) and torch.equal(b5.reshape(-1), b1.reshape(-1))
    a6, b6 = O.make_inputs("fp32", 8, 40, 16, "uniform", 1.0, 3)
    assert torch.equal(a1, a6) and torch.equal(b1, b6)
    # values are representable in the dtype (cast once, no further rounding)
    a7, b7 = O.make_inputs("fp16", 64, 64, 64, "normal", 0.1, 0)
    assert np.array_equal(O.round_fp16(O.to_f64(a7)), O.to_f64(a7))
    a8, _ = O.make_inputs("bf16", 64, 64, 64, "normal", 0.1, 0)
    assert np.array_equal(O.round_bf16(O.to_f64(a8)), O.to_f64(a8))


def _mutant_inputs(kind, M, N, K, dist, scale, seed):
    """make_inputs with one plausible mistake (for the planted-mistake check)."""
    g = torch.Generator().manual_seed(seed)
    if kind == "rand_for_randn":
        return torch.rand((M, K), generator=g) * scale, torch.rand((K, N), generator=g) * scale
    if kind == "wrong_scale":
        return torch.randn((M, K), generator=g) * scale * 1.25, torch.randn((K, N), generator=g) * scale * 1.25
    if kind == "unit_range":
        return torch.rand((M, K), generator=g), torch.rand((K, N), generator=g)
    if kind == "half_range":
        return torch.rand((M, K), generator=g) - 0.5, torch.rand((K, N), generator=g) - 0.5
    if kind == "b_equals_a":
        a = torch.randn((M, K), generator=g) * scale
        return a, a.clone().reshape(K, N)
    raise ValueError(kind)


@pytest.mark.parametrize("kind,dist", [("rand_for_randn", "normal"), ("wrong_scale", "normal"),
                                       ("unit_range", "uniform"), ("half_range", "uniform"),
                                       ("b_equals_a", "normal")])
def test_make_inputs_checks_catch_planted_mistakes(kind, dist):
    a, b = _mutant_inputs(kind, 256, 256, 256, dist, 0.02, 0)
    ok = distribution_ok(a, dist, 0.02) and distribution_ok(b, dist, 0.02) and independent(a, b)
    assert not ok, kind
