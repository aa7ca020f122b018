"""Host-side pieces of bench.py (no GPU): the timed operands are the ones the
oracle checks, and the CPU baseline's sample-size check."""
import torch

import bench
from oracle import gemm_oracle as O


def test_bench_inputs_are_the_oracle_inputs():
    # every config's A and first B, drawn as bench.py draws them (shapes scaled down by
    # keeping the config's dtype and distribution), equal the oracle's seeded inputs
    for name, c in bench.CONFIGS.items():
        small = dict(c, M=7, N=24, K=40)
        a, bs = bench.make_cpu_inputs(small, 3)
        ra, rb = O.make_inputs(c["dtype"], 7, 24, 40, c["dist"], c.get("scale", 1.0), 0)
        assert torch.equal(a, ra) and torch.equal(bs[0], rb), name
        assert len(bs) == 3 and not torch.equal(bs[1], bs[0]) and not torch.equal(bs[2], bs[1]), name
        assert a.dtype == bs[0].dtype == {"fp16": torch.float16, "bf16": torch.bfloat16,
                                          "fp32": torch.float32}[c["dtype"]]


def test_bench_callers_cover_the_reference_suites():
    # linear and bmm in the three dtypes of the reference harness, conv 1x1 in fp16
    ops = {(c["op"], c["dtype"]) for c in bench.CALLERS.values()}
    for op in ("linear", "bmm"):
        for dt in ("fp16", "bf16", "fp32"):
            assert (op, dt) in ops
    assert ("conv", "fp16") in ops
    assert set(bench.ORDER) == set(bench.CONFIGS) | set(bench.CALLERS)
    x, w, b = bench.caller_inputs(bench.CALLERS["linear_bf16_4096"])
    assert x.shape == (4096, 4096) and w.shape == (4096, 4096) and b.shape == (4096,)
    assert x.dtype == torch.bfloat16


def test_cpu_baseline_ratio_gate():
    # rates that agree give a value; rates that differ by more than 0.8..1.25 give none
    ok = bench.rate_summary({8: (8.0, 1.0, 3), 16: (16.0, 2.1, 3)}, "TFLOP/s", "x")
    assert ok["value"] == round(16 / 2.1, 6) and 0.8 <= ok["rate_ratio_large_over_small"] <= 1.25
    bad = bench.rate_summary({8: (8.0, 1.0, 3), 16: (16.0, 8.0, 3)}, "TFLOP/s", "x")
    assert bad["value"] is None and "differ" in bad["null_reason"]
    whole = bench.rate_summary({16: (0.27, 5.0, 2)}, "GB/s", "x")
    assert whole["value"] == round(0.27 / 5.0, 6) and "rate_ratio_large_over_small" not in whole


def test_sample_rate_sizes():
    calls = []

    def run(n):
        calls.append(n)
        return float(n)

    r = bench.sample_rate(run, 64, 0.0, probe_s=10.0)  # never slow: doubles up to the limit
    assert sorted(r) == [32, 64]
    r = bench.sample_rate(run, 16, 0.0, whole=True)
    assert list(r) == [16] and r[16][2] >= 2


def test_cpu_conv_baseline_is_the_convolution():
    # the CPU baseline's per-image product is the 1x1 convolution (float32, so exact enough)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 8, 5, 7, generator=g)
    w = torch.randn(6, 8, 1, 1, generator=g)
    b = torch.randn(6, generator=g)
    ref = torch.nn.functional.conv2d(x, w, b)
    got = bench.conv1x1_cpu(x, w, b)
    assert got.shape == ref.shape and torch.allclose(got, ref, rtol=1e-5, atol=1e-5)
