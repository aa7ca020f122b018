"""Host-side half of the random C-ABI sweep (the GPU half is test_gpu_sweep.py).

cmpext3_gemm_prepare validates the arguments and picks the kernels without
touching a GPU, so every sweep case can be prepared here with host addresses of
the same alignment: each must be accepted, and together they must reach most
kernel families.  The sweep's check() is itself checked against the float64
oracle: an exact emulation of a correct call passes it, and the same output
with one element written into C's row padding, or one result element changed,
fails it.
"""
import numpy as np
import pytest
import torch

from cmp_ext_amd import cabi
from sweep_cases import CASES, CODE, DT, N_TALL, check, describe_case, logical, make_buffers, output_mask, reference

BASE = 1 << 32  # a 4 KiB-aligned host address standing in for each buffer
ESZ = {"fp16": 2, "bf16": 2, "fp32": 4}


def _prepare_on_host(c):
    e = ESZ[c["dtype"]]
    bias = None if c["bias"] is None else BASE * 4 + c["off_bias"] * e
    return cabi.prepare(CODE[c["dtype"]], c["layout"], BASE + c["off_a"] * e, c["lda"], c["stride_a"],
                        BASE * 2 + c["off_b"] * e, c["ldb"], c["stride_b"], BASE * 3 + c["off_c"] * e, c["ldc"],
                        c["stride_c"], bias, c["M"], c["N"], c["K"], c["batch"],
                        cabi.BIAS_PER_ROW if c["bias"] == "row" else 0, (1 << 63) - 1 if c["workspace"] else 0)


def test_every_sweep_case_is_accepted_and_the_families_are_reached():
    kernels = {}
    for c in CASES:
        st, call = _prepare_on_host(c)
        assert st == cabi.OK, f"{describe_case(c)}: {cabi.status_string(st)}"
        ws = cabi.call_workspace_size(call)
        assert ws >= 0 and (c["workspace"] or ws == 0), describe_case(c)
        k = cabi.describe(call)[1].split()[0].split("=")[1]
        kernels[k] = kernels.get(k, 0) + 1
        if c["idx"] >= len(CASES) - N_TALL:
            assert k == "tall", describe_case(c)
    assert len(kernels) >= 13, kernels


def _emulated(c, a, b, bias, cbuf):
    """The output of a correct call: the oracle's result rounded to the dtype, written
    into the logical region of every batch entry (everything else left as it was)."""
    out = cbuf.clone()
    for e in range(c["batch"]):
        r = torch.from_numpy(reference(c, a, b, bias, e)).to(DT[c["dtype"]])
        logical(out, c["off_c"], e, c["stride_c"], c["M"], c["ldc"], c["N"]).copy_(r)
    return out


SMALL = [c for c in CASES if c["sample"] is None and c["M"] * c["N"] * max(c["K"], 1) * c["batch"] < 2e7]


@pytest.mark.parametrize("c", SMALL[:24], ids=[f"c{c['idx']}" for c in SMALL[:24]])
def test_check_passes_a_correct_output_and_catches_planted_mistakes(c):
    a, b, bias, cbuf = make_buffers(c, torch.Generator().manual_seed(1000 + c["idx"]))
    out = _emulated(c, a, b, bias, cbuf)
    check(c, a, b, bias, out)
    # a result element changed (a zero result with K = 0 and no bias: any change is caught)
    bad = out.clone()
    bad[c["off_c"]] = bad[c["off_c"]].float() + 100.0
    with pytest.raises(AssertionError):
        check(c, a, b, bias, bad)
    # one element written outside the result: the first such element after C's start (row
    # padding, a gap between batch entries, or the tail), the buffer's last element, and the
    # element just before C's start when the buffer has room there
    outside = np.flatnonzero(~output_mask(c))
    planted = {int(outside[outside > c["off_c"]][0]), out.numel() - 1}
    if c["off_c"] > 0:
        planted.add(c["off_c"] - 1)
    for i in sorted(planted):
        bad = out.clone()
        bad[i] = 0.0
        with pytest.raises(AssertionError):
            check(c, a, b, bias, bad)
