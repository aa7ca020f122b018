"""Seeded random sweep of the C ABI's prepared calls (cmpext3_gemm_prepare / _run).

Each case draws a dtype, a B layout ([K,N] or [N,K]), M, N and K (ragged or
multiples of 8, K = 0 now and then), row pitches with padding, element offsets
of every base pointer (16-byte aligned or not), a batch with gaps between the
entries (A shared by every entry in some cases: stride_a = 0), no bias or a
bias per column or per row (aligned or not), and no workspace or as much as the
plan asks for.  Every case checks, against the float64 oracle:

  * the logical result of every batch entry (relative Frobenius bound of the
    operator contract: fp32 1e-5, fp16 2e-3, bf16 1e-2; exact zeros for K = 0
    without bias);
  * that every element of C's buffer outside the logical result (row padding,
    gaps between batch entries, the buffer's tail) still holds its sentinel
    bits, so no kernel, padded copy or reduction writes outside its region;
  * that A, B and the bias are unchanged.

A handful of larger cases have the 1x1-convolution shape (one A for the batch,
many 128-column tiles) that selects the streaming kernels, or few rows over
many 256-column tiles; for those the oracle checks three sampled batch entries
and the sentinel check covers all of C.
The kernel each case ran is collected, and the sweep must reach most kernel
families.
"""
import pytest
import torch

from cmp_ext_amd import cabi
from sweep_cases import BITS, CASES, CODE, check, describe_case, make_buffers

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def seen():
    return {"cases": 0, "kernels": {}}


@pytest.mark.parametrize("c", CASES, ids=[f"c{c['idx']}" for c in CASES])
def test_sweep_case(c, seen):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    gen = torch.Generator().manual_seed(1000 + c["idx"])
    a, b, bias, cbuf = make_buffers(c, gen)
    ag, bg, cg = a.cuda(), b.cuda(), cbuf.cuda()
    biasg = bias.cuda() if bias is not None else None
    M, N, K = c["M"], c["N"], c["K"]
    st, call = cabi.prepare(CODE[c["dtype"]], c["layout"], ag[c["off_a"]:], c["lda"], c["stride_a"],
                            bg[c["off_b"]:], c["ldb"], c["stride_b"], cg[c["off_c"]:], c["ldc"], c["stride_c"],
                            None if biasg is None else biasg[c["off_bias"]:],
                            M, N, K, c["batch"], cabi.BIAS_PER_ROW if c["bias"] == "row" else 0,
                            (1 << 63) - 1 if c["workspace"] else 0)
    assert st == cabi.OK, f"{describe_case(c)}: prepare -> {cabi.status_string(st)}"
    _, desc = cabi.describe(call)
    print(f"{describe_case(c)} -> {desc}", flush=True)
    ws_bytes = cabi.call_workspace_size(call)
    assert ws_bytes >= 0 and (c["workspace"] or ws_bytes == 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda") if ws_bytes > 0 else None
    assert cabi.run(call, ws) == cabi.OK
    torch.cuda.synchronize()
    check(c, a, b, bias, cg.cpu())
    assert torch.equal(ag.cpu().view(BITS[c["dtype"]]), a.view(BITS[c["dtype"]]))
    assert torch.equal(bg.cpu().view(BITS[c["dtype"]]), b.view(BITS[c["dtype"]]))
    if bias is not None:
        assert torch.equal(biasg.cpu().view(BITS[c["dtype"]]), bias.view(BITS[c["dtype"]]))
    kernel = desc.split()[0].split("=")[1]
    seen["kernels"][kernel] = seen["kernels"].get(kernel, 0) + 1
    seen["cases"] += 1


def test_sweep_reached_the_kernel_families(seen):
    if seen["cases"] < len(CASES):
        pytest.skip("needs every case of the sweep in the same session")
    print("kernels run by the sweep:", dict(sorted(seen["kernels"].items())), flush=True)
    assert len(seen["kernels"]) >= 10, seen["kernels"]
