"""Cases and checks of the random C-ABI sweep (test_gpu_sweep.py runs them on the GPU;
test_sweep_plan.py prepares every case on the host and checks the checks).

Nothing here touches a GPU: the cases are plain dicts drawn from a seeded RNG, the
buffers are CPU tensors, and check() compares a call's output (copied back to the
host) with the float64 oracle and the sentinel bits around it.
"""
import numpy as np
import torch

from cmp_ext_amd import cabi
from oracle import gemm_oracle as O

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
BITS = {"fp16": torch.int16, "bf16": torch.int16, "fp32": torch.int32}
CODE = {"fp16": cabi.F16, "bf16": cabi.BF16, "fp32": cabi.F32}
# a NaN bit pattern no kernel produces from finite inputs
SENTINEL = {"fp16": 0x7E5A, "bf16": 0x7FA5, "fp32": 0x7FC0BEEF}
TAIL = 64  # elements after every buffer's last logical element
N_CASES = 320
N_STREAM = 6
N_WIDE = 3
N_TALL = 6


def _round8(x):
    return (x + 7) // 8 * 8


def draw_case(rng: np.random.Generator, idx: int) -> dict:
    """One random case (plain ints; nothing here touches a GPU)."""
    dtype = ["fp16", "bf16", "fp32"][rng.choice(3, p=[0.4, 0.3, 0.3])]
    family = ["skinny", "tile", "big", "small"][rng.choice(4, p=[0.3, 0.3, 0.2, 0.2])]
    if family == "skinny":
        M, N, K = int(rng.integers(1, 65)), int(rng.integers(1, 3000)), int(rng.integers(1, 2500))
    elif family == "tile":
        M, N, K = int(rng.integers(65, 700)), int(rng.integers(1, 700)), int(rng.integers(1, 900))
    elif family == "big":
        M, N, K = int(rng.integers(700, 1400)), int(rng.integers(700, 1400)), int(rng.integers(32, 400))
    else:
        M, N, K = (int(x) for x in rng.integers(1, 40, size=3))
    # the fast paths need multiples of 8: most dimensions are rounded up
    M, N, K = (_round8(x) if rng.random() < 0.65 else x for x in (M, N, K))
    if rng.random() < 0.04:
        K = 0
    layout = [cabi.B_KN, cabi.B_NK][rng.integers(2)]
    pads = [0, 0, 0, 0, 8, 16, 1, 3, 13]
    lda = max(K + int(rng.choice(pads)), 1)
    ldb = max((N if layout == cabi.B_KN else K) + int(rng.choice(pads)), 1)
    ldc = max(N + int(rng.choice(pads)), 1)
    offs = [0, 0, 0, 0, 8, 1]
    off_a, off_b, off_c = (int(rng.choice(offs)) for _ in range(3))
    batch = int(rng.choice([1, 1, 2, 3]))
    gaps = [0, 0, 8, 5, 16]
    shared_a = batch > 1 and rng.random() < 0.3
    stride_a = 0 if shared_a else M * lda + int(rng.choice(gaps))
    rows_b = K if layout == cabi.B_KN else N
    stride_b = rows_b * ldb + int(rng.choice(gaps))
    stride_c = M * ldc + int(rng.choice(gaps))
    bias = [None, "col", "row"][rng.integers(3)]
    return dict(idx=idx, dtype=dtype, layout=layout, M=M, N=N, K=K, lda=lda, ldb=ldb, ldc=ldc, off_a=off_a,
                off_b=off_b, off_c=off_c, batch=batch, stride_a=stride_a, stride_b=stride_b, stride_c=stride_c,
                bias=bias, off_bias=int(rng.choice([0, 0, 1])), workspace=bool(rng.integers(2)), sample=None)


def draw_stream_case(rng: np.random.Generator, idx: int, wide_rows: bool) -> dict:
    """A 1x1-convolution-shaped case: one A for the batch, B as [K,N] (or [N,K] for every
    third case), >= 4096 column tiles (M of 65 to 320 if wide_rows)."""
    dtype = ["fp16", "bf16"][rng.integers(2)]
    M = int(rng.integers(65, 321)) if wide_rows else int(rng.integers(1, 65))
    K = int(rng.choice([8, 64, 72, 128, 136, 200, 256]))
    N = int(rng.choice([8192, 8200, 16384, 16376]))
    batch = -(-4096 // -(-N // 128))
    ldb = N + int(rng.choice([0, 8]))
    ldc = N + int(rng.choice([0, 8]))
    layout = cabi.B_NK if idx % 3 == 2 else cabi.B_KN  # every third as NHWC images: B given as [N, K]
    if layout == cabi.B_NK:
        ldb = K + int(rng.choice([0, 8]))
    rows_b = K if layout == cabi.B_KN else N
    return dict(idx=idx, dtype=dtype, layout=layout, M=M, N=N, K=K, lda=K + int(rng.choice([0, 8])), ldb=ldb,
                ldc=ldc, off_a=0, off_b=int(rng.choice([0, 8])), off_c=int(rng.choice([0, 8])), batch=batch,
                stride_a=0, stride_b=rows_b * ldb + int(rng.choice([0, 8])), stride_c=M * ldc + int(rng.choice([0, 8])),
                bias=["row", None][rng.integers(2)], off_bias=0, workspace=bool(rng.integers(2)),
                sample=sorted({0, batch // 2, batch - 1}))


def draw_wide_case(rng: np.random.Generator, idx: int) -> dict:
    """Few rows, many 256-column tiles over a batch with one A per entry (short K)."""
    dtype = ["fp16", "bf16"][rng.integers(2)]
    M, N, K = int(rng.integers(1, 65)), int(rng.choice([4096, 4104, 6144])), int(rng.choice([64, 200, 512]))
    batch = -(-256 // -(-N // 256))
    return dict(idx=idx, dtype=dtype, layout=cabi.B_KN, M=M, N=N, K=K, lda=K, ldb=N, ldc=N, off_a=0, off_b=0,
                off_c=0, batch=batch, stride_a=M * K, stride_b=K * N, stride_c=M * N,
                bias=["col", None][rng.integers(2)], off_bias=0, workspace=False,
                sample=sorted({0, batch // 2, batch - 1}))


def draw_tall_case(rng: np.random.Generator, idx: int) -> dict:
    """Many rows of A, a narrow B (<= 64 columns) and K of 1024 .. 2048: strips of A's rows
    (the tall kernel).  Padded pitches, offset bases and batch gaps in multiples of 8."""
    dtype = ["fp16", "bf16"][rng.integers(2)]
    layout = [cabi.B_KN, cabi.B_NK][rng.integers(2)]
    M = int(rng.integers(1024, 3001))
    N = int(rng.choice([8, 16, 40, 64])) if layout == cabi.B_KN else int(rng.integers(1, 65))
    K = int(rng.choice([1024, 1032, 1536, 2048]))
    batch = int(rng.choice([1, 2]))
    lda = K + int(rng.choice([0, 8]))
    ldb = (N if layout == cabi.B_KN else K) + int(rng.choice([0, 8]))
    ldc = N + int(rng.choice([0, 3, 8]))
    rows_b = K if layout == cabi.B_KN else N
    return dict(idx=idx, dtype=dtype, layout=layout, M=M, N=N, K=K, lda=lda, ldb=ldb, ldc=ldc,
                off_a=int(rng.choice([0, 8])), off_b=int(rng.choice([0, 8])), off_c=int(rng.choice([0, 1])),
                batch=batch, stride_a=M * lda + int(rng.choice([0, 8])), stride_b=rows_b * ldb + int(rng.choice([0, 8])),
                stride_c=M * ldc + int(rng.choice([0, 5])), bias=[None, "col", "row"][rng.integers(3)],
                off_bias=int(rng.choice([0, 1])), workspace=bool(rng.integers(2)), sample=None)


def cases():
    rng = np.random.default_rng(20261202)
    out = [draw_case(rng, i) for i in range(N_CASES)]
    out += [draw_stream_case(rng, N_CASES + i, i % 2 == 1) for i in range(N_STREAM)]
    out += [draw_wide_case(rng, N_CASES + N_STREAM + i) for i in range(N_WIDE)]
    out += [draw_tall_case(rng, N_CASES + N_STREAM + N_WIDE + i) for i in range(N_TALL)]
    return out


def extent(off, batch, stride, rows, ld, cols):
    """Number of elements a buffer needs: the last logical element + 1, plus TAIL."""
    if rows == 0 or cols == 0 or batch == 0:
        return off + TAIL
    return off + (batch - 1) * stride + (rows - 1) * ld + cols + TAIL


def logical(flat, off, b, stride, rows, ld, cols):
    """Batch entry b of a row-pitched matrix inside a flat CPU tensor."""
    return flat[off + b * stride:].as_strided((rows, cols), (ld, 1))


def output_mask(c):
    """Boolean mask of C's buffer: True where the call writes its result."""
    n = extent(c["off_c"], c["batch"], c["stride_c"], c["M"], c["ldc"], c["N"])
    mask = np.zeros(n, dtype=bool)
    rows = np.arange(c["M"])[:, None] * c["ldc"] + np.arange(c["N"])[None, :]
    for b in range(c["batch"]):
        mask[c["off_c"] + b * c["stride_c"] + rows] = True
    return mask


def make_buffers(c, gen: torch.Generator):
    """CPU buffers of the case: random A, B, bias (padding included), C all sentinel."""
    dt = DT[c["dtype"]]
    M, N, K, batch = c["M"], c["N"], c["K"], c["batch"]
    rows_b, cols_b = (K, N) if c["layout"] == cabi.B_KN else (N, K)
    na = extent(c["off_a"], batch if c["stride_a"] else 1, c["stride_a"], M, c["lda"], K)
    nb = extent(c["off_b"], batch, c["stride_b"], rows_b, c["ldb"], cols_b)
    a = (torch.randn(na, generator=gen) / max(K, 1) ** 0.5).to(dt)
    b = torch.randn(nb, generator=gen).to(dt)
    nbias = (N if c["bias"] == "col" else M) + c["off_bias"] + TAIL
    bias = torch.randn(nbias, generator=gen).to(dt) if c["bias"] else None
    cbuf = torch.full((extent(c["off_c"], batch, c["stride_c"], M, c["ldc"], N),), SENTINEL[c["dtype"]],
                      dtype=BITS[c["dtype"]]).view(dt)
    return a, b, bias, cbuf


def reference(c, a, b, bias, entry):
    """float64 oracle of batch entry `entry`."""
    M, N, K = c["M"], c["N"], c["K"]
    ae = O.to_f64(logical(a, c["off_a"], entry, c["stride_a"], M, c["lda"], K))
    if c["layout"] == cabi.B_KN:
        be = O.to_f64(logical(b, c["off_b"], entry, c["stride_b"], K, c["ldb"], N))
    else:
        be = O.to_f64(logical(b, c["off_b"], entry, c["stride_b"], N, c["ldb"], K)).T
    r = O.matmul_f64(ae, be)
    if bias is not None:
        bv = O.to_f64(bias[c["off_bias"]:c["off_bias"] + (N if c["bias"] == "col" else M)])
        r = r + (bv[None, :] if c["bias"] == "col" else bv[:, None])
    return r


def check(c, a, b, bias, cbuf_after):
    """Every check of one case on CPU tensors (the call's output copied back)."""
    M, N, K = c["M"], c["N"], c["K"]
    entries = c["sample"] if c["sample"] is not None else range(c["batch"])
    for e in entries:
        out = O.to_f64(logical(cbuf_after, c["off_c"], e, c["stride_c"], M, c["ldc"], N))
        ref = reference(c, a, b, bias, e)
        if K == 0 and bias is None:
            assert np.array_equal(out, ref), f"case {c['idx']} entry {e}: K = 0 must give zeros"
        else:
            err = O.rel_frobenius(out, ref)
            assert err <= O.TOLERANCE[c["dtype"]], f"case {c['idx']} entry {e}: rel err {err:.3e}"
    bits = cbuf_after.view(BITS[c["dtype"]]).numpy()
    outside = ~output_mask(c)
    bad = np.flatnonzero(outside & (bits != np.array(SENTINEL[c["dtype"]]).astype(bits.dtype)))
    assert bad.size == 0, f"case {c['idx']}: {bad.size} elements outside C's result written (first at {bad[:4]})"


def describe_case(c):
    lay = "KN" if c["layout"] == cabi.B_KN else "NK"
    return (f"case {c['idx']} {c['dtype']} {lay} M={c['M']} N={c['N']} K={c['K']} batch={c['batch']} "
            f"ld=({c['lda']},{c['ldb']},{c['ldc']}) off=({c['off_a']},{c['off_b']},{c['off_c']}) "
            f"strides=({c['stride_a']},{c['stride_b']},{c['stride_c']}) bias={c['bias']}+{c['off_bias']} "
            f"ws={c['workspace']}")



CASES = cases()
