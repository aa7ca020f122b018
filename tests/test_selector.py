"""Host-side kernel selection and argument validation (no GPU needed)."""
import pytest

from cmp_ext_amd import cabi

K_TILE256, K_TILE224, K_TILE128, K_SKINNY, K_F32_128, K_F32_64, K_GENERIC, K_SKINNY_WIDE, K_F32_96, K_TILE64, \
    K_SKINNY_NK, K_F32_64K4, K_F32_16K4, K_STREAM, K_STREAM128, K_TALL = range(16)


@pytest.mark.parametrize("dtype,M,N,K,expect", [
    (cabi.F32, 512, 512, 512, K_F32_64K4),        # cfg1: 64 tiles of 64x64, K split over each one's waves
    (cabi.F32, 3000, 2000, 1000, K_F32_64),       # 1504 tiles of 64x64: ~6 per CU
    (cabi.F16, 4096, 4096, 4096, K_TILE256),      # cfg2: 256 tiles = one per CU
    (cabi.BF16, 4096, 14336, 4096, K_TILE224),    # cfg3: 1024 tiles = 4 full waves
    (cabi.F16, 16, 8192, 8192, K_SKINNY),         # cfg4
    (cabi.F32, 4097, 3001, 2049, K_F32_96),       # cfg5: 2021 tiles of 96x64 (<= 8 per CU)
    (cabi.F32, 4096, 4096, 4096, K_F32_128),
    (cabi.F32, 1440, 768, 200, K_F32_96),
    (cabi.F16, 1024, 1024, 1024, K_TILE128),      # small: more tiles wanted
    (cabi.BF16, 64, 4096, 4096, K_SKINNY),
    (cabi.BF16, 65, 4096, 4096, K_TILE128),
    (cabi.F16, 16, 32768, 4096, K_TILE128),       # M <= 64 but 256 column tiles: tiled beats skinny
    (cabi.F16, 64, 32768, 128, K_TILE128),
    (cabi.F16, 64, 65536, 512, K_TILE64),         # ... and with short K and 256 tiles of 256 columns
    (cabi.BF16, 32, 131072, 256, K_TILE64),
])
def test_config_kernel_choice(dtype, M, N, K, expect):
    kid, desc = cabi.plan(dtype, cabi.B_KN, M, N, K)
    assert kid == expect, desc


def test_skinny_wide_needs_workspace():
    need = cabi.workspace_size(cabi.F16, cabi.B_KN, 16, 8192, 8192)
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 16, 8192, 8192, workspace_bytes=need)
    assert kid == K_SKINNY_WIDE and "splits=4" in desc and "ksplit=2048" in desc and "grid=1x256x1" in desc
    kid, _ = cabi.plan(cabi.F16, cabi.B_KN, 16, 8192, 8192, workspace_bytes=need - 1)
    assert kid == K_SKINNY                      # too little workspace: narrow strips, no split
    kid, desc = cabi.plan(cabi.BF16, cabi.B_KN, 16, 25600, 4096)
    assert kid == K_SKINNY_WIDE and "splits=1" in desc   # 200 strips: no split, no workspace
    kid, _ = cabi.plan(cabi.F16, cabi.B_KN, 17, 200, 72, workspace_bytes=1 << 30)
    assert kid == K_SKINNY                      # tiny grid either way: narrow has more workgroups


def test_skinny_m_batches_with_many_tiles_go_tiled():
    # a product of 64 rows with 64 x 128 column tiles of 128: tiled (cabi.plan gives the
    # batch entries their own A, so the streaming kernel, which shares one A, is out)
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 64, 16384, 128, batch=64)
    assert kid == K_TILE64, desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 64, 16384, 128, batch=1)
    assert kid in (K_SKINNY, K_SKINNY_WIDE), desc       # 128 tiles alone would leave CUs idle


def _prepared_kernel(dtype, M, N, K, batch, stride_a, flags=0, bias=None, lda=None, ldc=None, align=0,
                     workspace_limit=0, layout=cabi.B_KN):
    """Kernel id and description the C ABI plans for these pointers and pitches (no GPU:
    prepare only; by default without a workspace; B packed, as [K, N] or [N, K])."""
    lda = lda or K
    ldc = ldc or N
    ldb = N if layout == cabi.B_KN else K
    a, b, c = 0x100000 + align, 0x40000000, 0x80000000
    st, call = cabi.prepare(dtype, layout, a, lda, stride_a, b, ldb, K * N, c, ldc, M * ldc, bias, M, N, K,
                            batch, flags, workspace_limit)
    assert st == cabi.OK
    return cabi.describe(call)


def test_stream_kernel_for_convolution_shapes():
    # a 1x1 convolution over 64 images of 128x128 pixels (the weight shared: stride_a 0,
    # bias per output channel): 8192 column tiles of 128, 32 per CU
    kid, desc = _prepared_kernel(cabi.F16, 64, 16384, 128, 64, 0, cabi.BIAS_PER_ROW, bias=0x1000)
    assert kid == K_STREAM and "tile=64x128" in desc, desc
    assert _prepared_kernel(cabi.BF16, 40, 16384, 72, 32, 0)[0] == K_STREAM      # 4096 tiles, ragged M, K
    assert _prepared_kernel(cabi.F16, 1, 524288, 8, 1, 0)[0] == K_STREAM
    assert _prepared_kernel(cabi.F16, 64, 8200, 128, 64, 0)[0] == K_STREAM       # 65 tiles per image
    # K up to 256 (two chunks of 128 k per tile), up to 64 rows or 65..128
    assert _prepared_kernel(cabi.F16, 64, 16384, 136, 64, 0)[0] == K_STREAM
    assert _prepared_kernel(cabi.BF16, 64, 16384, 256, 32, 0, cabi.BIAS_PER_ROW, bias=0x1000)[0] == K_STREAM
    assert _prepared_kernel(cabi.F16, 65, 16384, 136, 64, 0)[0] == K_STREAM128
    assert _prepared_kernel(cabi.BF16, 128, 16384, 256, 32, 0, cabi.BIAS_PER_ROW, bias=0x1000)[0] == K_STREAM128
    # not the streaming kernel: too few tiles per CU, K above 256, M above 2048, one A per
    # batch entry, a bias per column, a misaligned A, or rows of C not 16-byte multiples
    assert _prepared_kernel(cabi.F16, 64, 16384, 128, 31, 0)[0] != K_STREAM
    assert _prepared_kernel(cabi.F16, 64, 16384, 264, 64, 0)[0] != K_STREAM
    assert _prepared_kernel(cabi.F16, 128, 16384, 264, 64, 0)[0] not in (K_STREAM, K_STREAM128)
    kid, desc = _prepared_kernel(cabi.F16, 65, 16384, 128, 64, 0)
    assert kid == K_STREAM128 and "tile=128x128" in desc, desc   # 65..128 rows: 128-row tiles
    assert _prepared_kernel(cabi.BF16, 128, 16384, 128, 64, 0, cabi.BIAS_PER_ROW, bias=0x1000)[0] == K_STREAM128
    # B as [N, K] (NHWC images: pixels x input channels), the same rules
    kid, desc = _prepared_kernel(cabi.F16, 64, 16384, 128, 64, 0, cabi.BIAS_PER_ROW, bias=0x1000, layout=cabi.B_NK)
    assert kid == K_STREAM and "layout=NK" in desc, desc
    assert _prepared_kernel(cabi.BF16, 200, 16384, 256, 32, 0, layout=cabi.B_NK)[0] == K_STREAM128
    assert _prepared_kernel(cabi.F16, 64, 16384, 264, 64, 0, layout=cabi.B_NK)[0] != K_STREAM
    # more than 128 rows: row blocks of 128, up to 2048 rows; the grid counts column tiles
    # only (the kernel walks its row blocks itself): 128 tiles x 1 x 32 images
    assert _prepared_kernel(cabi.F16, 129, 16384, 128, 64, 0)[0] == K_STREAM128
    kid, desc = _prepared_kernel(cabi.F16, 256, 16384, 64, 32, 0)
    assert kid == K_STREAM128 and "grid=1x128x32 " in desc and "threads=512" in desc, desc
    assert _prepared_kernel(cabi.BF16, 512, 16384, 256, 32, 0, cabi.BIAS_PER_ROW, bias=0x1000)[0] == K_STREAM128
    assert _prepared_kernel(cabi.F16, 2048, 16384, 128, 8, 0)[0] == K_STREAM128
    assert _prepared_kernel(cabi.F16, 2049, 16384, 128, 8, 0)[0] not in (K_STREAM, K_STREAM128)
    # >= 16 tiles per workgroup counts the row blocks: 1024 rows x 2048 column tiles (8 x 2048
    # = 16384 block-tiles), but not 128 rows x 2048 column tiles
    assert _prepared_kernel(cabi.F16, 1024, 16384, 256, 16, 0)[0] == K_STREAM128
    assert _prepared_kernel(cabi.F16, 128, 16384, 256, 16, 0)[0] != K_STREAM128
    assert _prepared_kernel(cabi.F16, 64, 16384, 128, 64, 64 * 128)[0] != K_STREAM
    assert _prepared_kernel(cabi.F16, 64, 16384, 128, 64, 0, 0, bias=0x1000)[0] != K_STREAM
    assert _prepared_kernel(cabi.F16, 64, 16384, 128, 64, 0, align=8)[0] != K_STREAM
    kid, desc = _prepared_kernel(cabi.F16, 64, 16384, 128, 64, 0, align=8, workspace_limit=1 << 20)
    assert kid == K_STREAM and "padded=A" in desc, desc   # with a workspace: one aligned copy of A
    assert _prepared_kernel(cabi.F16, 64, 16380, 128, 64, 0, ldc=16380)[0] != K_STREAM
    assert _prepared_kernel(cabi.F32, 64, 16384, 128, 64, 0)[0] != K_STREAM
    assert _prepared_kernel(cabi.F16, 64, 4194296, 128, 256, 0)[0] == K_STREAM
    assert _prepared_kernel(cabi.F16, 64, 4194296, 128, 70000, 0)[0] != K_STREAM   # > 2^31 tiles


def test_skinny_linear_weight_layout():
    # decode-shaped Linear (W is [N, K]): strips of W rows over all of K, no workspace;
    # 16-row strips until 32-row ones give every CU one
    assert cabi.workspace_size(cabi.F16, cabi.B_NK, 16, 4096, 14336) == 0
    kid, desc = cabi.plan(cabi.F16, cabi.B_NK, 16, 4096, 14336, workspace_bytes=1 << 30)
    assert kid == K_SKINNY_NK and "tile=16x16" in desc and "grid=1x256x1" in desc, desc
    kid, desc = cabi.plan(cabi.BF16, cabi.B_NK, 16, 14336, 4096)
    assert kid == K_SKINNY_NK and "tile=16x32" in desc and "mb=1" in desc, desc
    # more than 16 rows of A: 64-row strips while they still give >= 192 workgroups
    kid, desc = cabi.plan(cabi.BF16, cabi.B_NK, 64, 14336, 4096)
    assert kid == K_SKINNY_NK and "tile=64x64" in desc and "mb=4" in desc and "grid=1x224x1" in desc, desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_NK, 32, 8192, 8192)
    assert kid == K_SKINNY_NK and "tile=32x32" in desc, desc      # 128 strips of 64: too few


def test_unaligned_16bit_operands_padded_in_the_workspace():
    # odd K / odd N: with a workspace the planner copies A and/or B, zero-padded to
    # 16-byte rows, and runs a tiled kernel; without one the generic kernel runs
    for M, N, K, layout, pads in [(4095, 4095, 4095, cabi.B_KN, "AB"), (4096, 4095, 4096, cabi.B_KN, "B"),
                                  (4096, 4096, 4095, cabi.B_NK, "AB"), (2047, 2049, 2051, cabi.B_KN, "AB")]:
        need = cabi.workspace_size(cabi.F16, layout, M, N, K)
        kp = (K + 7) // 8 * 8
        a_bytes = M * kp * 2 if "A" in pads else 0
        b_bytes = (kp * ((N + 7) // 8 * 8) if layout == cabi.B_KN else N * kp) * 2 if "B" in pads else 0
        assert need == sum((x + 255) // 256 * 256 for x in (a_bytes, b_bytes)), (M, N, K, need)
        kid, desc = cabi.plan(cabi.F16, layout, M, N, K, workspace_bytes=need)
        assert kid in (K_TILE256, K_TILE224, K_TILE128) and f"padded={pads} kp={kp}" in desc, desc
        kid, desc = cabi.plan(cabi.F16, layout, M, N, K, workspace_bytes=need - 1)
        assert kid == K_GENERIC, desc
    # a misaligned view (offset by one element) is copied even when the shape is aligned
    kid, desc = cabi.plan(cabi.BF16, cabi.B_KN, 2048, 2048, 2048, lda=2049, workspace_bytes=1 << 30)
    assert kid != K_GENERIC and "padded=A " in desc, desc
    # small products stay on the generic kernel (two copies would cost more than they save)
    kid, _ = cabi.plan(cabi.F16, cabi.B_KN, 129, 257, 65, workspace_bytes=1 << 30)
    assert kid == K_GENERIC


def test_split_k_tiles():
    need = cabi.workspace_size(cabi.F16, cabi.B_KN, 256, 4096, 14336)
    assert need == 8 * 256 * 4096 * 4
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 256, 4096, 14336, workspace_bytes=need)
    assert kid == K_TILE128 and "splits=8 ksplit=1792" in desc, desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 256, 4096, 14336)      # no workspace: one pass
    assert kid != K_TILE128 or "splits" not in desc, desc
    kid, desc = cabi.plan(cabi.BF16, cabi.B_NK, 200, 1000, 3000, has_bias=True, workspace_bytes=1 << 30)
    assert kid == K_TILE128 and "splits=5 ksplit=640" in desc, desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 1024, 1024, 1024, workspace_bytes=1 << 30)
    assert "splits" not in desc, desc                              # short K: no split
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 4096, 4096, 4096, workspace_bytes=1 << 30)
    assert kid == K_TILE256, desc                                  # enough tiles: no split


def test_skinny_parameters():
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 16, 8192, 8192)
    assert kid == K_SKINNY
    assert "mb=1" in desc and "grid=1x256x1" in desc and "threads=256" in desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_KN, 33, 104, 72)
    assert kid == K_SKINNY and "mb=3" in desc and "grid=1x4x1" in desc


@pytest.mark.parametrize("M,N,K,layout,align,expect", [
    (300, 7, 64, cabi.B_KN, 16, K_GENERIC),     # N % 8 != 0 with KN layout
    (300, 12, 64, cabi.B_NK, 16, K_TILE128),    # NK layout needs only N % 4 (8-byte C rows)
    (300, 7, 64, cabi.B_NK, 16, K_TILE128),     # any C pitch: stores narrow to 8 or 2 bytes
    (300, 64, 33, cabi.B_KN, 16, K_GENERIC),    # K % 8 != 0
    (300, 64, 64, cabi.B_KN, 8, K_GENERIC),     # misaligned operand
    (16, 63, 64, cabi.B_KN, 16, K_GENERIC),     # skinny needs N % 8 == 0
    (16, 100, 64, cabi.B_KN, 16, K_GENERIC),
    (16, 64, 60, cabi.B_KN, 16, K_GENERIC),     # skinny needs K % 8 == 0
    (16, 64, 64, cabi.B_NK, 16, K_SKINNY_NK),   # [N,K] B (Linear weight): strips of W rows
])
def test_alignment_fallbacks(M, N, K, layout, align, expect):
    kid, desc = cabi.plan(cabi.F16, layout, M, N, K, align=align)
    assert kid == expect, desc


def test_fp32_any_alignment():
    kid, _ = cabi.plan(cabi.F32, cabi.B_KN, 4097, 3001, 2049, align=4)
    assert kid in (K_F32_64, K_F32_96, K_F32_128)


@pytest.mark.parametrize("args,err", [
    (dict(dtype=7), cabi.ERR_UNSUPPORTED),
    (dict(layout=2), cabi.ERR_UNSUPPORTED),
    (dict(M=-1), cabi.ERR_INVALID_ARG),
    (dict(K=-5), cabi.ERR_INVALID_ARG),
    (dict(lda=3), cabi.ERR_INVALID_ARG),          # lda < K
    (dict(ldb=3), cabi.ERR_INVALID_ARG),          # ldb < N
    (dict(ldc=3), cabi.ERR_INVALID_ARG),          # ldc < N
    (dict(lda=1 << 30), cabi.ERR_TOO_LARGE),      # 256 rows no longer fit 32-bit offsets
])
def test_validation_errors(args, err):
    base = dict(dtype=cabi.F16, layout=cabi.B_KN, M=64, N=64, K=64)
    base.update(args)
    kw = {k: base[k] for k in ("lda", "ldb", "ldc") if k in base}
    kid, _ = cabi.plan(base["dtype"], base["layout"], base["M"], base["N"], base["K"], **kw)
    assert kid == err
    assert cabi.status_string(err) not in ("success", "unknown status")


def test_zero_sizes_are_valid():
    for M, N, K in [(0, 5, 5), (5, 0, 5), (5, 5, 0)]:
        kid, _ = cabi.plan(cabi.F16, cabi.B_KN, M, N, K)
        assert kid >= 0


@pytest.mark.parametrize("layout,M,N,K,batch,expect,strip", [
    (cabi.B_KN, 2048, 64, 2048, 8, K_TALL, 64),       # attention's P V: 128 tiles of 128 rows, 256 strips of 64
    (cabi.B_NK, 2048, 64, 2048, 1, K_TALL, 32),       # 16 tiles: 64 strips of 32 rows
    (cabi.B_NK, 16384, 16, 4096, 1, K_TALL, 64),      # a LoRA down-projection / router, K = 4096
    (cabi.B_KN, 16384, 64, 1024, 1, K_TALL, 32),      # K < 2048: 32-row strips, two per CU
    (cabi.B_KN, 4096, 64, 4096, 1, K_TILE128, 0),     # K = 4096 below 8192 rows: the split tile
    (cabi.B_NK, 4096, 16, 4096, 1, K_TALL, 32),       # ... unless B is [N, K] with <= 32 rows
    (cabi.B_NK, 4096, 48, 4096, 1, K_TILE128, 0),
    (cabi.B_NK, 16384, 64, 8192, 1, K_TILE128, 0),    # K = 8192: the split tile
    (cabi.B_KN, 32768, 64, 1024, 1, K_TILE128, 0),    # 256 tiles already fill the GPU
    (cabi.B_KN, 1024, 64, 1024, 32, K_TILE128, 0),    # ... over a batch
    (cabi.B_KN, 2048, 128, 2048, 8, K_TILE128, 0),    # 128 columns: measured slower
    (cabi.B_KN, 2048, 60, 2048, 1, K_GENERIC, 0),     # [K, N] rows not in 16-byte chunks (no workspace)
    (cabi.B_NK, 2048, 60, 2048, 1, K_TALL, 32),       # ... which B as [N, K] does not need
])
def test_tall_kernel_for_narrow_b(layout, M, N, K, batch, expect, strip):
    kid, desc = cabi.plan(cabi.F16, layout, M, N, K, batch=batch, workspace_bytes=0 if expect == K_GENERIC else 1 << 40)
    assert kid == expect, desc
    if expect == K_TALL:
        # 16-row blocks of B's columns: 4 for [K, N] (64-column LDS rows); as needed for [N, K]
        mb = 4 if layout == cabi.B_KN or N > 32 else (1 if N <= 16 else 2)
        assert f"tile={strip}x{16 * mb} " in desc and f"mb={mb}" in desc, desc
        assert f"grid={-(-M // strip)}x1x{batch}" in desc, desc


def test_tall_split_k_rule():
    """Narrow B, few 32-row strips of A and K >= 8192: the tall kernel with K split so that
    ~256 workgroups run (8 ways over 32 strips, 4 over 64), with the workspace only."""
    ws = 1 << 40
    for lay, M, N, K, B, expect in [(cabi.B_NK, 1024, 16, 14336, 1, 8), (cabi.B_KN, 2048, 64, 8192, 1, 4),
                                    (cabi.B_KN, 1024, 64, 8192, 2, 4), (cabi.B_NK, 1024, 8, 8192, 1, 8)]:
        kid, desc = cabi.plan(cabi.F16, lay, M, N, K, batch=B, workspace_bytes=ws)
        assert kid == K_TALL and "tile=32x" in desc and f"splits={expect} " in desc, desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_NK, 4096, 16, 14336, workspace_bytes=ws)
    assert kid == K_TILE128, desc                       # 128 strips: the split tile
    kid, desc = cabi.plan(cabi.F16, cabi.B_NK, 1024, 16, 14336)
    assert kid == K_TALL and "splits" not in desc, desc  # no workspace: unsplit strips


def test_skinny_nk_split_k_rule():
    """skinny_nk splits K when its strips leave half the CUs or more idle and each
    workgroup would stream >= 700 KB (W rows + A's 16-row blocks over K), into ~256
    workgroups (2..8 ways), and only with the workspace for the partials."""
    ws = 1 << 40
    for M, N, K, expect in [(1, 1024, 14336, 4), (16, 512, 14336, 8), (64, 1024, 8192, 4), (64, 2048, 14336, 2),
                            (32, 512, 8192, 8), (64, 1024, 4096, 1),
                            (16, 1024, 8192, 1), (64, 1024, 2048, 1), (1, 4096, 14336, 1), (64, 14336, 4096, 1)]:
        kid, desc = cabi.plan(cabi.F16, cabi.B_NK, M, N, K, workspace_bytes=ws)
        assert kid == K_SKINNY_NK, desc
        assert (f"splits={expect} " in desc) if expect > 1 else ("splits" not in desc), (M, N, K, desc)
    kid, desc = cabi.plan(cabi.F16, cabi.B_NK, 1, 1024, 14336)
    assert kid == K_SKINNY_NK and "splits" not in desc, desc
    # more than 16 rows of A and K >= 10240 over <= 128 strips of 64 W rows: those strips, split
    for M, N, K, expect in [(64, 4096, 14336, 4), (32, 4096, 14336, 4), (64, 8192, 14336, 2), (48, 4096, 10240, 4)]:
        kid, desc = cabi.plan(cabi.F16, cabi.B_NK, M, N, K, workspace_bytes=ws)
        assert kid == K_SKINNY_NK and f"x64 " in desc and f"splits={expect} " in desc, (M, N, K, desc)
    for M, N, K in [(64, 4096, 4096), (16, 4096, 14336), (64, 14336, 8192), (64, 4096, 8192)]:
        kid, desc = cabi.plan(cabi.F16, cabi.B_NK, M, N, K, workspace_bytes=ws)
        assert kid == K_SKINNY_NK and "splits" not in desc, (M, N, K, desc)


def test_gemm_config_override(monkeypatch):
    """CMPEXT3_GEMM_CONFIG forces a kernel (and a K split) where that kernel's requirements
    hold for the call, and is ignored otherwise."""
    ws = 1 << 40
    base = cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2048, workspace_bytes=ws)[1]
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tile256x256,splits=2")
    desc = cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2048, workspace_bytes=ws)[1]
    assert desc.startswith("kernel=tile256x256") and "splits=2 ksplit=1024" in desc, desc
    # the split needs the workspace for its fp32 partials: without it, the tile alone
    desc = cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2048)[1]
    assert desc.startswith("kernel=tile256x256") and "splits" not in desc, desc
    # misaligned rows without a workspace: no tiled kernel can run them, so the override is
    # ignored (generic); with one, the padded copies run the forced tile
    assert cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2047)[1].startswith("kernel=generic64x64")
    desc = cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2047, workspace_bytes=ws)[1]
    assert desc.startswith("kernel=tile256x256") and "padded=AB" in desc, desc
    # the streaming kernel on a product it can take, however few its tiles (B as [K, N] or
    # [N, K]); not with a bias per column or K above 256
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=stream64x128")
    desc = cabi.plan(cabi.F16, cabi.B_KN, 200, 1000, 96)[1]
    assert desc.startswith("kernel=stream128x128") and "grid=1x8x1" in desc, desc
    assert not cabi.plan(cabi.F16, cabi.B_KN, 200, 1000, 96, has_bias=True)[1].startswith("kernel=stream")
    assert cabi.plan(cabi.F16, cabi.B_NK, 200, 1000, 96)[1].startswith("kernel=stream128x128")
    assert not cabi.plan(cabi.F16, cabi.B_KN, 200, 1000, 264)[1].startswith("kernel=stream")
    # the tall kernel (N <= 128; 16-row blocks of B's columns: 4 up to 64, else 8; for B as
    # [N, K] 1 up to 16 columns, 2 up to 32), with the
    # strip height asked for; not for wider B or [K, N] rows not in 16-byte chunks
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tall,strip=32")
    desc = cabi.plan(cabi.BF16, cabi.B_KN, 1000, 72, 200, batch=3)[1]
    assert desc.startswith("kernel=tall") and "tile=32x128 grid=32x1x3" in desc and "mb=8" in desc, desc
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tall")
    desc = cabi.plan(cabi.F16, cabi.B_NK, 100, 20, 40)[1]
    assert desc.startswith("kernel=tall") and "tile=64x32 grid=2x1x1" in desc and "mb=2" in desc, desc
    desc = cabi.plan(cabi.F16, cabi.B_KN, 100, 16, 40)[1]
    assert desc.startswith("kernel=tall") and "tile=64x64 grid=2x1x1" in desc and "mb=4" in desc, desc
    assert not cabi.plan(cabi.F16, cabi.B_KN, 1000, 136, 200)[1].startswith("kernel=tall")
    assert not cabi.plan(cabi.F16, cabi.B_KN, 1000, 60, 200)[1].startswith("kernel=tall")
    # 16-row strips exist for skinny_nk only: a tall override asking for them is ignored
    # (the selector's own plan), never run as another strip height
    monkeypatch.delenv("CMPEXT3_GEMM_CONFIG")
    own = cabi.plan(cabi.BF16, cabi.B_KN, 1000, 72, 200, batch=3)[1]
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tall,strip=16")
    assert cabi.plan(cabi.BF16, cabi.B_KN, 1000, 72, 200, batch=3)[1] == own
    # the generic kernel, with no padded copies in its place
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=generic64x64")
    desc = cabi.plan(cabi.BF16, cabi.B_KN, 2048, 2048, 2047, workspace_bytes=ws)[1]
    assert desc.startswith("kernel=generic64x64") and "padded" not in desc, desc
    # fp32 tiles, split
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=f32tile64x64 splits=4")
    desc = cabi.plan(cabi.F32, cabi.B_KN, 512, 512, 4096, workspace_bytes=ws)[1]
    assert desc.startswith("kernel=f32tile64x64 ") and "splits=4 ksplit=1024" in desc, desc
    # an fp32 name on a 16-bit call, an unknown name, a malformed split: ignored
    assert cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2048, workspace_bytes=ws)[1] == base
    for bad in ("kernel=tile999", "kernel=", "splits=2", "kernel=tile128x128,splits=zero"):
        monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", bad)
        desc = cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2048, workspace_bytes=ws)[1]
        assert desc == base or (bad.startswith("kernel=tile128x128") and "splits" not in desc), (bad, desc)
    monkeypatch.delenv("CMPEXT3_GEMM_CONFIG")
    assert cabi.plan(cabi.F16, cabi.B_KN, 2048, 2048, 2048, workspace_bytes=ws)[1] == base


def test_row_split_of_mostly_empty_last_rounds():
    # 4100 rows: whole 256x256 rounds for 4096 rows (one round), the 4 left over on the
    # skinny kernel (split K with a workspace, narrow strips without)
    kid, desc = cabi.plan(cabi.BF16, cabi.B_KN, 4100, 4096, 4096, workspace_bytes=1 << 30)
    assert kid == K_TILE256 and "grid=16x16x1" in desc and " rows=4096 | rows 4096..4099: kernel=skinny_wide" in desc
    kid, desc = cabi.plan(cabi.BF16, cabi.B_KN, 4100, 4096, 4096)
    assert kid == K_TILE256 and " rows=4096 | rows 4096..4099: kernel=skinny " in desc, desc
    kid, desc = cabi.plan(cabi.F16, cabi.B_NK, 4100, 4096, 4096, has_bias=True, workspace_bytes=1 << 30)
    assert " rows=4096 | rows 4096..4099: kernel=skinny_nk" in desc, desc
    kid, desc = cabi.plan(cabi.BF16, cabi.B_NK, 5000, 4096, 4096, workspace_bytes=1 << 30)
    assert " rows=4096 | rows 4096..4999: kernel=tile128x128" in desc, desc
    # the workspace the call asks for is the larger of the two launches' (they share it)
    assert cabi.workspace_size(cabi.BF16, cabi.B_KN, 4100, 4096, 4096) == 8 * 4 * 4096 * 4
    # whole rounds, a last round more than half full, or fp32: one launch
    for dtype, M, N, K in [(cabi.F16, 4096, 4096, 4096), (cabi.F16, 2100, 4096, 4096),
                           (cabi.BF16, 1030, 14336, 4096), (cabi.F32, 4100, 4096, 4096), (cabi.F16, 4100, 64, 4096)]:
        _, desc = cabi.plan(dtype, cabi.B_KN, M, N, K, workspace_bytes=1 << 30)
        assert " rows=" not in desc, desc


def test_row_split_not_under_override(monkeypatch):
    monkeypatch.setenv("CMPEXT3_GEMM_CONFIG", "kernel=tile128x128")
    kid, desc = cabi.plan(cabi.BF16, cabi.B_KN, 4100, 4096, 4096, workspace_bytes=1 << 30)
    assert kid == K_TILE128 and " rows=" not in desc, desc


def test_row_split_plans_cover_the_rows():
    # random 16-bit shapes: where the plan splits the rows, the first launch covers a
    # multiple of 256 rows short of M, the second the rest, and the workspace the call asks
    # for is what both launches need (the larger of the two)
    import numpy as np

    rng = np.random.default_rng(3)
    splits = 0
    for _ in range(400):
        dtype = [cabi.F16, cabi.BF16][rng.integers(2)]
        layout = [cabi.B_KN, cabi.B_NK][rng.integers(2)]
        M, N, K = int(rng.integers(1, 9000)), int(rng.integers(1, 1025)) * 8, int(rng.integers(1, 513)) * 8
        batch = int(rng.choice([1, 2, 3]))
        ws = int(rng.choice([0, 1 << 40]))
        kid, desc = cabi.plan(dtype, layout, M, N, K, batch=batch, workspace_bytes=ws)
        assert kid >= 0, desc
        if " rows=" not in desc:
            continue
        splits += 1
        m_main = int(desc.split(" rows=")[1].split()[0])
        assert 0 < m_main < M and m_main % 256 == 0, desc
        assert f" | rows {m_main}..{M - 1}: kernel=" in desc, desc
        head, tail = desc.split(" rows=")[0], desc.split(": ", 1)[1]
        _, head_alone = cabi.plan(dtype, layout, m_main, N, K, batch=batch, workspace_bytes=ws)
        _, tail_alone = cabi.plan(dtype, layout, M - m_main, N, K, batch=batch, workspace_bytes=ws)
        assert head == head_alone and tail == tail_alone, (desc, head_alone, tail_alone)
        if ws == 0:
            assert "workspace=" not in desc, desc
    assert splits >= 10
