"""GPU parity of the FP8 GEMMs against the oracle's dequantize-then-matmul
(float64). Bars: max-abs 2e-2 and rel-L2 1e-2 (north star); the blockwise
GEMM additionally meets the reference test's own bound, rel-L2 < 0.004
(tests/inference/test_pixelumm_decoder_optimizations.py:201-221)."""
import numpy as np
import pytest
import torch

from conftest import assert_close_bf16, bf16_bits, pkg_module, u8

pytestmark = pytest.mark.gpu


def _config1_inputs(M, K, N, seed=1234):
    """BASELINE config 1 generators: X ~ N(0,1) with 0.1% outliers x20,
    W ~ N(0, 0.02), bias ~ N(0, 0.01), one CPU generator per tensor. For
    K > 3072 the weight std shrinks by sqrt(3072 / K) so that |Y| stays below
    8, where bf16's half-ulp (<= 0.0156) fits the 2e-2 bar."""
    w_std = 0.02 * min(1.0, (3072 / K) ** 0.5)
    gx = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=gx)
    x = torch.where(torch.rand(M, K, generator=gx) < 0.001, x * 20, x).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=torch.Generator().manual_seed(seed + 1)) * w_std).to(torch.bfloat16)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(seed + 2)) * 0.01).to(torch.bfloat16)
    return x, w, b


def _check_linear(O, dev, M, K, N, gelu, bias=True, rows=None):
    ops = pkg_module("ops")
    x, w, b = _config1_inputs(M, K, N, seed=M + 7 * K + N)
    qw, sw = ops.quantize_rows_fp8(w.to(dev))
    y = ops.linear_fp8(x.to(dev), qw, sw, b.to(dev) if bias else None, 1 if gelu else 0)
    qx, sx = ops.quantize_rows_fp8(x.to(dev))
    qxo, sxo = O.quantize_rows_fp8(bf16_bits(x))
    qwo, swo = O.quantize_rows_fp8(bf16_bits(w))
    assert np.array_equal(u8(qx), qxo) and np.array_equal(u8(qw), qwo)
    assert np.array_equal(sx.cpu().numpy(), sxo) and np.array_equal(sw.cpu().numpy(), swo)
    sel = np.arange(M) if rows is None else rows
    ref = O.linear_reference(qxo[sel], sxo[sel], qwo, swo,
                             O.bf16_bits_to_f32(bf16_bits(b)) if bias else None, gelu=gelu)
    got = y.float().cpu().numpy()[sel]
    return assert_close_bf16(got, ref, what=f"linear {M}x{K}x{N} gelu={gelu}")


@pytest.mark.parametrize("M,K,N", [(1, 128, 128), (129, 256, 384), (300, 384, 256), (64, 12288, 3072),
                                   (1000, 256, 640), (2777, 384, 1152)])
@pytest.mark.parametrize("gelu", [False, True])
def test_linear_fp8_small_shapes(O, dev, M, K, N, gelu):
    print(f"case linear {M}x{K}x{N} gelu={gelu}", flush=True)
    _check_linear(O, dev, M, K, N, gelu)


def test_linear_fp8_config1_full(O, dev):
    """X [4096, 3072] x W [3072, 3072] + bias."""
    print("case linear config1", flush=True)
    _check_linear(O, dev, 4096, 3072, 3072, gelu=False)


def test_linear_fp8_north_star_sampled_rows(O, dev):
    """[10800 x 3072] x [3072 x 12288] with GELU; 600 rows checked (incl. the
    ragged last M tile)."""
    print("case linear north star", flush=True)
    rows = np.concatenate([np.arange(0, 200), np.arange(5300, 5500), np.arange(10600, 10800)])
    _check_linear(O, dev, 10800, 3072, 12288, gelu=True, rows=rows)


def test_linear_fp8_no_bias_and_strided_out(O, dev):
    ops = pkg_module("ops")
    _check_linear(O, dev, 200, 256, 128, gelu=False, bias=False)
    # row stride ldc > N through the C ABI
    L = pkg_module("_lib")
    a = torch.randint(0, 120, (70, 256), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    b = torch.randint(0, 120, (128, 256), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    sa = torch.rand(70, device=dev) + 0.5
    sb = torch.rand(128, device=dev) + 0.5
    out = torch.full((70, 136), 3.0, dtype=torch.bfloat16, device=dev)
    L.check(L.load().hn_gemm_fp8_rowcol(a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                                        None, out.data_ptr(), 70, 128, 256, 136, 0,
                                        torch.cuda.current_stream().cuda_stream), "gemm")
    ref = ops.gemm_fp8_rowcol(a, b, sa, sb)
    assert torch.equal(out[:, :128], ref)
    assert (out[:, 128:] == 3.0).all()


@pytest.mark.parametrize("M,K,N,act", [
    (100, 1024, 256, 1),    # 256 x 192 tiles; the wave of rows 0-127 has 100 rows (four row blocks)
    (1000, 1280, 640, 0),   # 256 x 192 tiles; the last tile's second row wave has 104 rows
    (4964, 1024, 4224, 1),  # 256-wide tiles (340); last row tile 100 deep
    (5092, 1024, 4224, 0),  # 256-wide tiles; last row tile 228 deep, its second row wave 100
])
def test_gemm_writes_nothing_past_m_or_n(dev, M, K, N, act):
    """The persistent GEMM into a buffer with 64 guard rows below M and 8
    guard columns right of N (row stride N + 8): the M x N block equals the
    plain call's output and the guards keep their fill. Shapes whose last
    row tile leaves a wave 97-127 rows: such a wave has four row blocks but
    is not wholly inside, and its tile-end stores must keep their bounds
    test (stores past row M faulted the GPU at M = 100 in a build that
    counted blocks)."""
    ops, L = pkg_module("ops"), pkg_module("_lib")
    print(f"case gemm guard band {M}x{K}x{N} act={act}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M + N)
    a = torch.randint(0, 120, (M, K), dtype=torch.uint8, device=dev, generator=g).view(torch.float8_e4m3fn)
    b = torch.randint(0, 120, (N, K), dtype=torch.uint8, device=dev, generator=g).view(torch.float8_e4m3fn)
    sa = torch.rand(M, device=dev, generator=g) * 1e-3 + 1e-4
    sb = torch.rand(N, device=dev, generator=g) * 1e-3 + 1e-4
    bias = torch.randn(N, device=dev, generator=g).to(torch.bfloat16)
    ldc = N + 8
    buf = torch.full((M + 64, ldc), 7.0, dtype=torch.bfloat16, device=dev)
    L.check(L.load().hn_gemm_fp8_rowcol(a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                                        bias.data_ptr(), buf.data_ptr(), M, N, K, ldc, act,
                                        torch.cuda.current_stream().cuda_stream), "gemm")
    ref = ops.gemm_fp8_rowcol(a, b, sa, sb, bias, act)
    assert torch.equal(buf[:M, :N], ref)
    assert bool((buf[M:] == 7.0).all()) and bool((buf[:, N:] == 7.0).all())


@pytest.mark.parametrize("M,N,K", [(300, 256, 512), (129, 384, 1024), (4097, 128, 4096)])
def test_blockwise_gemm_writes_nothing_past_m(dev, M, N, K):
    """The blockwise GEMM into a buffer 16 rows longer than its output: the
    output rows equal the op's own result and the guard rows keep their fill
    (last row tiles 44, 1 and 1 deep)."""
    print(f"case blockwise guard band {M}x{N}x{K}", flush=True)
    ops, L = pkg_module("ops"), pkg_module("_lib")
    pf = pkg_module("pixelumm_fp8")
    g = torch.Generator(device=dev).manual_seed(M)
    qa, sa = pf._quantize_blockwise(torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16))
    qb, sb = pf._quantize_blockwise(torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16))
    buf = torch.full((M + 16, N), 9.0, dtype=torch.bfloat16, device=dev)
    L.check(L.load().hn_gemm_fp8_blockwise(qa.data_ptr(), qb.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                                           buf.data_ptr(), M, N, K, torch.cuda.current_stream().cuda_stream),
            "blockwise")
    ref = ops.gemm_fp8_blockwise(qa, qb, sa, sb)
    assert torch.equal(buf[:M], ref) and bool((buf[M:] == 9.0).all())


# K >= 7 x 128 takes the persistent kernel that carries half of each tile's
# epilogue into the next tile's K loop. Cases: the smallest such K and the
# largest K below it; ragged M and N (edge tiles); more tiles than CUs, so a
# workgroup walks whole and edge tiles in turn; with and without bias / GELU.
# A launch with fewer 256-wide tiles than CUs runs 256 x 192 tiles when that
# gives more tiles and still one round (96 columns per wave): config 1 and
# (64, 12288, 3072) above, and the 1000 x 640 and 700 x 1280 cases here, whose
# last column stripes are 64 wide (one wave with two blocks, one with none) and
# 128 wide (three blocks and one).
@pytest.mark.parametrize("M,K,N,gelu,bias", [
    (300, 896, 384, True, True),      # smallest K on the carried-epilogue path
    (300, 768, 384, True, True),      # largest K below it
    (1000, 1280, 640, True, True),    # M and N edges, 256 x 192 tiles (16)
    (700, 1024, 1280, True, False),   # 256 x 192 tiles (21), both edges, no bias
    (4700, 1024, 4224, True, False),  # 323 tiles: two per workgroup, both edges, no bias
    (4700, 1024, 4224, False, True),
    # Last row tile 132 deep: waves of rows 0-127 multiply a whole block while
    # the stage rows they load (128-191) lie partly past M; the loads must
    # stay inside A. On 256 x 192 tiles, and on 256-wide ones (340 tiles).
    (132, 12288, 3072, True, True),
    (4996, 1024, 4224, False, True),
])
def test_linear_fp8_persistent_tiles(O, dev, M, K, N, gelu, bias):
    print(f"case linear persistent {M}x{K}x{N} gelu={gelu} bias={bias}", flush=True)
    rows = None if M <= 1000 else np.concatenate([np.arange(0, 64), np.arange(2300, 2364), np.arange(M - 300, M)])
    _check_linear(O, dev, M, K, N, gelu, bias=bias, rows=rows)


# A last row stripe of at most 64 rows (M % 256) goes to gemm_tail_kernel
# (K split over 4 waves when the stripe has fewer 32-column groups than CUs,
# else over 2; one or two 32-row blocks) while the persistent kernel tiles the
# rows above it; M <= 64 runs the tail kernel alone. Tails of 1, 20, 32, 33,
# 48 and 64 rows, with and without GELU and bias.
@pytest.mark.parametrize("M,K,N,gelu,bias", [
    (257, 1024, 384, True, True),      # 1 tail row: one block, 4 waves
    (288, 896, 640, False, True),      # 32 tail rows: one block
    (289, 3072, 512, True, False),     # 33 tail rows: two blocks, no bias
    (48, 3072, 1280, True, True),      # tail only (no persistent launch)
    (10800, 12288, 384, False, True),  # 48 tail rows, K 12288
    (1, 4224, 256, True, True),        # one row, K past 4096
    (276, 4224, 8192, False, True),    # 20 tail rows, 256 column groups: K split over 2 waves
    (576, 4352, 8192, True, True),     # 64 tail rows (two blocks), 2 waves, GELU
])
def test_linear_fp8_tail_rows(O, dev, M, K, N, gelu, bias):
    print(f"case linear tail {M}x{K}x{N} gelu={gelu} bias={bias}", flush=True)
    rows = None if M <= 1000 else np.concatenate([np.arange(0, 64), np.arange(M - 320, M)])
    _check_linear(O, dev, M, K, N, gelu, bias=bias, rows=rows)


# When every XCD has "light" workgroups (one full tile fewer) and the launch
# has no edge tiles, the persistent kernel's light workgroups compute the tail
# stripe themselves after their last tile (tail_wide: up to 384 columns each,
# the four waves sharing the stripe's A rows), instead of a second launch:
# the north-star shapes (M 10800) and these.
@pytest.mark.parametrize("M,K,N,gelu,bias", [
    (10785, 896, 4096, True, True),    # 33 tail rows (two blocks), 96 light workgroups of 64 columns
    (10770, 1024, 2048, False, False),  # 18 tail rows (one block)
])
def test_linear_fp8_tail_on_light_workgroups(O, dev, M, K, N, gelu, bias):
    print(f"case linear fused tail {M}x{K}x{N} gelu={gelu} bias={bias}", flush=True)
    rows = np.concatenate([np.arange(0, 64), np.arange(5000, 5064), np.arange(M - 320, M)])
    _check_linear(O, dev, M, K, N, gelu, bias=bias, rows=rows)


@pytest.mark.parametrize("M,K,N,act", [(300, 1024, 384, 1), (289, 4352, 256, 0), (33, 896, 128, 1),
                                       (10785, 896, 4096, 1), (276, 4224, 8192, 0)])
def test_gemm_tail_writes_nothing_past_m_or_n(dev, M, K, N, act):
    """Tail stripes (44, 33 and 33 rows; the last two on 8 and 4 waves) into a
    buffer with 64 guard rows and 8 guard columns (row stride N + 8): the
    M x N block equals the plain call's output, the guards keep their fill,
    and a second call gives the same bits (the wave-ordered split-K sum)."""
    ops, L = pkg_module("ops"), pkg_module("_lib")
    print(f"case gemm tail guard band {M}x{K}x{N} act={act}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M + K)
    a = torch.randint(0, 120, (M, K), dtype=torch.uint8, device=dev, generator=g).view(torch.float8_e4m3fn)
    b = torch.randint(0, 120, (N, K), dtype=torch.uint8, device=dev, generator=g).view(torch.float8_e4m3fn)
    sa = torch.rand(M, device=dev, generator=g) * 1e-3 + 1e-4
    sb = torch.rand(N, device=dev, generator=g) * 1e-3 + 1e-4
    bias = torch.randn(N, device=dev, generator=g).to(torch.bfloat16)
    ldc = N + 8
    buf = torch.full((M + 64, ldc), 7.0, dtype=torch.bfloat16, device=dev)
    L.check(L.load().hn_gemm_fp8_rowcol(a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                                        bias.data_ptr(), buf.data_ptr(), M, N, K, ldc, act,
                                        torch.cuda.current_stream().cuda_stream), "gemm")
    ref = ops.gemm_fp8_rowcol(a, b, sa, sb, bias, act)
    assert torch.equal(buf[:M, :N], ref)
    assert bool((buf[M:] == 7.0).all()) and bool((buf[:, N:] == 7.0).all())
    assert torch.equal(ops.gemm_fp8_rowcol(a, b, sa, sb, bias, act), ref)


@pytest.mark.parametrize("N", [384, 640])
def test_gemm_rowcol_persistent_strided_out(dev, N):
    """ldc > N on the carried-epilogue path (K = 1024): columns past N untouched.
    N = 384 runs 256-wide tiles; N = 640 runs 256 x 192 tiles with a 64-wide
    last stripe, whose 96-column waves must not write past their own columns."""
    ops = pkg_module("ops")
    L = pkg_module("_lib")
    ldc = N + 8
    a = torch.randint(0, 120, (300, 1024), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    b = torch.randint(0, 120, (N, 1024), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    sa = torch.rand(300, device=dev) + 0.5
    sb = torch.rand(N, device=dev) + 0.5
    out = torch.full((300, ldc), 3.0, dtype=torch.bfloat16, device=dev)
    L.check(L.load().hn_gemm_fp8_rowcol(a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                                        None, out.data_ptr(), 300, N, 1024, ldc, 0,
                                        torch.cuda.current_stream().cuda_stream), "gemm")
    ref = ops.gemm_fp8_rowcol(a, b, sa, sb)
    assert torch.equal(out[:, :N], ref)
    assert (out[:, N:] == 3.0).all()


def test_gemm_rowcol_is_deterministic(dev):
    ops = pkg_module("ops")
    a = torch.randint(0, 120, (1000, 1024), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    b = torch.randint(0, 120, (512, 1024), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    sa = torch.rand(1000, device=dev)
    sb = torch.rand(512, device=dev)
    assert torch.equal(ops.gemm_fp8_rowcol(a, b, sa, sb), ops.gemm_fp8_rowcol(a, b, sa, sb))


@pytest.mark.parametrize("m,n,k", [(1, 128, 128), (129, 256, 384), (2560, 4096, 4096), (4097, 128, 4096)])
def test_blockwise_gemm_reference_harness(O, dev, m, n, k):
    """The reference's own GEMM test (seed 44, a[:,128:256] *= 20, b[:128] *= 0.03)."""
    print(f"case blockwise gemm {m}x{n}x{k}", flush=True)
    pf = pkg_module("pixelumm_fp8")
    torch.manual_seed(44)
    a = torch.randn(m, k).to(torch.bfloat16)
    b = torch.randn(n, k).to(torch.bfloat16)
    a[:, 128:256] *= 20
    b[:128] *= 0.03
    qa, sa = pf._quantize_blockwise(a.to(dev))
    qb, sb = pf._quantize_blockwise(b.to(dev))
    actual = pf.load_extension().gemm(qa, qb, sa, sb)
    expected = O.blockwise_gemm_reference(u8(qa), sa.cpu().numpy(), u8(qb), sb.cpu().numpy())
    got = actual.float().cpu().numpy()
    assert np.isfinite(got).all()
    rel = np.linalg.norm(got - expected) / np.linalg.norm(expected)
    assert rel < 0.004, rel
    # and the bf16 rounding bound of the output itself
    assert np.all(np.abs(got - expected) <= np.abs(expected) * 2 ** -8 + 1e-3 * np.abs(expected).max())


def _blockwise_check(got, expected):
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all()
    rel = np.linalg.norm(got - expected) / np.linalg.norm(expected)
    assert rel < 0.004, rel
    assert np.all(np.abs(got - expected) <= np.abs(expected) * 2 ** -8 + 1e-3 * np.abs(expected).max())


@pytest.mark.parametrize("m,n,k", [(1536, 4096, 12288), (1536, 12288, 4096), (10800, 4096, 4096)])
def test_blockwise_gemm_decoder_shapes(O, dev, m, n, k):
    """The decoder's projection shapes (pixelumm_decoder/model.py:43-53: q/o/gate/up
    and down, K 4096 and 12288), with activation K blocks whose magnitudes differ
    by up to 2^16 and one all-zero K block, so the per-K-block promotion sees
    widely different factors. Row blocks 0 and last against the oracle."""
    print(f"case blockwise decoder gemm {m}x{n}x{k}", flush=True)
    pf = pkg_module("pixelumm_fp8")
    g = torch.Generator().manual_seed(11)
    a = torch.randn(m, k, generator=g)
    b = torch.randn(n, k, generator=g)
    gain = 2.0 ** torch.randint(-8, 9, (k // 128,), generator=g).float()
    a = a * gain.repeat_interleave(128)[None, :]
    a[:, 256:384] = 0.0
    qa, sa = pf._quantize_blockwise(a.to(torch.bfloat16).to(dev))
    qb, sb = pf._quantize_blockwise(b.to(torch.bfloat16).to(dev))
    got = pf.load_extension().gemm(qa, qb, sa, sb)
    last = (m - 1) // 128
    rows = list(range(0, 128)) + list(range(last * 128, m))
    expected = O.blockwise_gemm_reference(u8(qa)[rows], sa.cpu().numpy()[[0, last]], u8(qb), sb.cpu().numpy())
    _blockwise_check(got[rows], expected)


# A blockwise launch whose last row stripe (at most 64 rows) would add a whole
# round of tiles hands the stripe to gemm_tail_kernel in its blockwise mode:
# the decoder's gate and up projections (10800 x 4096 -> 12288), 4116 rows
# over 16 column tiles (257 -> 256 tiles), and M <= 64 (the stripe alone).
# Activation K blocks of gains up to 2^+-8, an all-zero K block and zero
# factors (a weight K block given scale 0, and the stripe's own row block).
@pytest.mark.parametrize("m,n,k", [(10800, 12288, 4096), (4116, 4096, 512), (48, 512, 1024), (33, 256, 4096)])
def test_blockwise_gemm_tail_stripe(O, dev, m, n, k):
    print(f"case blockwise tail stripe {m}x{n}x{k}", flush=True)
    pf = pkg_module("pixelumm_fp8")
    g = torch.Generator().manual_seed(m + n)
    a = torch.randn(m, k, generator=g)
    b = torch.randn(n, k, generator=g)
    gain = 2.0 ** torch.randint(-8, 9, (k // 128,), generator=g).float()
    a = a * gain.repeat_interleave(128)[None, :]
    a[:, 256:384] = 0.0
    qa, sa = pf._quantize_blockwise(a.to(torch.bfloat16).to(dev))
    qb, sb = pf._quantize_blockwise(b.to(torch.bfloat16).to(dev))
    last = (m - 1) // 128
    sb[0, 1] = 0.0        # a weight K block with factor 0 in the first column block
    sa[last, 2] = 0.0     # and one in the stripe's own row block
    got = pf.load_extension().gemm(qa, qb, sa, sb)
    rows = sorted(set(range(0, min(m, 64))) | set(range(max(0, m - 96), m)))
    rblocks = sorted(set(r // 128 for r in rows))
    sa_sel = sa.cpu().numpy()[rblocks]
    # re-index the selected rows' scale blocks for the oracle (rows in order, one scale row per 128)
    expected = np.concatenate([
        O.blockwise_gemm_reference(u8(qa)[[r for r in rows if r // 128 == rb]], sa_sel[[i]], u8(qb), sb.cpu().numpy())
        for i, rb in enumerate(rblocks)])
    _blockwise_check(got[rows], expected)
    assert torch.equal(pf.load_extension().gemm(qa, qb, sa, sb), got)


def test_blockwise_gemm_zero_block_factors(O, dev):
    """Block factors of 0 (an activation K block and a weight K block given scale 0
    by the caller) contribute nothing; the other blocks are promoted as usual."""
    pf = pkg_module("pixelumm_fp8")
    g = torch.Generator().manual_seed(12)
    a = torch.randn(300, 1024, generator=g).to(torch.bfloat16)
    b = torch.randn(384, 1024, generator=g).to(torch.bfloat16)
    qa, sa = pf._quantize_blockwise(a.to(dev))
    qb, sb = pf._quantize_blockwise(b.to(dev))
    sa[:, 1] = 0.0
    sa[2, 0] = 0.0
    sb[0, 3] = 0.0
    sb[:, 7] = 0.0
    got = pf.load_extension().gemm(qa, qb, sa, sb)
    expected = O.blockwise_gemm_reference(u8(qa), sa.cpu().numpy(), u8(qb), sb.cpu().numpy())
    _blockwise_check(got, expected)


@pytest.mark.parametrize("direction", ["up", "down"])
def test_blockwise_gemm_factor_jump_of_2_to_60(O, dev, direction):
    """Adjacent K blocks whose weight factors differ by 2^60, the widest span
    the FP8Linear loader accepts: the carried accumulator's rescale by
    f_prev / f (2^60 or 2^-60 here) stays finite, and the result matches the
    float64 dequantize-then-matmul reference."""
    pf = pkg_module("pixelumm_fp8")
    g = torch.Generator().manual_seed(31)
    a = torch.randn(256, 512, generator=g).to(torch.bfloat16)
    b = torch.randn(256, 512, generator=g).to(torch.bfloat16)
    qa, sa = pf._quantize_blockwise(a.to(dev))
    qb, sb = pf._quantize_blockwise(b.to(dev))
    # K blocks 2, 3 at exactly 2^60 (2^-60) times the row's smallest (largest)
    # factor of blocks 0, 1: the row span is then 2^60, the loader's bound
    if direction == "up":
        sb[:, 2:] = sb[:, :2].amin(dim=1, keepdim=True) * 2.0 ** 60
    else:
        sb[:, 2:] = sb[:, :2].amax(dim=1, keepdim=True) * 2.0 ** -60
    span = sb.amax(dim=1) / sb.amin(dim=1)
    assert bool((span == 2.0 ** 60).all()), span
    pf.validate_serialized_tensors(qb, sb, (256, 512))  # within the loader's bound
    with pytest.raises(ValueError, match="span more than 2"):
        pf.validate_serialized_tensors(qb, sb * torch.tensor([1.0, 1.0, 2.0, 2.0], device=dev) ** (
            1 if direction == "up" else -1), (256, 512))
    got = pf.load_extension().gemm(qa, qb, sa, sb)
    assert torch.isfinite(got.float()).all()
    expected = O.blockwise_gemm_reference(u8(qa), sa.cpu().numpy(), u8(qb), sb.cpu().numpy())
    _blockwise_check(got, expected)


def test_blockwise_gemm_contract_errors(dev):
    pf = pkg_module("pixelumm_fp8")
    ext = pf.load_extension()
    a = torch.zeros(64, 256, dtype=torch.float8_e4m3fn, device=dev)
    b = torch.zeros(128, 256, dtype=torch.float8_e4m3fn, device=dev)
    sa = torch.ones(1, 2, device=dev)
    sb = torch.ones(1, 2, device=dev)
    assert ext.gemm(a, b, sa, sb).shape == (64, 128)
    with pytest.raises(RuntimeError, match="Invalid activation scales"):
        ext.gemm(a, b, torch.ones(2, 2, device=dev), sb)
    with pytest.raises(RuntimeError, match="Invalid GEMM shape"):
        ext.gemm(a, torch.zeros(96, 256, dtype=torch.float8_e4m3fn, device=dev), sa, sb)
    with pytest.raises(RuntimeError, match="E4M3"):
        ext.gemm(a.view(torch.uint8), b, sa, sb)


def test_fp8_linear_modules(O, dev):
    """FP8Linear (decoder, blockwise) and FP8StoredLinear (DiT, per-channel)
    forwards against the oracle."""
    pf = pkg_module("pixelumm_fp8")
    dl = pkg_module("dit_fp8_linear")
    torch.manual_seed(3)
    lin = torch.nn.Linear(256, 384, bias=False).to(dev, torch.bfloat16).eval()
    m = pf.FP8Linear(lin)
    x = torch.randn(2, 65, 256, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y = m(x)
    assert y.shape == (2, 65, 384)
    qa, sa = O.quantize_blockwise_fp8(bf16_bits(x.reshape(-1, 256)))
    ref = O.blockwise_gemm_reference(qa, sa, u8(m.fp8_weight), m.fp8_scale.cpu().numpy())
    assert_close_bf16(y.reshape(-1, 384).float().cpu().numpy(), ref, what="FP8Linear")
    assert pf.execution_stats()[-1]["calls"] >= 1

    lin2 = torch.nn.Linear(256, 128).to(dev, torch.bfloat16)
    d = dl.FP8StoredLinear(lin2)
    with torch.no_grad():
        y2 = d(x)
    qx, sx = O.quantize_rows_fp8(bf16_bits(x.reshape(-1, 256)))
    ref2 = O.linear_reference(qx, sx, u8(d.weight_q), d.weight_scale.cpu().numpy(),
                              O.bf16_bits_to_f32(bf16_bits(lin2.bias)))
    assert_close_bf16(y2.reshape(-1, 128).float().cpu().numpy(), ref2, what="FP8StoredLinear")
    with pytest.raises(TypeError):
        d(x.float())
