"""Parity of the HIP Q8_0 product (libgrx.so through its C ABI) with the CPU
oracle: bit-exact for the int8 work and for the float32 outputs, since the
kernels keep the VNNI kernel's per-output order (vnni_amd64.s:58-69).

Structure follows the reference tests (internal/kern/q8int_test.go,
odd_test.go, kern_test.go of github.com/xattribution/gorelaxor).
"""
import os

import numpy as np
import pytest

from gorelaxor_amd.synth import gemv_inputs, q8_weight

pytestmark = pytest.mark.gpu

QK = 32


def _bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _bits_equal_nan(a, b):
    """Bit-equal, except that a NaN matches any NaN (the sign and payload of
    a NaN made from non-NaN operands differ between x86 and gfx950)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _report(got, want):
    d = np.abs(got.astype(np.float64) - want)
    i = int(np.argmax(d))
    return f"max |diff| {d.max():.3g} at {i}: got {got.ravel()[i]!r} want {want.ravel()[i]!r}"


@pytest.fixture
def dev(kern):
    """Device buffers on the library's own HIP runtime (gorelaxor_amd.hiprt)."""
    from gorelaxor_amd import hiprt

    return hiprt


# ---------------------------------------------------------------- weights

def test_row_and_float32_exact(kern, orc):
    """Weight.Row / Float32 (kern.go:115-134) exactly d*q, a negative
    subnormal scale (0x8001, odd_test.go:86-88) included."""
    rng = np.random.default_rng(8)
    n, k = 37, 96
    wv = (rng.random(n * k) * 2 - 1).astype(np.float32)
    q8 = orc.quant_q8(wv)
    q8[0], q8[1] = 0x01, 0x80
    w = kern.NewQ8(n, k, q8)
    ref = orc.dequant_q8(q8, n * k)
    assert _bits_equal(w.Float32(), ref)
    row = np.zeros(k, np.float32)
    for j in (0, 1, 36):
        w.Row(row, j)
        assert _bits_equal(row, ref[j * k:(j + 1) * k])
    assert w.Bytes() >= n * k


def test_newq8_errors(kern):
    """NewQ8's checks (kern.go:76-84): cols % 32 and a short buffer."""
    with pytest.raises(kern.GrxError, match="multiple of 32"):
        kern.NewQ8(2, 40, np.zeros(200, np.uint8))
    with pytest.raises(kern.GrxError, match="bytes for a"):
        kern.NewQ8(2, 64, np.zeros(2 * 2 * 34 - 1, np.uint8))


def test_to_q8_matches_oracle(kern, orc):
    """Weight.ToQ8 (kern.go:136-170) on the GPU: bytes identical to the
    oracle's, zero blocks and exact halves included."""
    rng = np.random.default_rng(7)
    n, k = 9, 96
    v = rng.standard_normal(n * k).astype(np.float32)
    v[:32] = 0
    v[32] = 127.0
    v[33:38] = [2.5, -2.5, 0.5, 1.5, -0.5]
    v[96:128] *= 1e-6
    got = kern.ToQ8(v, n, k)
    assert np.array_equal(got, orc.quant_q8(v))


# ---------------------------------------------------------------- activations and dots

def test_quant_act_exact(kern, orc, dev):
    """quantU8 (q8int.go:88-105) on the GPU: bytes and scales bit-exact;
    TestQuantU8AsmMatchesGo's cases (zero block, extreme -40) included."""
    rng = np.random.default_rng(3)
    m, k = 3, 9 * QK
    x = (rng.standard_normal((m, k)) * (1 + np.arange(k) // QK)).astype(np.float32)
    x[0, 2 * QK:3 * QK] = 0
    x[0, 5 * QK] = -40
    x[1, :QK] = 127.0
    x[1, 1:5] = [2.5, 3.5, -2.5, -0.5]
    x[2, QK:2 * QK] *= 1e-30  # subnormal-range products
    dx = dev.DeviceBuffer.from_array(x)
    dq = dev.DeviceBuffer(m * k)
    ds = dev.DeviceBuffer(m * (k // QK) * 4)
    kern.quant_act_dev(dq, ds, dx, m, k)
    kern.default_context().sync()
    q, sc = orc.quant_act_i8(x)
    assert np.array_equal(dq.download(np.int8, (m, k)), q)
    assert _bits_equal(ds.download(np.float32, (m, k // QK)), sc)


def test_block_dots_exact(kern, orc, dev):
    """Per-block int32 dots bit-exact with the oracle (and so with the int64
    brute force the oracle is pinned to)."""
    rng = np.random.default_rng(11)
    m, n, k = 3, 130, 320
    qa = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    qa[0, :QK] = -128
    w8 = q8_weight(rng, n, k)
    w = kern.NewQ8(n, k, w8)
    ds = dev.DeviceBuffer(m * n * (k // QK) * 4)
    dqa = dev.DeviceBuffer.from_array(qa)
    kern.block_dots_dev(ds, dqa, m, w)
    kern.default_context().sync()
    assert np.array_equal(ds.download(np.int32, (m, n, k // QK)), orc.block_dots(qa, w8, n, k))


def test_float_kernels_bit_exact(kern, orc, dev):
    """expf (scalar form), EXP8 and geluVec as the decode and encode kernels
    evaluate them (branch-free), bit-identical to the oracle: a dense sweep
    of the ranges the softmax and GELU reach, the cut-offs at -87 / 88 and
    +-9 (GELU's tanh), NaN and infinities, and geluVec's scalar tail."""
    rng = np.random.default_rng(5)
    x = np.concatenate([
        np.linspace(-100.0, 100.0, 20001, dtype=np.float32),
        rng.standard_normal(4000).astype(np.float32) * 30,
        np.array([-87.0, np.nextafter(np.float32(-87.0), np.float32(0)), np.nextafter(np.float32(-87.0), np.float32(-100)),
                  88.0, np.nextafter(np.float32(88.0), np.float32(0)), np.nextafter(np.float32(88.0), np.float32(100)),
                  0.0, -0.0, 1e-30, -1e-30, np.inf, -np.inf, np.nan], np.float32),
    ]).astype(np.float32)
    dx = dev.DeviceBuffer.from_array(x)
    dy = dev.DeviceBuffer(x.size * 4)
    for fn, want in ((kern.VEC_EXPF, np.array([orc.expf(float(v)) for v in x], np.float32)),
                     (kern.VEC_EXP8, np.array([orc.exp8(float(v)) for v in x], np.float32))):
        kern.vec_dev(fn, dy, dx, x.size)
        kern.default_context().sync()
        got = dy.download(np.float32, (x.size,))
        assert _bits_equal_nan(got, want), f"function {fn}: " + _report(got, want)
    # geluVec: |2u| crosses the +-9 cut-off near |v| = 3.3; lengths leave a
    # scalar tail of 0..7 values
    g = np.concatenate([np.linspace(-12.0, 12.0, 4801, dtype=np.float32),
                        np.array([np.inf, -np.inf, np.nan, 0.0, -0.0], np.float32)])
    for n in (g.size, g.size - 3, 7, 1):
        gx = np.ascontiguousarray(g[:n])
        dg = dev.DeviceBuffer.from_array(gx)
        kern.vec_dev(kern.VEC_GELU, dg, dg, n)
        kern.default_context().sync()
        got = dg.download(np.float32, (n,))
        want = orc.gelu(gx)
        assert _bits_equal_nan(got, want), f"gelu n={n}: " + _report(got, want)


# ---------------------------------------------------------------- products

def _check_matmul(kern, orc, rng, m, n, k, bias=True, lda_pad=3, ldc_pad=2):
    x = rng.standard_normal((m, k + lda_pad)).astype(np.float32)
    w8 = q8_weight(rng, n, k)
    b = rng.standard_normal(n).astype(np.float32) if bias else None
    w = kern.NewQ8(n, k, w8)
    got = np.full((m, n + ldc_pad), 7.0, np.float32)
    kern.MatMul(got, n + ldc_pad, x, k + lda_pad, m, w, b)
    want = orc.matmul_q8_int(np.ascontiguousarray(x[:, :k]), w8, n, k, b)
    assert _bits_equal(got[:, :n], want), f"{m}x{n}x{k}: " + _report(got[:, :n], want)
    assert (got[:, n:] == 7.0).all(), "wrote past ldc's row"


@pytest.mark.parametrize("mx", [1, 0])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 6, 7, 8, 9, 16, 17])
def test_matmul_odd_sizes_bit_exact(kern, orc, m, mx):
    """TestOddSizesBothPaths / TestInt8MatMul shapes (odd_test.go:33-35,
    q8int_test.go:87): every output bit-identical to the oracle's EVEX order,
    strided rows (lda = k+3, ldc = n+2), with and without bias; groups of 4
    and 8 rows on the matrix-core GEMV or (GEMV_MX=0) the dot-product one."""
    rng = np.random.default_rng(100 + m)
    with kern.tuned(GEMV_MX=mx):
        for n in (1, 3, 4, 5, 15, 16, 17, 33, 64, 65, 129):
            for k in (32, 64, 96, 544, 4096):
                if k == 4096 and n > 65:
                    continue
                _check_matmul(kern, orc, rng, m, n, k, bias=(n % 2 == 1))


@pytest.mark.parametrize("waves", [1, 2, 4, 8, 16])
def test_matmul_every_wave_split(kern, orc, waves):
    """Splitting a tile's blocks over 1..16 waves (ordered chain in LDS)
    changes no bit."""
    rng = np.random.default_rng(31)
    with kern.tuned(GEMV_WAVES=waves):
        for m, n, k in ((1, 200, 1024), (2, 64, 512), (4, 70, 2048), (8, 130, 1280), (1, 64, 5120)):
            _check_matmul(kern, orc, rng, m, n, k)


@pytest.mark.parametrize("gemv1", [0, 1])
def test_matmul_one_row_kernels(kern, orc, gemv1):
    """One-row products through the decode kernel (GEMV1=1: loads issued
    before the prologue, batched fold, partial last batch) and the general
    kernel (GEMV1=0), every wave split, block counts that leave waves
    with 1, 2, 3 and 10 blocks and a partial batch: every bit as the oracle."""
    rng = np.random.default_rng(57)
    with kern.tuned(GEMV1=gemv1):
        for waves in (1, 2, 4, 8, 16):
            with kern.tuned(GEMV_WAVES=waves):
                for n, k in ((64, 32), (65, 96), (130, 512), (64, 1024), (200, 1280), (70, 1312), (64, 5120)):
                    _check_matmul(kern, orc, rng, 1, n, k, bias=(n % 2 == 0))


@pytest.mark.parametrize("rows", [8, 16, 32, 64])
def test_matmul_one_row_slices(kern, orc, rows):
    """One-row products on slices of 8, 16 or 32 rows of the weight's
    64-row tiles (GEMV1_ROWS; 64 = whole tiles), every wave count: block
    counts that leave a partial last group of blocks and waves with no
    block, row counts with partial tiles and slices past the last row,
    tile counts that are not a multiple of the 8 XCDs: every bit as the
    oracle."""
    rng = np.random.default_rng(61 + rows)
    with kern.tuned(GEMV1_ROWS=rows):
        for waves in (-1, 1, 2, 4, 8, 16):
            with kern.tuned(GEMV_WAVES=waves):
                for n, k in ((8, 32), (65, 96), (130, 512), (64, 1024), (200, 1280), (70, 1312), (520, 2048),
                             (64, 5120), (1000, 160)):
                    _check_matmul(kern, orc, rng, 1, n, k, bias=(n % 2 == 0))


@pytest.mark.parametrize("kernel", [1, 2])
def test_matmul_matrix_cores_all_small_sizes(kern, orc, kernel):
    """The matrix-core products forced for every m (GEMM_MIN_M=1), the
    whole-K register kernel (1) and the K-split one (2): the odd sizes
    again, bit-identical to the oracle."""
    rng = np.random.default_rng(41)
    with kern.tuned(GEMM_MIN_M=1, GEMM_KERNEL=kernel):
        for m in (1, 2, 7, 15, 16, 17, 63, 64, 65):
            for n in (1, 17, 64, 65, 129):
                for k in (32, 96, 544):
                    _check_matmul(kern, orc, rng, m, n, k, bias=(n % 2 == 1))


@pytest.mark.parametrize("ns", [1, 2, 4])
def test_matmul_matrix_cores_each_tile_width(kern, orc, ns):
    """Every wave-tile width of the register-walk product (16, 32 or 64
    weight rows per wave, GEMM_NS) over block counts that hit each branch of
    its two-register-set walk (nb = 1 .. 40 around multiples of 4, 6, 8)."""
    rng = np.random.default_rng(43 + ns)
    with kern.tuned(GEMM_MIN_M=1, GEMM_KERNEL=1, GEMM_NS=ns):
        for nb in (1, 3, 4, 5, 6, 7, 8, 9, 11, 12, 13, 16, 17, 18, 24, 25, 40):
            for m, n in ((1, 64), (17, 100), (70, 130)):
                _check_matmul(kern, orc, rng, m, n, 32 * nb, bias=(nb % 2 == 1))


@pytest.mark.parametrize("sa", [0, 1])
@pytest.mark.parametrize("ns,kb", [(1, 4), (1, 8), (1, 16), (2, 4), (2, 8)])
def test_matmul_k_split_each_shape(kern, orc, ns, kb, sa):
    """The K-split product at every tile width and blocks per wave (GEMM_NS,
    GEMM_KB), with the activations read straight from memory or staged
    through LDS (GEMM_STAGE_A; the staged route needs whole groups of four
    blocks): block counts that give 1 to 8 waves per tile, a last wave with
    1 to KB blocks, activation-scale rows not in whole groups of four, and
    row counts with partial 16-row groups: bit-identical to the oracle."""
    rng = np.random.default_rng(53 + 7 * ns + kb)
    with kern.tuned(GEMM_MIN_M=1, GEMM_KERNEL=2, GEMM_NS=ns, GEMM_KB=kb, GEMM_STAGE_A=sa):
        for nb in sorted({1, 2, 3, 4, 5, 7, 8, 9, kb - 1, kb, kb + 1, 2 * kb + 3, 4 * kb, 8 * kb - 1, 8 * kb} - {0}):
            for m, n in ((1, 64), (14, 100), (33, 130), (126, 48), (200, 40)):
                _check_matmul(kern, orc, rng, m, n, 32 * nb, bias=(nb % 2 == 1))


@pytest.mark.parametrize("kernel", [3, 1])
def test_matmul_lds_tiles_and_register_tiles(kern, orc, kernel):
    """The LDS-staged 64 x 128 product forced for every row count
    (GEMM_KERNEL=3), and the register-tiled one for every row count (1),
    over partial row, column and block groups: bit-identical to the oracle."""
    rng = np.random.default_rng(47)
    with kern.tuned(GEMM_MIN_M=1, GEMM_KERNEL=kernel):
        for nb in (1, 3, 4, 5, 8, 9, 13):
            for m, n in ((1, 64), (20, 100), (64, 128), (65, 129), (200, 300)):
                _check_matmul(kern, orc, rng, m, n, 32 * nb, bias=(m % 2 == 1))


@pytest.mark.parametrize("m,n,k", [(126, 4096, 1024), (300, 1024, 1024), (1500, 512, 512), (251, 1024, 1024),
                                   (16, 4096, 1024)])
def test_matmul_many_rows_bit_exact(kern, orc, m, n, k):
    """Encoder, prefill and cross-attention shapes (M >= 16: matrix cores),
    and the reference benchmark's 300 x 1024 x 1024 (bench_test.go:35-55)."""
    rng = np.random.default_rng(m * 7 + n)
    _check_matmul(kern, orc, rng, m, n, k, lda_pad=0, ldc_pad=0)


def test_gemv_single_1024(kern, orc):
    """The single Q8_0 GEMV workload: N = K = 1024, int8 U[-127,127], f16
    scales |N(0,0.02)|/127 (~30% subnormal), x ~ N(0,1): bit-exact."""
    w8, x = gemv_inputs(seed=1)
    w = kern.NewQ8(1024, 1024, w8)
    got = np.zeros(1024, np.float32)
    kern.Linear(got, x, 1, w)
    want = orc.matmul_q8_int(x, w8, 1024, 1024)[0]
    assert _bits_equal(got, want), _report(got, want)


def test_gemv_golden_fixture(kern):
    """The committed fixture (tests/golden/q8_gemv_64x1024.npz) reproduced."""
    path = os.path.join(os.path.dirname(__file__), "golden", "q8_gemv_64x1024.npz")
    f = np.load(path)
    n, k = int(f["n"]), int(f["k"])
    w = kern.NewQ8(n, k, f["w"])
    got = np.zeros((f["x"].shape[0], n), np.float32)
    kern.MatMul(got, n, f["x"], k, f["x"].shape[0], w, f["bias"])
    assert _bits_equal(got, f["y"])


def test_gemv_logits_shape(kern, orc):
    """A vocabulary-sized product (51864 x 512, whisper base.en logits)."""
    rng = np.random.default_rng(5)
    n, k = 51864, 512
    w8 = q8_weight(rng, n, k, sigma=0.5)
    x = rng.standard_normal(k).astype(np.float32)
    w = kern.NewQ8(n, k, w8)
    got = np.zeros(n, np.float32)
    kern.Linear(got, x, 1, w)
    want = orc.matmul_q8_int(x, w8, n, k)[0]
    assert _bits_equal(got, want), _report(got, want)


def test_matmul_zero_rows_is_noop(kern):
    rng = np.random.default_rng(1)
    w = kern.NewQ8(4, 32, q8_weight(rng, 4, 32))
    dst = np.full(4, 3.0, np.float32)
    kern.MatMul(dst, 4, np.zeros(32, np.float32), 32, 0, w)
    assert (dst == 3.0).all()


@pytest.mark.parametrize("m", [1, 3, 40])
def test_matmul_no_columns_gives_bias(kern, m):
    """A product with K = 0 (no blocks): every output is its bias, or 0."""
    rng = np.random.default_rng(2)
    n = 70
    w = kern.NewQ8(n, 0, np.zeros(0, np.uint8))
    b = rng.standard_normal(n).astype(np.float32)
    dst = np.full((m, n), 3.0, np.float32)
    x = np.zeros((m, 1), np.float32)
    kern.MatMul(dst, n, x, 0, m, w, bias=b)
    assert _bits_equal(dst, np.tile(b, (m, 1)))
    kern.MatMul(dst, n, x, 0, m, w)
    assert (dst == 0.0).all()


def test_matmul_short_buffer_raises(kern):
    """The reference panics on a short slice (kernels_amd64.go:206-211);
    the mirror raises IndexError before any launch."""
    rng = np.random.default_rng(1)
    w = kern.NewQ8(4, 64, q8_weight(rng, 4, 64))
    with pytest.raises(IndexError):
        kern.MatMul(np.zeros(4, np.float32), 4, np.zeros(63, np.float32), 64, 1, w)


def test_device_pointer_forms(kern, orc, dev):
    """grx_matmul_q8_dev and the pre-rounded form on device buffers."""
    rng = np.random.default_rng(17)
    m, n, k = 4, 300, 768
    x = rng.standard_normal((m, k)).astype(np.float32)
    w8 = q8_weight(rng, n, k)
    b = rng.standard_normal(n).astype(np.float32)
    w = kern.NewQ8(n, k, w8)
    want = orc.matmul_q8_int(x, w8, n, k, b)
    dx, db = dev.DeviceBuffer.from_array(x), dev.DeviceBuffer.from_array(b)
    dy = dev.DeviceBuffer(m * n * 4)
    kern.matmul_dev(dy, dx, m, w, db)
    kern.default_context().sync()
    assert _bits_equal(dy.download(np.float32, (m, n)), want)
    dq = dev.DeviceBuffer(m * k)
    ds = dev.DeviceBuffer(m * (k // QK) * 4)
    kern.quant_act_dev(dq, ds, dx, m, k)
    dy2 = dev.DeviceBuffer(m * n * 4)
    kern.matmul_prequant_dev(dy2, dq, ds, m, w, db)
    kern.default_context().sync()
    assert _bits_equal(dy2.download(np.float32, (m, n)), want)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 63, 65, 130, 515, 2561])
@pytest.mark.parametrize("k", [32, 96, 640, 1024])
def test_linear_float_route_bit_exact(kern, orc, n, k):
    """The float route of a Q8_0 weight that keeps its rows (m = 1):
    dot4q8avx for rows in whole groups of four, dotQ8Go for the last partial
    group (n % 4 rows), then the bias - bit for bit, with subnormal scales."""
    rng = np.random.default_rng(n * 7 + k)
    w8 = q8_weight(rng, n, k, sigma=0.05)
    x = rng.standard_normal(k).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    w = kern.NewQ8(n, k, w8)
    for b in (None, bias):
        got = np.zeros(n, np.float32)
        kern.LinearFloat(got, x, w, b)
        want = orc.matmul_q8_float(x, w8, n, k, b)[0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, k, b is None)


@pytest.mark.parametrize("n,k", [(1, 16), (3, 17), (4, 32), (5, 47), (64, 256), (67, 100), (512, 32), (32, 512)])
def test_linear_f32_bit_exact(kern, orc, n, k):
    """A float32 weight's one-row product: dotF32x4 (the 16-wide kernel over
    k &^ 15 and dotF32Go past it) for rows in groups of four, dotF32Go for
    the rest, then the bias."""
    rng = np.random.default_rng(n + 31 * k)
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    for b in (None, bias):
        got = np.zeros(n, np.float32)
        kern.LinearF32(got, x, w, n, k, b)
        want = orc.matmul_f32(x[None], w, b)[0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, k, b is None)
