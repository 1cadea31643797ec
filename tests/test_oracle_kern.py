"""Pins the CPU oracle's restatement of internal/kern's Q8_0 path against what
the mathematics and the reference's own tests fix (no GPU).

Each test names the reference test whose structure, sizes or tolerance it
follows (github.com/xattribution/gorelaxor, internal/kern/*_test.go).
"""
from fractions import Fraction

import numpy as np
import pytest

from tests._exact import bits, f32_round, fma32, mul32

QK = 32


def _sample_f32(rng, n):
    """float32 values over every exponent range, both signs, plus specials."""
    u = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    v = u.view(np.float32)
    extra = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 6.1035156e-05,
                      5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10, -3.0517578e-05],
                     np.float32)
    return np.concatenate([v, extra])


# ---------------------------------------------------------------- f16.go

def test_f16_to_f32_exhaustive(orc):
    """f16toF32 (f16.go:14-33) for all 65,536 halves against IEEE-754
    widening (numpy's float16), NaNs by class."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(x)) for x in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_ieee(orc):
    """f32toF16 (f16.go:36-71) rounds to nearest even, subnormals and
    overflow included, as IEEE-754 narrowing does; NaN -> sign|0x7e00."""
    rng = np.random.default_rng(1)
    v = _sample_f32(rng, 200000)
    got = np.array([orc.f32_to_f16(float(x)) for x in v], np.uint16)
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    nan = np.isnan(v)
    assert np.array_equal(got[~nan], want[~nan])
    assert all(orc.f32_to_f16(float(x)) in (0x7e00, 0xfe00) for x in v[nan][:100])
    # ties: 1 + 2^-11 is halfway between 1 and the next half -> even (1.0)
    assert orc.f32_to_f16(1 + 2**-11) == 0x3c00
    assert orc.f32_to_f16(1 + 3 * 2**-11) == 0x3c02


# ---------------------------------------------------------------- constants

@pytest.mark.parametrize("num,den,hexval", [
    (1, 127, 0x3c010204),    # quantU8's 1/127 (vnni_amd64.s:182)
    (1, 720, 0x3ab60b61), (1, 120, 0x3c088889), (1, 24, 0x3d2aaaab), (1, 6, 0x3e2aaaab),
])
def test_constants_are_nearest_floats(num, den, hexval):
    """The hex constants the oracle (and kernels) use are the float32 values
    Go's constant conversion gives: the nearest float32 of the exact ratio."""
    assert bits(f32_round(Fraction(num, den))) == hexval


def test_decimal_constants():
    for dec, hexval in [("1.4426950408889634", 0x3fb8aa3b), ("0.693145751953125", 0x3f317200),
                        ("1.428606765330187e-06", 0x35bfbe8e), ("0.044715", 0x3d372713),
                        ("0.7978845608028654", 0x3f4c422a)]:
        assert bits(f32_round(Fraction(dec))) == hexval, dec


# ---------------------------------------------------------------- ToQ8

def test_quant_q8_properties(orc):
    """ToQ8 / quantQ8 (kern.go:149-164, kern_test.go:10-28): the scale is
    f16(amax/127); the largest value maps to +-127; every value is within
    half a step of d*q (d before f16 rounding); exact halves round away."""
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(96 * 9) * rng.uniform(0.01, 10, 96 * 9)).astype(np.float32)
    v[32:64] = 0
    q8 = orc.quant_q8(v).reshape(-1, 34)
    for b in range(q8.shape[0]):
        xs = v[b * QK:(b + 1) * QK]
        amax = np.float32(np.abs(xs).max())
        d = np.float32(amax / np.float32(127))
        assert q8[b, 0:2].view(np.uint16)[0] == np.array([d], np.float32).astype(np.float16).view(np.uint16)[0]
        q = q8[b, 2:].view(np.int8).astype(np.int32)
        if amax == 0:
            assert (q == 0).all()
            continue
        assert np.abs(q).max() == 127
        assert q[np.argmax(np.abs(xs))] == (127 if xs[np.argmax(np.abs(xs))] > 0 else -127)
        idv = np.float32(1) / d
        exact = xs.astype(np.float64) * float(idv)
        assert (np.abs(q - exact) <= 0.5 + 1e-6).all()


def test_quant_q8_half_away(orc):
    """math.Round rounds x*id = k+0.5 away from zero (kern.go:163, as the
    converter's roundf, tools/convert_nemo.py:161), unlike quantU8's
    round-half-even: with amax = 127, d = 1 and id = 1 exactly."""
    v = np.zeros(32, np.float32)
    v[0] = 127.0
    v[1:6] = [2.5, -2.5, 0.5, 1.5, -0.5]
    q8 = orc.quant_q8(v)
    assert q8[0:2].view(np.uint16)[0] == 0x3c00
    assert list(q8[2:].view(np.int8)[1:6]) == [3, -3, 1, 2, -1]


def test_dequant_exact_with_subnormal_scale(orc):
    """TestDequantAsmExact (odd_test.go:79-112): d*q exactly, the negative
    subnormal half 0x8001 included."""
    rng = np.random.default_rng(4)
    for nb in (1, 2, 3, 7, 33):
        v = ((rng.random(nb * QK) * 2 - 1) * 1000).astype(np.float32)
        q = orc.quant_q8(v)
        q[0], q[1] = 0x01, 0x80
        got = orc.dequant_q8(q, nb * QK)
        blk = q.reshape(nb, 34)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
        want = (blk[:, 2:].copy().view(np.int8).astype(np.float64) * d).astype(np.float32).ravel()
        assert np.array_equal(got, want)


# ---------------------------------------------------------------- quantU8

def test_quant_u8_reference_cases(orc):
    """TestQuantU8AsmMatchesGo (q8int_test.go:9-35): a zero block -> scale 0
    and bytes 128; a negative extreme -40 -> byte 1."""
    rng = np.random.default_rng(3)
    nb = 9
    x = np.array([rng.standard_normal() * (1 + i // QK) for i in range(nb * QK)], np.float32)
    x[2 * QK:3 * QK] = 0
    x[5 * QK] = -40
    q, sc = orc.quant_u8(x)
    assert q[5 * QK] == 1 and sc[2] == 0 and q[2 * QK] == 128
    for b in range(nb):
        xs = x[b * QK:(b + 1) * QK]
        amax = np.float32(np.abs(xs).max())
        assert bits(sc[b]) == bits(mul32(amax, f32_round(Fraction(1, 127))))
        if amax == 0:
            continue
        idv = np.float32(127) / amax
        p = (xs * idv).astype(np.float32)
        want = np.clip(np.rint(p), -128, 127).astype(np.int32) + 128  # rint: half to even
        assert np.array_equal(q[b * QK:(b + 1) * QK].astype(np.int32), want)
        assert q[b * QK + np.argmax(np.abs(xs))] in (1, 255)


def test_quant_u8_half_even(orc):
    """quantU8 uses math.RoundToEven (q8int.go:101): x*id = 2.5 -> 2, 3.5 -> 4."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0            # amax 127 -> id = 1 exactly
    x[1], x[2], x[3], x[4] = 2.5, 3.5, -2.5, -0.5
    q, sc = orc.quant_u8(x)
    assert list(q[1:5].astype(int) - 128) == [2, 4, -2, 0]
    qi, sci = orc.quant_act_i8(x)
    assert list(qi[0, 1:5]) == [2, 4, -2, 0] and sci[0, 0] == sc[0]


# ---------------------------------------------------------------- int8 products

def test_block_dots_brute_force(orc):
    """Per-block int32 dots (vnni_amd64.s:34-54 minus 128*sum(w)) equal the
    int64 brute force sum of qa*qw."""
    rng = np.random.default_rng(11)
    m, n, k = 3, 37, 160
    qa = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    from gorelaxor_amd.synth import q8_weight
    w = q8_weight(rng, n, k)
    s = orc.block_dots(qa, w, n, k)
    wq = w.reshape(n, k // QK, 34)[:, :, 2:].copy().view(np.int8).astype(np.int64)
    want = np.einsum("mbi,nbi->mnb", qa.astype(np.int64).reshape(m, k // QK, QK), wq)
    assert np.array_equal(s.astype(np.int64), want)
    # the unsigned form of the VNNI kernel gives the same integer
    ua = qa.astype(np.int64) + 128
    alt = np.einsum("mbi,nbi->mnb", ua.reshape(m, k // QK, QK), wq) - 128 * wq.sum(axis=2)[None]
    assert np.array_equal(alt, want)


def test_matmul_int_fma_order_exact(orc):
    """The EVEX finalize (vnni_amd64.s:58-69, driven from the bias by
    q8int.go:175-222): c = fma(f32(s)*dw, da, c) block by block, checked in
    exact rational arithmetic; the unfused Go-twin order differs somewhere."""
    rng = np.random.default_rng(21)
    from gorelaxor_amd.synth import q8_weight, q8_dequant
    m, n, k = 2, 12, 256
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = q8_weight(rng, n, k)
    bias = rng.standard_normal(n).astype(np.float32)
    got = orc.matmul_q8_int(x, w, n, k, bias)
    qa, sa = orc.quant_act_i8(x)
    blk = w.reshape(n, k // QK, 34)
    dw = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    wq = blk[:, :, 2:].copy().view(np.int8).astype(np.int64)
    go_differs = False
    for i in range(m):
        for j in range(n):
            c = float(bias[j])
            cg = np.float32(bias[j])
            for b in range(k // QK):
                s = int((qa[i, b * QK:(b + 1) * QK].astype(np.int64) * wq[j, b]).sum())
                p = mul32(np.float32(s), dw[j, b])
                c = fma32(p, sa[i, b], c)
                cg = np.float32(cg + np.float32(np.float32(p) * sa[i, b]))
            assert bits(got[i, j]) == bits(c), (i, j)
            go_differs |= bits(cg) != bits(c)
    assert go_differs
    # and the Go-twin mode of the oracle reproduces the unfused order
    got_go = orc.matmul_q8_int(x, w, n, k, bias, evex=False)
    assert not np.array_equal(got_go, got)
    assert np.allclose(got_go, got, rtol=1e-4, atol=1e-4)  # TestInt8TileKernels tolerance
    del q8_dequant


@pytest.mark.parametrize("m,n,k", [(2, 1, 32), (5, 15, 64), (6, 16, 96), (7, 17, 32), (13, 40, 128),
                                   (50, 33, 256), (100, 70, 64)])
def test_matmul_int_rms(orc, m, n, k):
    """TestInt8MatMul (q8int_test.go:80-126): relative RMS <= 0.02 against
    float64 with the exact weights, odd sizes, lda = k+3, ldc = n+2."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wv = (rng.random(n * k) * 2 - 1).astype(np.float32)
    bias = rng.random(n).astype(np.float32)
    w = orc.quant_q8(wv)
    ref = orc.dequant_q8(w, n * k).reshape(n, k).astype(np.float64)
    got = orc.matmul_q8_int(x, w, n, k, bias)
    want = x.astype(np.float64) @ ref.T + bias
    rel = np.sqrt(((got - want) ** 2).sum() / (want ** 2).sum())
    assert rel <= 0.02


@pytest.mark.parametrize("m,n,k", [(1, 70, 64), (3, 33, 96), (17, 40, 128)])
def test_matmul_float_route(orc, m, n, k):
    """TestMatMulTypes (kern_test.go:30-73) on the float route (m <= 16 here:
    17 is skipped, the packed route is not restated): abs <= 1e-3."""
    if m > 16:
        pytest.skip("the m > 16 packed float route is outside the restatement")
    rng = np.random.default_rng(1)
    x = (rng.random((m, k)) * 2 - 1).astype(np.float32)
    wv = (rng.random(n * k) * 2 - 1).astype(np.float32)
    bias = rng.random(n).astype(np.float32)
    w = orc.quant_q8(wv)
    ref = orc.dequant_q8(w, n * k).reshape(n, k).astype(np.float64)
    got = orc.matmul_q8_float(x, w, n, k, bias)
    want = x.astype(np.float64) @ ref.T + bias
    assert np.abs(got - want).max() <= 1e-3


def test_odd_sizes_float_route(orc):
    """TestOddSizesBothPaths (odd_test.go:26-77), Q8_0 weights, m <= 16:
    |got - ref| <= 1e-4*(1+k)."""
    rng = np.random.default_rng(3)
    for m in (1, 2, 5, 6, 7, 16):
        for n in (1, 3, 4, 5, 15, 16, 17, 33):
            for k in (32, 96, 544):
                x = (rng.random((m, k)) * 2 - 1).astype(np.float32)
                wv = (rng.random(n * k) * 2 - 1).astype(np.float32)
                bias = rng.random(n).astype(np.float32)
                w = orc.quant_q8(wv)
                ref = orc.dequant_q8(w, n * k).reshape(n, k).astype(np.float64)
                got = orc.matmul_q8_float(x, w, n, k, bias)
                want = x.astype(np.float64) @ ref.T + bias
                assert np.abs(got - want).max() <= 1e-4 * (1 + k), (m, n, k)


def test_dot_q8_asm_vs_go_order(orc):
    """TestDotQ8AsmMatchesGo (kern_test.go:75-95): the dot4q8avx order and
    the dotQ8Go order agree within 1e-3 at k = 1024 (m = 1 uses the first,
    the last partial group of rows the second)."""
    rng = np.random.default_rng(2)
    k = 1024
    x = (rng.random(k) * 2 - 1).astype(np.float32)
    wv = (rng.random(5 * k) * 2 - 1).astype(np.float32)
    w = orc.quant_q8(wv)
    got = orc.matmul_q8_float(x[None], w, 5, k)[0]   # rows 0-3 asm order, row 4 Go order
    ref = orc.dequant_q8(w, 5 * k).reshape(5, k).astype(np.float64) @ x.astype(np.float64)
    assert np.abs(got - ref).max() <= 1e-3


# ---------------------------------------------------------------- vector math

def test_expf_vs_libm(orc):
    """expf (mathx.go:7-33) within 1e-6 relative of math.Exp over [-87, 88)
    (whisper_test.go:98-104); EXP8 (kernels_amd64.s:236-258) likewise."""
    v = np.float32(-87)
    while v < 88:
        want = np.exp(np.float64(v))
        assert abs(orc.expf(float(v)) - want) <= 1e-6 * want
        assert abs(orc.exp8(float(v)) - want) <= 1e-6 * want
        v = np.float32(v + np.float32(0.731))
    assert orc.expf(-88.0) == 0.0 and orc.expf(89.0) == float("inf")
    # the vector form clamps instead
    assert orc.exp8(-200.0) == orc.exp8(-87.0) > 0 and orc.exp8(200.0) == orc.exp8(88.0)


def test_expsub_vector_vs_scalar(orc):
    """TestVectorMath (whisper_test.go:69-86): expSub's assembly part and
    expSubGo agree within 1e-5 relative, sums within 1e-4."""
    x = np.array([(i % 97) * 0.37 - 20 for i in range(1003)], np.float32)
    e, s = orc.expsub(x, 3.0)
    want = np.exp(x.astype(np.float64) - 3.0)
    assert np.all(np.abs(e - want) <= 1e-5 * want + 1e-30)
    assert abs(s - want.sum()) <= 1e-4 * want.sum()


def test_softmax_vs_float64(orc):
    rng = np.random.default_rng(9)
    for n in (1, 7, 8, 9, 224, 1500):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        got = orc.softmax(x)
        e = np.exp(x.astype(np.float64) - x.max())
        assert np.abs(got - e / e.sum()).max() <= 2e-6
        assert abs(got.sum() - 1) <= 1e-5


def test_gelu_vs_tanh(orc):
    """geluVec vs the scalar gelu within 1e-5 (whisper_test.go:87-97) and
    both vs the tanh formula in float64."""
    x = np.array([(i % 211) * 0.05 - 5 for i in range(1003)], np.float32)
    got = orc.gelu(x)
    v = x.astype(np.float64)
    want = 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * v * (1 + 0.044715 * v * v)))
    assert np.abs(got - want).max() <= 1e-5


def test_silu_axpy(orc):
    """TestVectorOpsMatchGo (vec_test.go:9-37): closed forms within 1e-6."""
    rng = np.random.default_rng(6)
    for n in (0, 1, 7, 8, 9, 100, 1027):
        x = (rng.standard_normal(n) * 8).astype(np.float32)
        y = rng.standard_normal(n).astype(np.float32)
        if n > 2:
            x[0], x[1] = -120, 120
        got = orc.silu(x)
        v = x.astype(np.float64)
        want = v / (1 + np.exp(-v))
        assert np.all(np.abs(got - want) <= 1e-6 * (1 + np.abs(want)))
        got = orc.axpy(x, y, 0.5)
        assert np.all(np.abs(got - (v + 0.5 * y)) <= 1e-6 * (1 + np.abs(v)))


def test_layernorm_vs_float64(orc):
    """layerNorm (mathx.go:55-75) vs float64 within 1e-5; the pockettts
    float64 form (pockettts/nn.go:27-49) within 1e-6."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((4, 512)) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(512).astype(np.float32)
    b = rng.standard_normal(512).astype(np.float32)
    v = x.astype(np.float64)
    norm = (v - v.mean(1, keepdims=True)) / np.sqrt(v.var(1, keepdims=True) + 1e-5)
    assert np.abs(orc.layernorm(x, w, b) - (norm * w + b)).max() <= 1e-5 * 8
    assert np.abs(orc.layernorm_f64(x) - norm).max() <= 1e-6


def test_dot_f32_forms(orc):
    rng = np.random.default_rng(13)
    for k in (16, 64, 1500, 1503):
        x = rng.standard_normal(k).astype(np.float32)
        w = rng.standard_normal(4 * k).astype(np.float32)
        got = orc.dot_f32_x4(x, w, k, k)
        want = w.reshape(4, k).astype(np.float64) @ x.astype(np.float64)
        assert np.abs(got - want).max() <= 1e-5 * k ** 0.5 * 4
        assert abs(orc.dot_f32_go(x, w[:k]) - want[0]) <= 1e-5 * k ** 0.5 * 4


def test_argmax_first_index():
    import oracle
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle.argmax(np.array([-1, -1], np.float32)) == 0
    assert oracle.argmax(np.array([0, np.nan, 5, 5], np.float32)) == 2
