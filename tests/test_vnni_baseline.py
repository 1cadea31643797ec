"""The benchmark's CPU baseline - the reference's int8 product with the
VNNI tile kernel and its task split (oracle/grx_vnni.cc, restating
internal/kern/q8int.go:35-223 and vnni_amd64.s) - gives the oracle's bits:
odd sizes (partial row tiles and panels, q8int_test.go / odd_test.go
shapes), the task split at several thread counts, a zero block, and the
ring loop the bench times."""
import numpy as np
import pytest

from gorelaxor_amd.synth import q8_weight


@pytest.fixture(scope="module")
def vnni(orc):
    if orc.vnni_kind() == 0:
        pytest.skip("this CPU has neither AVX512-VNNI nor AVX-VNNI")
    return orc


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("m", [1, 2, 5, 6, 7, 16, 17, 23, 49])
@pytest.mark.parametrize("n", [1, 3, 16, 17, 33])
def test_odd_sizes_equal_the_oracle(vnni, m, n):
    rng = np.random.default_rng(m * 100 + n)
    for k in (32, 96):
        w8 = q8_weight(rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32) if n % 2 else None
        want = vnni.matmul_q8_int(x, w8, n, k, b)
        vw = vnni.VnniWeight(w8, n, k)
        for threads in (1, 3, 8):
            assert np.array_equal(_bits(vnni.vnni_matmul(x, vw, b, threads=threads)), _bits(want)), (m, n, k, threads)


def test_large_and_zero_blocks(vnni):
    rng = np.random.default_rng(7)
    m, n, k = 300, 1024, 1024  # the reference benchmark's 300 x 1024 x 1024
    w8 = q8_weight(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3, 64:96] = 0.0  # a block of zeros: scale 0, bytes 128
    want = vnni.matmul_q8_int(x, w8, n, k)
    got = vnni.vnni_matmul(x, vnni.VnniWeight(w8, n, k), threads=8)
    assert np.array_equal(_bits(got), _bits(want))


def test_ring_loop(vnni):
    rng = np.random.default_rng(9)
    n, k, count = 64, 256, 5
    w8 = q8_weight(rng, n * count, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    panels, per = vnni.vnni_pack_many(w8, count, n, k)
    y = np.zeros(count * n, np.float32)
    vnni.vnni_ring(y, x, panels, per, count, n, k, 2, 2)
    src = n * (k // 32) * 34
    for i in range(count):
        want = vnni.matmul_q8_int(x, w8[i * src:(i + 1) * src], n, k)[0]
        assert np.array_equal(_bits(y[i * n:(i + 1) * n]), _bits(want)), i
