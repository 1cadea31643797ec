"""grx_matmul_q8_dev_noalloc (the allocation-free product: the library's
fixed per-GPU scratch holds the rounded activations) against
grx_matmul_q8_dev, bit for bit, through the C ABI: two calls in a row, the
second smaller (so the scratch keeps the first call's bytes past the
second's), a call near the scratch's limit, and one past it.  Every
noalloc call runs with the library's allocation hook armed to fail the
next allocation (grx_debug_fail_alloc_after(0)): the call must succeed and
leave the hook armed, i.e. allocate nothing."""
import numpy as np
import pytest

from gorelaxor_amd import GrxError, _lib
from gorelaxor_amd.synth import q8_weight

pytestmark = pytest.mark.gpu


def _both(kern, rng, m, n, k, bias, lda_pad=8, ldc_pad=3):
    from gorelaxor_amd import hiprt

    x = rng.standard_normal((m, k + lda_pad)).astype(np.float32)
    w = kern.NewQ8(n, k, q8_weight(rng, n, k))
    b = hiprt.DeviceBuffer.from_array(rng.standard_normal(n).astype(np.float32)) if bias else None
    dx = hiprt.DeviceBuffer.from_array(x)
    d1 = hiprt.DeviceBuffer.from_array(np.full((m, n + ldc_pad), 7.0, np.float32))
    d2 = hiprt.DeviceBuffer.from_array(np.full((m, n + ldc_pad), 7.0, np.float32))
    kern.matmul_dev(d1, dx, m, w, b, ldc=n + ldc_pad, lda=k + lda_pad)
    kern.default_context().sync()
    lib = _lib.lib()
    lib.grx_debug_fail_alloc_after(0)  # the next allocation fails
    try:
        kern.matmul_dev_noalloc(d2, dx, m, w, b, ldc=n + ldc_pad, lda=k + lda_pad)
        kern.default_context().sync()
        assert lib.grx_debug_alloc_countdown() == 0, "the allocation-free product allocated"
    finally:
        lib.grx_debug_fail_alloc_after(-1)
    y1 = d1.download(np.float32, (m, n + ldc_pad))
    y2 = d2.download(np.float32, (m, n + ldc_pad))
    return y1, y2


@pytest.mark.parametrize("shapes", [[(40, 1000, 1024, True), (3, 517, 256, False)],
                                    [(3600, 256, 1024, True), (17, 96, 64, True), (1, 1500, 1280, False)]],
                         ids=["gemm_then_gemv", "near_limit_then_smaller"])
def test_noalloc_equals_dev(kern, shapes):
    rng = np.random.default_rng(len(shapes))
    for m, n, k, bias in shapes:
        print(f"noalloc m={m} n={n} k={k} bias={bias}", flush=True)
        y1, y2 = _both(kern, rng, m, n, k, bias)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), (m, n, k)
        assert (y2[:, n:] == 7.0).all(), "wrote past ldc's row"


def test_noalloc_refuses_past_its_scratch(kern):
    from gorelaxor_amd import hiprt

    rng = np.random.default_rng(1)
    m, n, k = 4000, 32, 1024  # 4000 * 1024 + 4000 * 32 * 4 bytes > 4 MiB
    w = kern.NewQ8(n, k, q8_weight(rng, n, k))
    dx = hiprt.DeviceBuffer(m * k * 4)
    dy = hiprt.DeviceBuffer(m * n * 4)
    with pytest.raises(GrxError, match="scratch"):
        kern.matmul_dev_noalloc(dy, dx, m, w)
