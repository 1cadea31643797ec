"""The C ABI library loads and exports every entry point include/grx.h
declares; argument errors come back as status codes (no GPU needed)."""
import ctypes as C

import numpy as np
import pytest

from gorelaxor_amd import _lib


def test_library_exports_every_declared_symbol():
    L = C.CDLL(_lib.LIB_PATH)
    declared = _lib.header_symbols()
    assert len(declared) >= 20
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    # the Python binding types every declared entry point
    assert sorted(_lib.SIGNATURES) == declared


def test_version_and_errors_without_context():
    L = _lib.lib()
    assert L.grx_version() >= 1
    h = C.c_void_p()
    buf = np.zeros(34, np.uint8)
    # NULL context -> GRX_EINVAL, message set for this thread
    rc = L.grx_weight_q8_create(None, 1, 32, buf.ctypes.data_as(C.c_void_p), 34, C.byref(h))
    assert rc == -1 and b"NULL" in L.grx_last_error()
    rc = L.grx_matmul_q8(None, None, 0, None, 0, 1, None, None)
    assert rc == -1
    with pytest.raises(_lib.GrxError):
        _lib.check(rc)


def test_no_device_is_an_error_not_a_fallback():
    """Without a GPU the library reports it (grx_device_count 0, ctx creation
    GRX_ENODEV); there is no CPU path to fall back to."""
    L = _lib.lib()
    if L.grx_device_count() > 0:
        pytest.skip("a GPU is visible here")
    h = C.c_void_p()
    assert L.grx_ctx_create(0, C.byref(h)) == -6
