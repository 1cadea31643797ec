"""gorelaxor_amd: MI355X (gfx950) Q8_0 product library with a host mirror of
gorelaxor's internal/kern API.

The compute lives in libgrx.so (HIP, built by gorelaxor_amd.build); the
Python modules are a thin ctypes layer over its C ABI (include/grx.h).
"""
from ._lib import GrxError, LIB_PATH  # noqa: F401

__all__ = ["GrxError", "LIB_PATH"]
