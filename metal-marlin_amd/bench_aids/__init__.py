"""ctypes binding of libmmfp4_bench.so: bench.py's measurement aids (an HBM
read stream and an MFMA-only loop).  They have no counterpart in the
reference and are not part of the GEMM library's ABI (declared in
mm_bench_aids.h beside this file, not in include/)."""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmmfp4_bench.so"
_c_int, _c_size, _vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
SIGNATURES = {
    "mm_bench_last_error": (ctypes.c_char_p, []),
    "mm_stream_read": (_c_int, [_vp, _c_size, _vp, _c_size, _c_int, _c_int, _c_int, _c_int, _vp]),
    "mm_mfma_ceiling": (_c_int, [_vp, _vp, _c_size, _c_int, _vp, _c_size, _vp]),
}
_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`python metal-marlin_amd/build.py`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            getattr(lib, name).restype = res
            getattr(lib, name).argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke `name`; ValueError for a bad argument (status 1), RuntimeError
    for a launch failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc:
        msg = lib.mm_bench_last_error().decode(errors="replace")
        raise (ValueError if rc == 1 else RuntimeError)(msg)
