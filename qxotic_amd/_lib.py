"""ctypes binding of libjamhip.so (include/jamhip.h). Raises if the library is not built: there is no
CPU fallback anywhere in this package."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libjamhip.so"

_lib = None

# (name, restype, argtypes) for every entry point of include/jamhip.h
_VP, _I, _I64 = C.c_void_p, C.c_int, C.c_int64
SIGNATURES = [
    ("jamhip_device_available", _I, []),
    ("jamhip_ctx_create", _VP, [_I]),
    ("jamhip_ctx_destroy", None, [_VP]),
    ("jamhip_ctx_arch", C.c_char_p, [_VP]),
    ("jamhip_last_error", C.c_char_p, [_VP]),
    ("jamhip_mm", _I, [_VP, _VP, _I, _I, _VP, _I, _I, _VP, _I, _I, _I, _I, _I]),
    ("jamhip_weight_pin", _I, [_VP, _VP, _I, _I, _I]),
    ("jamhip_weight_evict", _I, [_VP, _VP]),
    ("jamhip_weight_bytes", _I64, [_VP]),
    ("jamhip_mm_device", _I, [_VP, _VP, _I, _I, _VP, _I, _I, _VP, _I, _I, _I, _I, _I]),
    ("jamhip_quantize_device", _I, [_VP, _I, _VP, _I, _I, _I, _VP, _VP, _VP]),
    ("jamhip_ctx_set_stream", _I, [_VP, _VP]),
    ("jamhip_ctx_stream", _VP, [_VP]),
    ("jamhip_ctx_synchronize", _I, [_VP]),
]


def lib() -> C.CDLL:
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m qxotic_amd.build` (no CPU fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
