"""ctypes binding of libjamhip.so (include/jamhip.h). Raises if the library is not built: there is no
CPU fallback anywhere in this package."""
from __future__ import annotations

import atexit
import ctypes as C
import weakref
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libjamhip.so"

_lib = None

# (name, restype, argtypes) for every entry point of include/jamhip.h
_VP, _I, _I64 = C.c_void_p, C.c_int, C.c_int64
SIGNATURES = [
    ("jamhip_device_available", _I, []),
    ("jamhip_ctx_create", _VP, [_I]),
    ("jamhip_ctx_destroy", None, [_VP]),
    ("jamhip_global_destroy", None, []),
    ("jamhip_ctx_arch", C.c_char_p, [_VP]),
    ("jamhip_last_error", C.c_char_p, [_VP]),
    ("jamhip_mm", _I, [_VP, _VP, _I, _I, _VP, _I, _I, _VP, _I, _I, _I, _I, _I]),
    ("jamhip_weight_pin", _I, [_VP, _VP, _I, _I, _I]),
    ("jamhip_weight_evict", _I, [_VP, _VP]),
    ("jamhip_weight_bytes", _I64, [_VP]),
    ("jamhip_ctx_set_autopin", _I, [_VP, _I, _I64]),
    ("jamhip_ctx_autopin_stats", _I, [_VP, _VP]),
    ("jamhip_ctx_set_mx_native", _I, [_VP, _I]),
    ("jamhip_mm_device", _I, [_VP, _VP, _I, _I, _VP, _I, _I, _VP, _I, _I, _I, _I, _I]),
    ("jamhip_mm_device_noalloc", _I, [_VP, _VP, _I, _I, _VP, _I, _I, _VP, _I, _I, _I, _I, _I]),
    ("jamhip_quantize_device", _I, [_VP, _I, _VP, _I, _I, _I, _VP, _VP, _VP]),
    ("jamhip_mm_grouped", _I, [_VP, _VP, _I, _I, _I, _I, _VP, _VP, _I, _I, _VP, _I, _I, _I, _I, _VP]),
    ("jamhip_mm_grouped_ex", _I, [_VP, _VP, _I, _I, _I, _I, _VP, _VP, _I, _I, _VP, _I, _I, _I, _I, _VP, _VP]),
    ("jamhip_mm_grouped_gather", _I, [_VP, _VP, _I, _I, _I, _I, _VP, _VP, _I, _I, _VP, _I, _VP, _I, _I, _I, _I, _VP, _VP]),
    ("jamhip_moe_route", _I, [_VP, _VP, _I, _I, _I, _VP, _VP, _VP, _VP]),
    ("jamhip_moe_gather", _I, [_VP, _VP, _I, _VP, _VP, _I, _I, _I, _I, _VP, _I]),
    ("jamhip_moe_combine", _I, [_VP, _VP, _I, _VP, _VP, _VP, _I, _I, _I, _I, _VP, _I]),
    ("jamhip_moe_select_topk", _I, [_VP, _VP, _VP, _I, _I, _I, _I, _I, C.c_float, _VP, _VP, _VP, _VP]),
    ("jamhip_mm_device_ex", _I, [_VP, _VP, _I, _I, _VP, _I, _I, _VP, _I, _I, _I, _I, _I, _VP, _I]),
    ("jamhip_glu_device", _I, [_VP, _I, _VP, _I, _VP, _I, _I, _I]),
    ("jamhip_glu_device_vector", _I, [_VP, _I, _VP, _I, _VP, _I, _I, _I, _I]),
    ("jamhip_ctx_set_stream", _I, [_VP, _VP]),
    ("jamhip_ctx_stream", _VP, [_VP]),
    ("jamhip_ctx_synchronize", _I, [_VP]),
    ("jamhip_read_floor", _I, [_VP, _VP, _I64, _VP]),
    ("jamhip_gguf_open", _VP, [C.c_char_p, C.c_char_p, C.c_size_t]),
    ("jamhip_gguf_close", None, [_VP]),
    ("jamhip_gguf_tensor_count", _I64, [_VP]),
    ("jamhip_gguf_tensor_at", _I, [_VP, _I64, _VP]),
    ("jamhip_gguf_find", _I64, [_VP, C.c_char_p]),
    ("jamhip_gguf_data_offset", _I64, [_VP]),
    ("jamhip_gguf_alignment", _I, [_VP]),
    ("jamhip_gguf_pin", _I, [_VP, _VP, _VP, _VP, _VP]),
    ("jamhip_gguf_evict", _I, [_VP, _VP, _VP, _VP]),
]


def _adopt_torch_runtime() -> None:
    """Load PyTorch's HIP runtime first when PyTorch is installed.

    torch ships its own libamdhip64 (SONAME libamdhip64.so.7) and its libc10_hip asks for it under the
    name "libamdhip64.so". If libjamhip.so were loaded first it would pull /opt/rocm's copy (same SONAME,
    other file) and torch would then load a second runtime that finds no GPU. Importing torch first makes
    the dynamic loader resolve libjamhip's libamdhip64.so.7 to the runtime already in the process, so both
    share one HIP runtime, one device context and one set of streams."""
    try:
        import torch  # noqa: F401
    except Exception:
        pass


_LIVE: "weakref.WeakSet" = weakref.WeakSet()   # objects holding contexts or mappings: released at exit


def register_for_teardown(obj) -> None:
    """obj.close() runs at interpreter exit, before any runtime finalizer (see on_exit)."""
    _LIVE.add(obj)


def on_exit() -> None:
    """Deterministic teardown before the interpreter and the HIP runtime finalize: every live HipJAM context
    is destroyed (its pins, scratch and stream released), then every open GGUF mapping is closed, then the
    library's process-global context. Registered with atexit when the library is first loaded; objects'
    __del__ make no native call once this has run."""
    if on_exit.done or _lib is None:
        return
    on_exit.done = True
    objs = list(_LIVE)
    for o in sorted(objs, key=lambda o: getattr(o, "TEARDOWN_ORDER", 0)):
        try:
            o.close()
        except Exception:
            pass
    try:
        _lib.jamhip_global_destroy()
    except Exception:
        pass


on_exit.done = False


def lib() -> C.CDLL:
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m qxotic_amd.build` (no CPU fallback)")
        _adopt_torch_runtime()
        L = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
        atexit.register(on_exit)
    return _lib
