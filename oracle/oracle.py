"""ctypes front-end for the test oracle. TEST INFRASTRUCTURE ONLY.

Two libraries, both built by ``oracle/Makefile``:

* ``_build/liboracle.so`` -- this repository's C restatement of jam's arithmetic (jam_oracle.c);
* ``_ref/libjam.so``      -- the reference's own libjam, compiled from its C sources in place
  (jam/jam-native/src), used to pin the restatement and as the CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import this module.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "liboracle.so"
REF_SO = HERE / "_ref" / "libjam.so"

# ggml / jam dtype tags (jam/jam-native/include/jam.h:59-77)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16, MXFP4, NVFP4, Q1_0 = 0, 1, 2, 8, 12, 13, 14, 30, 39, 40, 41
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), MXFP4: (32, 17),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), NVFP4: (64, 36), Q1_0: (128, 18)}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", MXFP4: "MXFP4", Q5_K: "Q5_K",
         F32: "F32", F16: "F16", BF16: "BF16", NVFP4: "NVFP4", Q1_0: "Q1_0"}
QUANT_TYPES = (Q8_0, Q4_0, Q4_K, Q6_K, MXFP4)
NEW_QUANT_TYPES = (Q5_K, NVFP4, Q1_0)          # jam's int8 pipeline, added after the first five
ALL_QUANT_TYPES = QUANT_TYPES + NEW_QUANT_TYPES
DENSE_TYPES = (F32, F16, BF16)                 # jam's dense float paths


def row_bytes(dt: int, k: int) -> int:
    be, bb = BLOCK[dt]
    return k // be * bb


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Oracle:
    """The C restatement (jam_oracle.c)."""

    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(str(path))
        vp, i32, i64, u64, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float
        L.jo_half2float.argtypes, L.jo_half2float.restype = [C.c_uint16], f32
        L.jo_float2half.argtypes, L.jo_float2half.restype = [f32], C.c_uint16
        L.jo_e8m0_half.argtypes, L.jo_e8m0_half.restype = [C.c_uint8], f32
        L.jo_span_bytes.argtypes, L.jo_span_bytes.restype = [i32, i32, i32, i32], i64
        L.jo_dequant_row.argtypes = [i32, vp, i32, vp]
        L.jo_dequant_row_f64.argtypes = [i32, vp, i32, vp]
        L.jo_quantize_row.argtypes = [i32, vp, i32, vp]
        L.jo_quant_f1.argtypes = [vp, i32, vp, vp, vp]
        L.jo_quant_f2.argtypes = [vp, i32, vp, vp, vp]
        L.jo_mm_int8.argtypes = [i32, vp, i32, vp, i32, vp, i32, i32, i32, i32, i32]
        L.jo_mm_int8.restype = i32
        L.jo_mm_ref.argtypes = [i32, vp, i32, vp, i32, vp, vp, i32, i32, i32, i32]
        L.jo_mm_ref.restype = i32
        L.jo_mm_dense.argtypes = [i32, vp, i32, vp, i32, vp, i32, i32, i32, i32]
        L.jo_mm_dense.restype = i32
        L.jo_bf16_rounds_activations.argtypes, L.jo_bf16_rounds_activations.restype = [i32, i32], i32
        L.jo_ue4m3.argtypes, L.jo_ue4m3.restype = [C.c_uint8], f32
        L.jo_float2bf16.argtypes, L.jo_float2bf16.restype = [f32], C.c_uint16
        L.jo_fill_normal.argtypes = [u64, vp, C.c_size_t, f32, f32]
        L.jo_fill_outliers.argtypes = [u64, vp, C.c_size_t, f32, f32]

    # -- generators ---------------------------------------------------------------------------
    def normal(self, seed: int, shape, mean=0.0, std=1.0) -> np.ndarray:
        x = np.empty(shape, dtype=np.float32)
        self.lib.jo_fill_normal(C.c_uint64(seed & (2**64 - 1)), _p(x), x.size, mean, std)
        return x

    def outliers(self, seed: int, shape, p=0.01, mag=20.0) -> np.ndarray:
        x = np.empty(shape, dtype=np.float32)
        self.lib.jo_fill_outliers(C.c_uint64(seed & (2**64 - 1)), _p(x), x.size, p, mag)
        return x

    # -- formats ------------------------------------------------------------------------------
    def quantize(self, dt: int, x: np.ndarray) -> np.ndarray:
        """[rows, k] f32 -> [rows, row_bytes] uint8 GGUF blocks (the repo's own quantizers)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, k = x.shape
        out = np.zeros((rows, row_bytes(dt, k)), dtype=np.uint8)
        for r in range(rows):
            self.lib.jo_quantize_row(dt, _p(x[r]), k, _p(out[r]))
        return out

    def dequant(self, dt: int, w: np.ndarray, k: int, f64=False) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(dt, k))
        out = np.empty((w.shape[0], k), dtype=np.float64 if f64 else np.float32)
        fn = self.lib.jo_dequant_row_f64 if f64 else self.lib.jo_dequant_row
        for r in range(w.shape[0]):
            fn(dt, _p(w[r]), k, _p(out[r]))
        return out

    def quant_f1(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = x.shape
        q = np.empty((n, k), np.int8)
        d = np.empty((n, k // 32), np.float32)
        s = np.empty((n, k // 32), np.float32)
        for j in range(n):
            self.lib.jo_quant_f1(_p(x[j]), k, _p(q[j]), _p(d[j]), _p(s[j]))
        return q, d, s

    def quant_f2(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = x.shape
        q = np.empty((n, k), np.int8)
        d = np.empty((n, k // 32), np.float32)
        s = np.empty((n, k // 16), np.float32)
        for j in range(n):
            self.lib.jo_quant_f2(_p(x[j]), k, _p(q[j]), _p(d[j]), _p(s[j]))
        return q, d, s

    # -- matmuls ------------------------------------------------------------------------------
    def mm_int8(self, dt, w, a, m, n, k, ldw=None, flavour=0) -> np.ndarray:
        """jam's int8 pipeline, C[n, m] (token-major). flavour 0 = jam's rule (n<8 -> F1)."""
        ldw = ldw or k
        w = np.ascontiguousarray(w, dtype=np.uint8)
        a = np.ascontiguousarray(a, dtype=np.float32)
        c = np.zeros((n, m), np.float32)
        rc = self.lib.jo_mm_int8(dt, _p(w), ldw, _p(a), a.shape[-1], _p(c), m, m, n, k, flavour)
        if rc:
            raise ValueError("jo_mm_int8: unsupported")
        return c

    def mm_dense(self, dt, w, a, m, n, k, ldw=None) -> np.ndarray:
        """jam's dense F32 / F16 / BF16 paths, C[n, m] (BF16 rounds the activations where jam does)."""
        ldw = ldw or k
        w = np.ascontiguousarray(w, dtype=np.uint8)
        a = np.ascontiguousarray(a, dtype=np.float32)
        c = np.zeros((n, m), np.float32)
        if self.lib.jo_mm_dense(dt, _p(w), ldw, _p(a), a.shape[-1], _p(c), m, m, n, k):
            raise ValueError("jo_mm_dense: unsupported")
        return c

    def mm(self, dt, w, a, m, n, k, ldw=None) -> np.ndarray:
        """jam's own answer for any dtype: the int8 pipeline for quantized weights, the dense paths else."""
        if dt in DENSE_TYPES:
            return self.mm_dense(dt, w, a, m, n, k, ldw)
        return self.mm_int8(dt, w, a, m, n, k, ldw)

    def mm_ref(self, dt, w, a, m, n, k, ldw=None):
        """Float reference in double: (C[n, m], sumabs[n, m])."""
        ldw = ldw or k
        w = np.ascontiguousarray(w, dtype=np.uint8)
        a = np.ascontiguousarray(a, dtype=np.float32)
        c = np.zeros((n, m), np.float64)
        s = np.zeros((n, m), np.float64)
        rc = self.lib.jo_mm_ref(dt, _p(w), ldw, _p(a), a.shape[-1], _p(c), _p(s), m, m, n, k)
        if rc:
            raise ValueError("jo_mm_ref: unsupported")
        return c, s


# ---------------------------------------------------------------------------------------------
# The reference's own libjam (jam/jam-native/include/jam.h), built from source into oracle/_ref/.

class _JamConfig(C.Structure):   # jam.h:98-104
    _fields_ = [("parallel_for", C.c_void_p), ("pool", C.c_void_p), ("nthreads", C.c_int32),
                ("max_isa", C.c_int), ("name", C.c_char_p)]


class _Q8Job(C.Structure):       # jam/jam-native/src/jam_internal.h:148-158 (jam_q8_job)
    _fields_ = [("a", C.c_void_p), ("lda", C.c_int), ("b", C.c_void_p), ("ldb", C.c_int),
                ("c", C.c_void_p), ("ldc", C.c_int), ("n", C.c_int), ("k", C.c_int), ("nb", C.c_int),
                ("aq", C.c_void_p), ("ad", C.c_void_p), ("asum", C.c_void_p), ("m", C.c_int)]


class _Q4KJob(C.Structure):      # jam_internal.h:167-174 (jam_q4k_job)
    _fields_ = [("w", C.c_void_p), ("w_stride", C.c_int64), ("rhs", C.c_void_p), ("rhs_stride", C.c_int),
                ("xq", C.c_void_p), ("dx", C.c_void_p), ("xsum", C.c_void_p), ("out", C.c_void_p),
                ("out_stride", C.c_int), ("dim0", C.c_int), ("dim1", C.c_int), ("seq", C.c_int),
                ("kblocks", C.c_int), ("repack", C.c_void_p)]


JAM_ISA_AVX512_VNNI = 8  # jam.h:89-107 ordinal


class RefJam:
    """libjam compiled from the reference sources (oracle/_ref/libjam.so)."""

    def __init__(self, path: Path = REF_SO, nthreads: int = 0, max_isa: int = 0):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle` where /root/reference exists")
        L = self.lib = C.CDLL(str(path))
        vp, i32 = C.c_void_p, C.c_int
        L.jam_ctx_create.argtypes, L.jam_ctx_create.restype = [C.POINTER(_JamConfig)], vp
        L.jam_ctx_destroy.argtypes = [vp]
        L.jam_mm.argtypes = [vp, vp, i32, i32, vp, i32, i32, vp, i32, i32, i32, i32, i32]
        L.jam_mm.restype = i32
        L.jam_active_isa.argtypes, L.jam_active_isa.restype = [vp], i32
        L.jam_q8_0_requant.argtypes = [vp, i32, i32, i32]
        L.jam_q4k_quant.argtypes = [vp, i32, i32, i32]
        cfg = _JamConfig(None, None, nthreads, max_isa, b"oracle")
        self.ctx = L.jam_ctx_create(C.byref(cfg))
        if not self.ctx:
            raise RuntimeError("jam_ctx_create failed")

    def close(self):
        if self.ctx:
            self.lib.jam_ctx_destroy(self.ctx)
            self.ctx = None

    def active_isa(self) -> int:
        return self.lib.jam_active_isa(self.ctx)

    def mm(self, dt, w, a, m, n, k, ldw=None, lda=None, ldc=None, out=None) -> np.ndarray:
        ldw, lda, ldc = ldw or k, lda or a.shape[-1], ldc or m
        c = out if out is not None else np.zeros((n, ldc), np.float32)
        st = self.lib.jam_mm(self.ctx, _p(w), dt, ldw, _p(a), F32, lda, _p(c), F32, ldc, m, n, k)
        if st:
            raise RuntimeError(f"jam_mm status {st}")
        return c[:, :m] if out is None else c

    def status(self, w, wt, ldw, a, at, lda, c, ct, ldc, m, n, k) -> int:
        return self.lib.jam_mm(self.ctx, w, wt, ldw, a, at, lda, c, ct, ldc, m, n, k)

    def quant_f1(self, x: np.ndarray):
        """jam_q8_0_requant (jam_kernels_generic.c:71-94) over every row of x."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = x.shape
        q = np.empty((n, k), np.int8)
        d = np.empty((n, k // 32), np.float32)
        s = np.empty((n, k // 32), np.float32)
        job = _Q8Job(None, 0, x.ctypes.data, k, None, 0, n, k, k // 32, q.ctypes.data, d.ctypes.data,
                     s.ctypes.data, 0)
        self.lib.jam_q8_0_requant(C.byref(job), 0, n, 0)
        return q, d, s

    def quant_f2(self, x: np.ndarray):
        """jam_q4k_quant -> quantize_row_q8s (jam_kernels_q4k_avx512.c:25-47) over every row of x."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = x.shape
        q = np.empty((n, k), np.int8)
        d = np.empty((n, k // 32), np.float32)
        s = np.empty((n, k // 16), np.float32)
        job = _Q4KJob(None, 0, x.ctypes.data, k, q.ctypes.data, d.ctypes.data, s.ctypes.data, None, 0,
                      0, k, n, k // 32, None)
        self.lib.jam_q4k_quant(C.byref(job), 0, n, 0)
        return q, d, s


def ref_available() -> bool:
    return REF_SO.exists()


def default_threads() -> int:
    """Threads for the CPU baseline: the process's CPU share (capped at 16 on the GPU box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))
