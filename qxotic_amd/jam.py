"""Host-side mirror of jam's backend SPI for the MI355X backend.

Mirrors, name for name, the Java contract a jam backend implements:

* ``JAM`` constants and ``JAM.mm`` (jam/jam-core/src/main/java/com/qxotic/jam/JAM.java:74-115);
* ``Provider`` / ``providers()`` discovery with ``jam.<id>.disabled`` (JAM.java:21-71), here read from
  the environment as ``JAM_<ID>_DISABLED`` (the NativeLoader config convention,
  jam/jam-native/src/main/java/com/qxotic/jam/NativeLoader.java:344-349);
* ``HipJAM.mm`` with NativeJAM's argument handling (NativeJAM.java:63-152): heap (non-native) operands
  raise ``IllegalArgumentError``; undersized operands raise ``IndexOutOfBoundsError`` before any native
  call, sized by ``GGMLType.span_bytes``; concurrent callers serialize FIFO unless
  ``JAM_HIP_SERIAL=false``, in which case a contended call returns ``EBUSY`` from the native guard.

Operands are ``Segment`` objects: a raw host address plus byte size (what a ``MemorySegment`` carries
across the FFM boundary). ``Segment.of(ndarray)`` wraps C-contiguous numpy memory.
"""
from __future__ import annotations

import ctypes as C
import os
import sys
import threading
from dataclasses import dataclass
from typing import Any

import numpy as np

from . import ggml
from ._lib import lib, on_exit, register_for_teardown


class JAM:
    """Constants of the JAM contract (JAM.java:74-87)."""

    F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4, NVFP4, Q1_0 = 0, 1, 30, 2, 8, 12, 13, 14, 39, 40, 41
    OK, EINVAL, EUNSUPPORTED, EBUSY = 0, 1, 2, 3


class IllegalArgumentError(ValueError):
    """java.lang.IllegalArgumentException (NativeJAM.requireNative, NativeJAM.java:115-122)."""


class IndexOutOfBoundsError(IndexError):
    """java.lang.IndexOutOfBoundsException (NativeJAM.checkSegment, NativeJAM.java:130-152)."""


@dataclass(frozen=True)
class Segment:
    """A native memory segment: address + byte size (+ an owner kept alive while referenced)."""

    address: int
    byte_size: int
    native: bool = True
    owner: Any = None

    @staticmethod
    def of(arr: np.ndarray) -> "Segment":
        if not isinstance(arr, np.ndarray) or not arr.flags.c_contiguous:
            return Segment(0, 0, native=False, owner=arr)
        return Segment(arr.ctypes.data, arr.nbytes, True, arr)

    @staticmethod
    def heap(obj: Any) -> "Segment":
        """A heap-backed segment: has no native address (rejected by mm)."""
        return Segment(0, 0, native=False, owner=obj)

    def is_native(self) -> bool:
        return self.native


def _config(key: str, default: str) -> str:
    """`jam.x.y` property convention read as env JAM_X_Y (NativeLoader.java:344-349)."""
    return os.environ.get(key.upper().replace(".", "_"), default)


class _FairLock:
    """FIFO lock (ReentrantLock(true) in NativeJAM.java:55)."""

    def __init__(self):
        self._cv = threading.Condition()
        self._next = 0
        self._serving = 0

    def __enter__(self):
        with self._cv:
            ticket = self._next
            self._next += 1
            while ticket != self._serving:
                self._cv.wait()

    def __exit__(self, *exc):
        with self._cv:
            self._serving += 1
            self._cv.notify_all()


class HipJAM:
    """The MI355X backend behind the JAM contract. One context = one HIP stream (a serial stream).

    ``HipJAM(device)`` owns a context of its own; ``HipJAM.global_context()`` is bound to the library's
    process-global context (ctx == NULL, as ``jam_mm(NULL, ...)``, jam/jam-native/include/jam.h:128). A
    call the GPU answers with EUNSUPPORTED is handed to ``fallback`` (the provider this one shadows) when
    one is set, so a dtype or shape the kernels do not cover still reaches the CPU backend."""

    def __init__(self, device: int = -1, *, _global: bool = False):
        L = lib()
        self._global = _global
        if _global:
            self._ctx = None
        else:
            self._ctx = L.jamhip_ctx_create(device)
            if not self._ctx:
                raise RuntimeError("jamhip_ctx_create: " + L.jamhip_last_error(None).decode())
        self._serial = _config("jam.hip.serial", "true").lower() == "true"
        self._lock = _FairLock() if self._serial else None
        self.fallback = None
        self._closed = False
        register_for_teardown(self)

    @classmethod
    def global_context(cls) -> "HipJAM":
        """A backend on the process-global context (created by the library on first use)."""
        return cls(_global=True)

    # -- lifecycle -------------------------------------------------------------------------------
    def close(self):
        """Destroys an owned context (a no-op for the global one: jamhip_global_destroy releases it)."""
        if not self._closed:
            self._closed = True
            if self._ctx:
                lib().jamhip_ctx_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        # never call into HIP while the interpreter shuts down: the exit-time teardown (_lib.on_exit) has
        # already released every context before the runtime's own finalizers run
        if sys.is_finalizing() or on_exit.done:
            return
        try:
            self.close()
        except Exception:
            pass

    @property
    def ctx(self) -> int | None:
        if self._closed:
            raise RuntimeError("HipJAM: context closed")
        return self._ctx

    def arch(self) -> str:
        return lib().jamhip_ctx_arch(self.ctx).decode()

    def last_error(self) -> str:
        return lib().jamhip_last_error(self.ctx).decode()

    # -- the contract ----------------------------------------------------------------------------
    def mm(self, w: Segment, w_off: int, wt: int, ldw: int, a: Segment, a_off: int, at: int, lda: int,
           r: Segment, r_off: int, rt: int, ldr: int, m: int, n: int, k: int) -> int:
        """R = W @ A^T; byte offsets, ELEMENT strides; returns a jam_status (JAM.java:95-110)."""
        _require_native(w, "weight W")
        _require_native(a, "activation A")
        _require_native(r, "result R")
        if m > 0 and n > 0 and k > 0 and ldw >= k and lda >= k and ldr >= m:   # else native -> EINVAL
            _check_segment("weight W", w, w_off, wt, ldw, m, k)
            _check_segment("activation A", a, a_off, at, lda, n, k)
            _check_segment("result R", r, r_off, rt, ldr, n, m)
        args = (self.ctx, w.address + w_off, wt, ldw, a.address + a_off, at, lda, r.address + r_off, rt, ldr, m, n, k)
        if self._lock is not None:
            with self._lock:
                st = self._native_mm(args)
        else:
            st = self._native_mm(args)
        if st == JAM.EUNSUPPORTED and self.fallback is not None:
            return self.fallback.mm(w, w_off, wt, ldw, a, a_off, at, lda, r, r_off, rt, ldr, m, n, k)
        return st

    @staticmethod
    def _native_mm(args) -> int:
        return lib().jamhip_mm(*args)

    def mm_contiguous(self, w: Segment, a: Segment, r: Segment, wt: int, m: int, n: int, k: int) -> int:
        """Offsets 0, strides k/k/m, F32 activations and result (JAM.java:113-115)."""
        return self.mm(w, 0, wt, k, a, 0, JAM.F32, k, r, 0, JAM.F32, m, m, n, k)

    # -- residency extensions (no JAM counterpart) -------------------------------------------------
    def pin(self, w: Segment, wt: int, ldw: int, m: int) -> int:
        _require_native(w, "weight W")
        g = ggml.by_code(wt)
        if g is not None and m > 0 and ldw > 0 and m * g.row_bytes(ldw) > w.byte_size:
            raise IndexOutOfBoundsError(f"pin: weight segment too small — need {m * g.row_bytes(ldw)} B, "
                                        f"segment is {w.byte_size} B")
        return lib().jamhip_weight_pin(self.ctx, w.address, wt, ldw, m)

    def evict(self, w: Segment) -> int:
        return lib().jamhip_weight_evict(self.ctx, w.address)

    def pinned_bytes(self) -> int:
        return lib().jamhip_weight_bytes(self._ctx)

    def set_autopin(self, sightings: int, max_bytes: int = 0) -> int:
        """Pin a whole W on its `sightings`-th jamhip_mm call (0 = off), content-checked per call
        (jamhip_ctx_set_autopin)."""
        return lib().jamhip_ctx_set_autopin(self.ctx, sightings, max_bytes)

    def set_mx_native(self, mode: int) -> int:
        """MXFP4 matrix-core calls on the native MX path: 0 off (jam semantics), 1 MX-FP8 hi + lo activations,
        2 hi only (jamhip_ctx_set_mx_native)."""
        return lib().jamhip_ctx_set_mx_native(self.ctx, mode)

    def autopin_stats(self) -> dict:
        """{pins, hits, staged, invalidated} since the context was created (jamhip_ctx_autopin_stats)."""
        out = (C.c_int64 * 4)()
        if lib().jamhip_ctx_autopin_stats(self.ctx, out) != 0:
            raise RuntimeError("autopin stats: " + self.last_error())
        return dict(zip(("pins", "hits", "staged", "invalidated"), list(out)))

    # -- device-resident path (torch tensors or raw device addresses) ------------------------------
    def mm_device(self, w: Segment, wt: int, ldw: int, a_dev: int, lda: int, c_dev: int, ldc: int,
                  m: int, n: int, k: int) -> int:
        return lib().jamhip_mm_device(self.ctx, w.address, wt, ldw, a_dev, JAM.F32, lda, c_dev, JAM.F32, ldc,
                                      m, n, k)

    def mm_device_noalloc(self, w: Segment, wt: int, ldw: int, a_dev: int, lda: int, c_dev: int, ldc: int,
                          m: int, n: int, k: int) -> int:
        """mm_device with no allocation on its path: W pinned, scratch from the GPU's static array
        (jamhip_mm_device_noalloc)."""
        return lib().jamhip_mm_device_noalloc(self.ctx, w.address, wt, ldw, a_dev, JAM.F32, lda, c_dev, JAM.F32, ldc,
                                              m, n, k)

    def mm_device_ex(self, w: Segment, wt: int, ldw: int, a_dev: int, lda: int, c_dev: int, ldc: int,
                     m: int, n: int, k: int, bias_dev: int | None = None, accumulate: bool = False) -> int:
        """mm_device with the fused epilogue C = [C +] (W·A^T [+ bias]) (jamhip_mm_device_ex)."""
        return lib().jamhip_mm_device_ex(self.ctx, w.address, wt, ldw, a_dev, JAM.F32, lda, c_dev, JAM.F32, ldc,
                                         m, n, k, bias_dev, int(accumulate))

    ACT_SWIGLU, ACT_SWIGLU_OAI = 1, 2

    def glu_device(self, act: int, gate_dev: int, ldg: int, up_dev: int, ldu: int, rows: int, cols: int) -> int:
        """In place on gate: SwiGLU (act 1) or gpt-oss clamped SwiGLU (act 2) (jamhip_glu_device)."""
        return lib().jamhip_glu_device(self.ctx, act, gate_dev, ldg, up_dev, ldu, rows, cols)

    def glu_device_vector(self, act: int, gate_dev: int, ldg: int, up_dev: int, ldu: int, rows: int, cols: int,
                          lanes: int) -> int:
        """glu_device in jinfer's default Vector API arithmetic (rational tanh) with a `lanes`-float species
        (jamhip_glu_device_vector)."""
        return lib().jamhip_glu_device_vector(self.ctx, act, gate_dev, ldg, up_dev, ldu, rows, cols, lanes)

    def read_floor(self, p_dev: int, nbytes: int, sink_dev: int) -> int:
        """Streaming read of nbytes at p_dev in the decode kernel's load shape (jamhip_read_floor)."""
        return lib().jamhip_read_floor(self.ctx, p_dev, nbytes, sink_dev)

    def quantize_device(self, flavour: int, a_dev: int, lda: int, n: int, k: int, q_dev: int, d_dev: int,
                        s_dev: int) -> int:
        return lib().jamhip_quantize_device(self.ctx, flavour, a_dev, lda, n, k, q_dev, d_dev, s_dev)

    # -- mixture of experts (device pointers; jamhip.h) -------------------------------------------
    def mm_grouped(self, w: Segment, wt: int, ldw: int, m: int, n_experts: int, counts_dev: int, a_dev: int,
                   lda: int, c_dev: int, ldc: int, k: int, rows_cap: int, offsets_dev: int | None = None) -> int:
        """One jam matmul per expert over CSR-grouped rows (Moe.dispatch's per-expert MatMul.gemm loop)."""
        _require_native(w, "weight W")
        return lib().jamhip_mm_grouped(self.ctx, w.address, wt, ldw, m, n_experts, counts_dev, a_dev, JAM.F32, lda,
                                       c_dev, JAM.F32, ldc, k, rows_cap, offsets_dev)

    def mm_grouped_ex(self, w: Segment, wt: int, ldw: int, m: int, n_experts: int, counts_dev: int, a_dev: int,
                      lda: int, c_dev: int, ldc: int, k: int, rows_cap: int, offsets_dev: int | None = None,
                      bias_dev: int | None = None) -> int:
        """mm_grouped with expert e's bias [m] (at bias + e·m) added in the store (jamhip_mm_grouped_ex)."""
        _require_native(w, "weight W")
        return lib().jamhip_mm_grouped_ex(self.ctx, w.address, wt, ldw, m, n_experts, counts_dev, a_dev, JAM.F32,
                                          lda, c_dev, JAM.F32, ldc, k, rows_cap, offsets_dev, bias_dev)

    def mm_grouped_gather(self, w: Segment, wt: int, ldw: int, m: int, n_experts: int, counts_dev: int, x_dev: int,
                          ldx: int, slot_route_dev: int, topk: int, c_dev: int, ldc: int, k: int, rows_cap: int,
                          offsets_dev: int | None = None, bias_dev: int | None = None) -> int:
        """moe_gather + mm_grouped_ex in one call: CSR row r of A is row slot_route[r] // topk of x
        (jamhip_mm_grouped_gather)."""
        _require_native(w, "weight W")
        return lib().jamhip_mm_grouped_gather(self.ctx, w.address, wt, ldw, m, n_experts, counts_dev, x_dev, JAM.F32,
                                              ldx, slot_route_dev, topk, c_dev, JAM.F32, ldc, k, rows_cap, offsets_dev,
                                              bias_dev)

    def moe_route(self, route_expert_dev: int, seq: int, topk: int, n_experts: int, counts_dev: int,
                  offsets_dev: int, slot_route_dev: int, route_slot_dev: int) -> int:
        """Moe.dispatch's CSR build on the device (Moe.java:188-206)."""
        return lib().jamhip_moe_route(self.ctx, route_expert_dev, seq, topk, n_experts, counts_dev, offsets_dev,
                                      slot_route_dev, route_slot_dev)

    def moe_gather(self, x_dev: int, ldx: int, slot_route_dev: int, offsets_dev: int, n_experts: int, seq: int,
                   topk: int, dim: int, g_dev: int, ldg: int) -> int:
        """Moe.dispatch's gather (Moe.java:214-222)."""
        return lib().jamhip_moe_gather(self.ctx, x_dev, ldx, slot_route_dev, offsets_dev, n_experts, seq, topk, dim,
                                       g_dev, ldg)

    TOPK_RAW, TOPK_SOFTMAX, TOPK_NORMALIZE = 0, 1, 2

    def moe_select_topk(self, selection_dev: int, weights_dev: int | None, rows: int, n_experts: int, ld: int,
                        topk: int, mode: int, route_expert_dev: int, route_prob_dev: int,
                        counts_dev: int | None = None, weights_scale: float = 1.0,
                        expert_scale_dev: int | None = None) -> int:
        """Moe.selectTopK on the device (selection consumed: winners masked to -Inf), then the row's weight
        step by mode: raw, gpt-oss's softmax over the selected logits x weights_scale, or normalizeTopP; the
        optional per-expert expertScale fold (jamhip_moe_select_topk)."""
        return lib().jamhip_moe_select_topk(self.ctx, selection_dev, weights_dev, rows, n_experts, ld, topk, mode,
                                            weights_scale, expert_scale_dev, route_expert_dev, route_prob_dev,
                                            counts_dev)

    def moe_combine(self, y_dev: int, ldy: int, route_expert_dev: int, route_prob_dev: int, route_slot_dev: int,
                    seq: int, topk: int, n_experts: int, dim: int, out_dev: int, ldo: int) -> int:
        """Moe.dispatch's prob-weighted scatter-add (Moe.java:208, 223-231), bit-identical order."""
        return lib().jamhip_moe_combine(self.ctx, y_dev, ldy, route_expert_dev, route_prob_dev, route_slot_dev, seq,
                                        topk, n_experts, dim, out_dev, ldo)

    def set_stream(self, stream: int | None) -> int:
        return lib().jamhip_ctx_set_stream(self.ctx, stream)

    def stream(self) -> int:
        return lib().jamhip_ctx_stream(self._ctx)

    def synchronize(self) -> int:
        return lib().jamhip_ctx_synchronize(self._ctx)


def _require_native(seg: Segment, which: str) -> None:
    if not isinstance(seg, Segment) or not seg.is_native():
        raise IllegalArgumentError(f"jam.mm: {which} must be a NATIVE (off-heap) MemorySegment — heap/array-backed "
                                   "has no native address")


def _check_segment(which: str, seg: Segment, off: int, dt: int, stride: int, rows: int, row_elems: int) -> None:
    g = ggml.by_code(dt)
    if g is None:
        return   # unrecognized dtype: native classifies it
    need = g.span_bytes(rows, stride, row_elems)
    if off < 0 or off > seg.byte_size - need:
        raise IndexOutOfBoundsError(f"jam.mm: {which} segment too small — need {need} B at offset {off}, "
                                    f"segment is {seg.byte_size} B")


# ------------------------------------------------------------------------------------ discovery
# Other JAM providers visible to discovery (what ServiceLoader finds on the class path besides this one;
# jam-native's NativeJAMProvider in a real deployment). register() adds one.
_REGISTERED: list = []


def register(provider) -> None:
    _REGISTERED.append(provider)


class Provider:
    """JAM.Provider (JAM.java:21-38) for the MI355X backend."""

    def id(self) -> str:
        """`native` by default: jinfer asks only for ids `native` and `vector` (MatMul.java:1770-1771),
        so answering to `native` above jam-native's priority puts the GPU under an unedited caller. The
        provider it shadows there (jam-native) stays reachable as the fallback of every call the GPU answers
        with EUNSUPPORTED. `JAM_HIP_ID=hip` (jam.hip.id) moves the GPU to its own id instead."""
        return _config("jam.hip.id", "native")

    def priority(self) -> int:
        return 2000   # above native (1000), vector (500), scalar (0)

    def is_available(self) -> bool:
        return bool(lib().jamhip_device_available())

    def create(self) -> HipJAM:
        jam = _shared()
        if jam.fallback is None:
            jam.fallback = self.shadowed()
        return jam

    def shadowed(self):
        """The backend of the highest-priority other available provider with this provider's id, or None."""
        for p in providers(_REGISTERED):
            if p is not self and not isinstance(p, Provider) and p.id() == self.id():
                return p.create()
        return None


_SHARED: HipJAM | None = None
_SHARED_LOCK = threading.Lock()


def _shared() -> HipJAM:
    """The provider's instance, on the process-global context (Provider.create may return a shared
    instance, JAM.java:31-37)."""
    global _SHARED
    with _SHARED_LOCK:
        if _SHARED is None:
            _SHARED = HipJAM.global_context()
        return _SHARED


def _disabled(p) -> bool:
    return _config(f"jam.{p.id()}.disabled", "false").lower() == "true"


def _available(p) -> bool:
    try:
        return bool(p.is_available())
    except Exception:
        return False


def providers(candidates=None) -> list:
    """Available providers, highest priority first; disabled ones are dropped BEFORE probing
    (JAM.java:52-71)."""
    ps = [Provider()] if candidates is None else list(candidates)
    ps = [p for p in ps if not _disabled(p)]
    ps = [p for p in ps if _available(p)]
    return sorted(ps, key=lambda p: p.priority(), reverse=True)


def addr(x) -> int:
    """Device address of a torch tensor (or pass-through int)."""
    return x if isinstance(x, int) else int(x.data_ptr())


__all__ = ["JAM", "HipJAM", "Provider", "providers", "register", "Segment", "IllegalArgumentError",
           "IndexOutOfBoundsError", "addr", "C"]
