"""GGUF files and the device weight registry.

``GGUF`` opens a GGUF v3 file through the native reader (``jamhip_gguf_open``, include/jamhip.h), the
load step of jinfer's ``ModelLoader.loadTensors`` (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
kernels/ModelLoader.java:54-104): one read-only mapping of the tensor data region and one entry per
tensor. ``GGUF.pin`` then makes every jam-typed tensor resident on the GPU once, keyed by the host address
jam calls will pass. ``write`` produces GGUF v3 files (the layout the qxotic writer emits,
gguf/src/main/java/com/qxotic/format/gguf/impl/WriterImpl.java) for tests and benchmarks.
"""
from __future__ import annotations

import ctypes as C
import struct
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable, Sequence

import numpy as np

from ._lib import lib, on_exit, register_for_teardown

MAGIC = 0x46554747
VERSION = 3
DEFAULT_ALIGNMENT = 32

# metadata value type indices of the GGUF format (MetadataValueType.java)
VALUE_TYPES = {"uint8": 0, "int8": 1, "uint16": 2, "int16": 3, "uint32": 4, "int32": 5, "float32": 6,
               "bool": 7, "string": 8, "array": 9, "uint64": 10, "int64": 11, "float64": 12}
_SCALAR_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GGUFFormatError(ValueError):
    """The file is not a valid GGUF v3 file (GGUFFormatException in the qxotic reader)."""


class _TensorC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_int), ("dims", C.c_int64 * 4),
                ("offset", C.c_int64), ("bytes", C.c_int64), ("data", C.c_void_p)]


@dataclass(frozen=True)
class TensorEntry:
    """One tensor of the file (TensorEntry.java): GGUF-order shape (shape[0] contiguous)."""
    name: str
    ggml_type: int
    shape: tuple[int, ...]
    offset: int          # from the start of the tensor data region
    byte_size: int
    address: int         # in the handle's read-only mapping (0 if the data region is empty)


class GGUF:
    """A GGUF file opened by the native reader; close() (or a with-block) unmaps it."""

    TEARDOWN_ORDER = 1   # closed at exit after the contexts (which hold device copies, not the mapping)

    def __init__(self, path: str | Path):
        L = lib()
        err = C.create_string_buffer(512)
        self._h = L.jamhip_gguf_open(str(path).encode(), err, len(err))
        if not self._h:
            raise GGUFFormatError(err.value.decode(errors="replace"))
        register_for_teardown(self)
        self.path = str(path)
        self.alignment = L.jamhip_gguf_alignment(self._h)
        self.tensor_data_offset = L.jamhip_gguf_data_offset(self._h)
        self.tensors: dict[str, TensorEntry] = {}
        t = _TensorC()
        for i in range(L.jamhip_gguf_tensor_count(self._h)):
            if L.jamhip_gguf_tensor_at(self._h, i, C.byref(t)) != 0:
                raise RuntimeError(f"jamhip_gguf_tensor_at({i}) failed")
            e = TensorEntry(t.name.decode(), t.type, tuple(t.dims[: t.n_dims]), t.offset, t.bytes, t.data or 0)
            self.tensors[e.name] = e

    def close(self) -> None:
        if self._h:
            lib().jamhip_gguf_close(self._h)
            self._h = None

    def __enter__(self) -> "GGUF":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        if sys.is_finalizing() or on_exit.done:   # the exit-time teardown already closed it
            return
        try:
            self.close()
        except Exception:
            pass

    def find(self, name: str) -> int:
        """Index of the tensor in file order, or -1."""
        return lib().jamhip_gguf_find(self._h, name.encode())

    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping (valid until close())."""
        e = self.tensors[name]
        if e.byte_size == 0:
            return np.zeros(0, np.uint8)
        buf = (C.c_uint8 * e.byte_size).from_address(e.address)
        arr = np.frombuffer(buf, dtype=np.uint8)
        arr.flags.writeable = False
        return arr

    def pin(self, jam, data_base: int | None = None) -> tuple[int, int, int]:
        """Pin every jam-typed tensor on `jam`'s GPU (jamhip_gguf_pin): returns (status, tensors, bytes)."""
        n, b = C.c_int64(), C.c_int64()
        st = lib().jamhip_gguf_pin(jam.ctx, self._h, data_base, C.byref(n), C.byref(b))
        return st, n.value, b.value

    def evict(self, jam, data_base: int | None = None) -> int:
        """Drop this file's pins from `jam` (jamhip_gguf_evict); returns how many were dropped."""
        n = C.c_int64()
        st = lib().jamhip_gguf_evict(jam.ctx, self._h, data_base, C.byref(n))
        if st != 0:
            raise RuntimeError(f"jamhip_gguf_evict: status {st}")
        return n.value


# ------------------------------------------------------------------------------------------- writer
def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: str, value: Any) -> bytes:
    if vtype == "string":
        return struct.pack("<I", 8) + _string(value)
    if vtype.startswith("array:"):
        ct = VALUE_TYPES[vtype[6:]]
        body = b"".join(_string(v) for v in value) if ct == 8 else b"".join(struct.pack(_SCALAR_FMT[ct], v) for v in value)
        return struct.pack("<IIQ", 9, ct, len(value)) + body
    t = VALUE_TYPES[vtype]
    return struct.pack("<I", t) + struct.pack(_SCALAR_FMT[t], value)


def write(path: str | Path, tensors: Sequence[tuple[str, int, Sequence[int], Any]],
          metadata: Iterable[tuple[str, str, Any]] = (), alignment: int | None = None) -> int:
    """Write a GGUF v3 file; returns the file offset of its tensor data region.

    tensors: (name, ggml_type id, GGUF-order shape, bytes-like data) in file order; each tensor's data is
    placed at the next multiple of the alignment. metadata: (key, value type, value) with value types
    "uint8" … "float64", "string", or "array:<type>". alignment != None writes general.alignment."""
    kv = list(metadata)
    if alignment is not None:
        kv = [("general.alignment", "uint32", alignment)] + [e for e in kv if e[0] != "general.alignment"]
    align = alignment or DEFAULT_ALIGNMENT
    head = [struct.pack("<IIQQ", MAGIC, VERSION, len(tensors), len(kv))]
    head += [_string(k) + _value(t, v) for k, t, v in kv]
    blobs, off = [], 0
    for name, ggml_type, shape, data in tensors:
        raw = bytes(memoryview(data).cast("B")) if not isinstance(data, bytes) else data
        head.append(_string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
                    + struct.pack("<IQ", ggml_type, off))
        blobs.append((off, raw))
        off = (off + len(raw) + align - 1) // align * align
    header = b"".join(head)
    data_offset = (len(header) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data_offset - len(header)))
        pos = 0
        for o, raw in blobs:
            f.write(b"\0" * (o - pos))
            f.write(raw)
            pos = o + len(raw)
    return data_offset
