"""GGUF block geometry (jam/jam-core/src/main/java/com/qxotic/jam/GGMLType.java:15-65) and vectorized
quantizers that build synthetic weights of the BASELINE shapes (N(0, 0.02) draws -> GGUF blocks).

The quantizers follow the same per-block rules as the repository's C restatement under oracle/ (which
the tests hold them to byte for byte); they exist here so the bench can make 14336x4096-class tensors in
well under a second without touching test infrastructure.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class GGMLType:
    name: str
    ggml: int           # ggml_type code (the GGUF on-disk tag)
    block_elems: int
    block_bytes: int

    def row_bytes(self, elements: int) -> int:
        """Byte span of `elements` consecutive elements (block multiple) (GGMLType.java:35-37)."""
        return elements // self.block_elems * self.block_bytes

    def span_bytes(self, rows: int, stride: int, row_elems: int) -> int:
        """Bytes touched by `rows` rows of `row_elems` at ELEMENT stride `stride` (GGMLType.java:46-54)."""
        return (rows - 1) * self.row_bytes(stride) + self.row_bytes(row_elems)


_TYPES = [GGMLType("F32", 0, 1, 4), GGMLType("F16", 1, 1, 2), GGMLType("BF16", 30, 1, 2),
          GGMLType("Q4_0", 2, 32, 18), GGMLType("Q8_0", 8, 32, 34), GGMLType("Q4_K", 12, 256, 144),
          GGMLType("Q5_K", 13, 256, 176), GGMLType("Q6_K", 14, 256, 210), GGMLType("MXFP4", 39, 32, 17),
          GGMLType("NVFP4", 40, 64, 36), GGMLType("Q1_0", 41, 128, 18)]
BY_CODE = {t.ggml: t for t in _TYPES}
BY_NAME = {t.name: t for t in _TYPES}


def by_code(code: int) -> GGMLType | None:
    """O(1) code -> type, None for an unknown code (GGMLType.java:57-60)."""
    return BY_CODE.get(code)


# ----------------------------------------------------------------------------------------- quantizers
_F32 = np.float32


def _half(x: np.ndarray) -> np.ndarray:
    """f32 -> fp16 bits (round-to-nearest-even) as uint16."""
    return np.asarray(x, dtype=_F32).astype(np.float16).view(np.uint16)


def _half_val(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=_F32).astype(np.float16).astype(_F32)


def _u16_bytes(h: np.ndarray) -> np.ndarray:
    return h.astype("<u2").view(np.uint8).reshape(*h.shape, 2)


def quantize(dtype: str, x: np.ndarray) -> np.ndarray:
    """[rows, k] float32 -> [rows, row_bytes] uint8 GGUF blocks."""
    x = np.ascontiguousarray(x, dtype=_F32)
    rows, k = x.shape
    t = BY_NAME[dtype]
    nb = k // t.block_elems
    fn = {"Q8_0": _q8_0, "Q4_0": _q4_0, "MXFP4": _mxfp4, "Q4_K": _q4_k, "Q6_K": _q6_k}[dtype]
    out = fn(x.reshape(rows, nb, t.block_elems))
    return np.ascontiguousarray(out.reshape(rows, nb * t.block_bytes))


def _q8_0(x):   # d = amax/127 (fp16 RNE), q = rint(x * (1/d))
    amax = np.max(np.abs(x), axis=-1)
    d = amax / _F32(127)
    with np.errstate(divide="ignore"):
        idd = np.where(d > 0, _F32(1) / d, _F32(0)).astype(_F32)
    q = np.clip(np.rint(x * idd[..., None]), -128, 127).astype(np.int8)
    return np.concatenate([_u16_bytes(_half(d)), q.view(np.uint8)], axis=-1)


def _q4_0(x):   # ggml: signed max mx, d = mx/-8, q = min(15, floor(x/d + 8.5))
    idx = np.argmax(np.abs(x), axis=-1)
    mx = np.take_along_axis(x, idx[..., None], axis=-1)[..., 0]
    d = mx / _F32(-8)
    with np.errstate(divide="ignore"):
        idd = np.where(d != 0, _F32(1) / d, _F32(0)).astype(_F32)
    q = np.clip(np.floor(x * idd[..., None] + _F32(8.5)), 0, 15).astype(np.uint8)
    packed = q[..., :16] | (q[..., 16:] << 4)
    return np.concatenate([_u16_bytes(_half(d)), packed], axis=-1)


_MAG = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=_F32)


def _mxfp4(x):   # e8m0 shared exponent floor(log2 amax) - 2, nearest E2M1 code (ties to the lower)
    am = np.max(np.abs(x), axis=-1)
    with np.errstate(divide="ignore"):
        e = np.where(am > 0, np.clip(np.floor(np.log2(am)).astype(np.int32) - 2 + 127, 1, 254), 127)
    scale = np.ldexp(_F32(1), (e - 127).astype(np.int32)).astype(_F32)
    v = x / scale[..., None]
    a = np.abs(v)
    dist = np.abs(a[..., None] - _MAG)
    best = np.argmin(dist, axis=-1).astype(np.uint8)   # first minimum == the C loop's strict '<'
    code = best | np.where((v < 0) & (best > 0), 8, 0).astype(np.uint8)
    packed = code[..., :16] | (code[..., 16:] << 4)
    return np.concatenate([e.astype(np.uint8)[..., None], packed], axis=-1)


def _q4_k(x):   # 8 sub-blocks (scale, min) under fp16 d/dmin with 6-bit sub-scales
    r, nb = x.shape[:2]
    s = x.reshape(r, nb, 8, 32)
    lo = np.minimum(np.min(s, axis=-1), _F32(0))
    hi = np.max(s, axis=-1)
    sub_s = ((hi - lo) / _F32(15)).astype(_F32)
    sub_m = (-lo).astype(_F32)
    ms, mm = np.max(sub_s, axis=-1), np.max(sub_m, axis=-1)
    dh, mh = ms / _F32(63), mm / _F32(63)
    d, dmin = _half_val(dh), _half_val(mh)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[..., None] > 0, np.clip(np.rint(sub_s / d[..., None]), 0, 63), 0).astype(np.int32)
        mn = np.where(dmin[..., None] > 0, np.clip(np.rint(sub_m / dmin[..., None]), 0, 63), 0).astype(np.int32)
        ds = (d[..., None] * sc.astype(_F32)).astype(_F32)
        mv = (dmin[..., None] * mn.astype(_F32)).astype(_F32)
        q = np.where(ds[..., None] > 0, np.clip(np.rint((s + mv[..., None]) / ds[..., None]), 0, 15), 0)
    q = q.astype(np.uint8)                                   # [r, nb, 8, 32]
    qs = q[:, :, 0::2, :] | (q[:, :, 1::2, :] << 4)          # [r, nb, 4, 32]: byte e of group g
    b = np.zeros((r, nb, 12), np.uint8)
    b[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    b[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    b[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
    return np.concatenate([_u16_bytes(_half(dh)), _u16_bytes(_half(mh)), b, qs.reshape(r, nb, 128)], axis=-1)


def _q6_k(x):   # 16 sub-blocks of 16: int8 sub-scale under fp16 d; codes q + 32 in 0..63
    r, nb = x.shape[:2]
    s = x.reshape(r, nb, 16, 16)
    sub = (np.max(np.abs(s), axis=-1) / _F32(31)).astype(_F32)
    ms = np.max(sub, axis=-1)
    dh = ms / _F32(127)
    d = _half_val(dh)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[..., None] > 0, np.clip(np.rint(sub / d[..., None]), -128, 127), 0).astype(np.int32)
        ds = (d[..., None] * sc.astype(_F32)).astype(_F32)
        q = np.where(ds[..., None] != 0, np.clip(np.rint(s / ds[..., None]), -32, 31), 0).astype(np.int32)
    u = (q + 32).reshape(r, nb, 2, 4, 32)                    # [h, j, l]
    lo4, hi2 = (u & 15).astype(np.uint8), (u >> 4).astype(np.uint8)
    ql = np.zeros((r, nb, 2, 64), np.uint8)
    ql[..., 0:32] = lo4[:, :, :, 0, :] | (lo4[:, :, :, 2, :] << 4)
    ql[..., 32:64] = lo4[:, :, :, 1, :] | (lo4[:, :, :, 3, :] << 4)
    qh = hi2[:, :, :, 0, :] | (hi2[:, :, :, 1, :] << 2) | (hi2[:, :, :, 2, :] << 4) | (hi2[:, :, :, 3, :] << 6)
    return np.concatenate([ql.reshape(r, nb, 128), qh.reshape(r, nb, 64), sc.astype(np.int8).view(np.uint8),
                           _u16_bytes(_half(dh))], axis=-1)
