"""Restatement of the opt-in native-MX mode for MXFP4 weights (no counterpart in the reference). TEST
INFRASTRUCTURE ONLY: only tests/ may import it.

The mode keeps jam's MXFP4 weight values (jam/jam-native/src/kernels/jam_mxfp4.h:14-24: kv[nib]·2^(e-128),
kv = 2·e2m1) and replaces jam's int8 activation codes by MX-FP8 (OCP e4m3 with one e8m0 scale per 32-block),
split into hi + lo:
    E  = the smallest integer with max|x_block|·2^-E <= 448, clamped to [-127, 127] (0 blocks: E = -127)
    hi = e4m3(x·2^-E)                 scale byte E + 127
    lo = e4m3((x·2^-E - hi)·16)       scale byte E - 4 + 127 (mode 1; 0 with lo = 0 where E - 4 < -127)
with e4m3() the nearest finite e4m3 value, ties to the even code. The product is then the exact f64 sum of
w·(hi·2^E + lo·2^(E-4)) up to the device's f32 accumulation order.

Pinned (tests/test_mx_oracle.py) by: the e4m3 value table against the format's closed form and its fixed
points (0x7E = 448, 0x08 = 2^-6, 0x01 = 2^-9, 0x38 = 1), encode == brute-force nearest over all 255 finite
codes with exact ties going to the even code, the choice of E (max·2^-E <= 448 < max·2^-(E-1)), and the
hi + lo reconstruction bound |x - x~| <= 2^-5 ulp-of-hi (so 2^-9·max per block at most).
"""
from __future__ import annotations

import numpy as np


def e4m3_values() -> np.ndarray:
    """f64 value of each of the 256 OCP e4m3 (E4M3FN) codes; NaN for 0x7F / 0xFF."""
    c = np.arange(256)
    be, mt = (c >> 3) & 15, c & 7
    mag = np.where(be == 0, mt * 2.0 ** -9, (1.0 + mt / 8.0) * 2.0 ** (be - 7))
    v = np.where(c & 0x80, -mag, mag)
    v[(c & 0x7F) == 0x7F] = np.nan
    return v


_VALS = e4m3_values()
_POS = np.arange(0x7F)                 # the finite non-negative codes, ascending in value
_POSV = _VALS[_POS]


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """Nearest finite e4m3 code of each |v| <= 448, ties to the even code (round to nearest even)."""
    v = np.asarray(v, np.float64)
    a = np.abs(v)
    i = np.clip(np.searchsorted(_POSV, a), 1, len(_POSV) - 1)
    lo_c, hi_c = _POS[i - 1], _POS[i]
    dlo, dhi = a - _POSV[i - 1], _POSV[i] - a
    pick = np.where(dlo < dhi, lo_c, np.where(dhi < dlo, hi_c, np.where(lo_c % 2 == 0, lo_c, hi_c)))
    pick = np.where(a <= 0, 0, pick)
    return (pick | np.where(v < 0, 0x80, 0)).astype(np.uint8)


def block_exponent(amax: np.ndarray) -> np.ndarray:
    """Smallest E with amax·2^-E <= 448 (E = -127 for amax == 0), clamped to [-127, 127]."""
    amax = np.asarray(amax, np.float64)
    with np.errstate(divide="ignore"):
        e = np.ceil(np.log2(np.where(amax > 0, amax, 1.0) / 448.0)).astype(np.int64)
    e = np.where(amax * 2.0 ** (-e.astype(np.float64)) > 448.0, e + 1, e)
    e = np.where((amax * 2.0 ** (-(e - 1).astype(np.float64)) <= 448.0) & (amax > 0), e - 1, e)
    return np.clip(np.where(amax > 0, e, -127), -127, 127)


def quantize(x: np.ndarray, mode: int = 1):
    """MX-FP8 codes of x [n][k] (k a multiple of 32): hi, lo uint8 [n][k]; E int [n][k/32]; lo_on bool."""
    x = np.asarray(x, np.float32).astype(np.float64)
    n, k = x.shape
    xb = x.reshape(n, k // 32, 32)
    amax = np.abs(xb).max(axis=2)
    E = block_exponent(amax)
    v = xb * (2.0 ** (-E.astype(np.float64)))[:, :, None]
    v = v.astype(np.float32).astype(np.float64)          # x·2^-E is exact in f32 (a power-of-two scale)
    hi = e4m3_encode(v)
    lo_on = (mode == 1) & (E - 4 >= -127)
    r = (v - _VALS[hi]) * 16.0
    lo = np.where(lo_on[:, :, None], e4m3_encode(r), 0).astype(np.uint8)
    return hi.reshape(n, k), lo.reshape(n, k), E, lo_on


def dequant_act(x: np.ndarray, mode: int = 1) -> np.ndarray:
    """The activation values the native-MX mode multiplies: hi·2^E + lo·2^(E-4), f64 [n][k]."""
    hi, lo, E, lo_on = quantize(x, mode)
    n, k = hi.shape
    s = 2.0 ** E.astype(np.float64)
    val = _VALS[hi].reshape(n, k // 32, 32) * s[:, :, None]
    val += np.where(lo_on[:, :, None], _VALS[lo].reshape(n, k // 32, 32) * (s / 16.0)[:, :, None], 0.0)
    return val.reshape(n, k)


def mm(w_deq_f64: np.ndarray, x: np.ndarray, mode: int = 1):
    """C [n][m] = W · x~^T in f64 with W the dequantized MXFP4 weights [m][k], and Σ|w·x~| per output."""
    xa = dequant_act(x, mode)
    return xa @ w_deq_f64.T, np.abs(xa) @ np.abs(w_deq_f64).T
