"""CPU restatement of the ops jinfer runs right after ``MatMul.gemm``. TEST INFRASTRUCTURE ONLY.

* ``add_row_bias``  -- ``Ops.addRowBiasInPlace`` (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
  kernels/Ops.java:375-400): ``x[r][c] += bias[c]`` in f32;
* ``add_in_place``  -- ``Ops.addInPlace`` (Ops.java:326-360): ``x[i] += y[i]`` in f32 (the residual add);
* ``silu_mul``      -- the full-scalar SwiGLU of ``Ops.siluMultiplyInPlace`` (Ops.java:578-583):
  ``(float) (g / (1.0 + Math.exp(-g)) * u)``, the arithmetic in double;
* ``clamped_swiglu`` -- gpt-oss's ``Activations.clampedSwiglu`` (Activations.java:183-187):
  ``x = min(g, 7f)``, ``y = clamp(u, -7f, 7f)``, ``(float) (x / (1.0 + Math.exp(1.702f * -x)) * (y + 1.0))``
  with ``1.702f * -x`` a float product;
* ``tanh_approx``   -- ``Ops.tanhApprox`` (Ops.java:620-663): njuffa's minimax rational tanh on f32 with
  fused multiply-adds, the scalar twin of the Vector API's ``tanhVec``;
* ``silu_mul_vector`` / ``clamped_swiglu_vector`` -- jinfer's default (Vector API) forms of the two gated
  activations: per row, the first ``cols - cols % lanes`` elements take the vector body (Ops.java:540-563:
  ``g * (tanh(g/2)*0.5 + 0.5) * u``; Activations.java:209-224: ``x*0.5 * (tanh(0.851x) + 1) * (y + 1)``),
  the remainder the loop's scalar tail (SwiGLU: the double formula above; gpt-oss: clampedSwigluApprox,
  Activations.java:189-194), ``lanes`` being the species length (8 on AVX2, 16 on AVX-512).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import this module.
"""
from __future__ import annotations

import numpy as np


def add_row_bias(x: np.ndarray, bias: np.ndarray) -> np.ndarray:
    return (x.astype(np.float32) + bias.astype(np.float32)[None, :]).astype(np.float32)


def add_in_place(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    return (x.astype(np.float32) + y.astype(np.float32)).astype(np.float32)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    gd = g.astype(np.float64)
    with np.errstate(over="ignore"):
        return (gd / (1.0 + np.exp(-gd)) * u.astype(np.float64)).astype(np.float32)


def clamped_swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = g.astype(np.float32)
    u = u.astype(np.float32)
    x = np.where(g > np.float32(7.0), np.float32(7.0), g)                       # Math.min(g, 7f), NaN kept
    y = np.where(u < np.float32(-7.0), np.float32(-7.0), np.where(u > np.float32(7.0), np.float32(7.0), u))
    t = (np.float32(1.702) * -x).astype(np.float32).astype(np.float64)        # float product, then double
    with np.errstate(over="ignore"):
        return (x.astype(np.float64) / (1.0 + np.exp(t)) * (y.astype(np.float64) + 1.0)).astype(np.float32)


def fma32(a, b, c) -> np.ndarray:
    """f32 fused multiply-add with one rounding: a*b is exact in double (24 + 24 bits); s = a*b + c rounded to
    double, e its exact error (TwoSum). s rounded to f32 is the correctly rounded a*b + c except when s sits
    exactly on the midpoint of two f32 values, where the sign of e picks the side (e = 0: the tie, to even)."""
    a, b, c = (np.asarray(v, np.float32).astype(np.float64) for v in (a, b, c))
    p = a * b
    s = p + c
    bb = s - p
    e = (p - (s - bb)) + (c - bb)
    r = s.astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        rd = r.astype(np.float64)
        lo = np.where(rd > s, np.nextafter(r, np.float32(-np.inf)), r).astype(np.float64)
        hi = np.where(rd < s, np.nextafter(r, np.float32(np.inf)), r).astype(np.float64)
        mid = (lo + hi) / 2
        tie = (lo != hi) & (s == mid)
        r = np.where(tie & (e > 0), hi.astype(np.float32), np.where(tie & (e < 0), lo.astype(np.float32), r))
    return r.astype(np.float32)


TANH_CUTOFF = np.float32(5.76110792)
TANH_N0, TANH_N1, TANH_N2 = np.float32(-1.60153955e-4), np.float32(-9.34448242e-1), np.float32(-2.19176636e+1)
TANH_D0, TANH_D1 = np.float32(29.0915985), np.float32(65.7667847)


def _jmax(a, b):   # Math.max on floats: NaN if either is NaN
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.where(np.isnan(a) | np.isnan(b), np.float32(np.nan), np.maximum(a, b)).astype(np.float32)


def _jmin(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.where(np.isnan(a) | np.isnan(b), np.float32(np.nan), np.minimum(a, b)).astype(np.float32)


def tanh_approx(x) -> np.ndarray:
    y = _jmax(-TANH_CUTOFF, _jmin(TANH_CUTOFF, x))
    y2 = (y * y).astype(np.float32)
    num = (fma32(fma32(TANH_N0, y2, TANH_N1), y2, TANH_N2) * y2).astype(np.float32)
    den = fma32((y2 + TANH_D0).astype(np.float32), y2, TANH_D1)
    with np.errstate(invalid="ignore"):
        q = (num / den).astype(np.float32)
    return fma32(q, y, y)


def _silu_vec_body(g, u):
    g, u = np.asarray(g, np.float32), np.asarray(u, np.float32)
    t = tanh_approx((g * np.float32(0.5)).astype(np.float32))       # clamp inside: max(-C).min(C)
    s = ((t * np.float32(0.5)).astype(np.float32) + np.float32(0.5)).astype(np.float32)
    return ((g * s).astype(np.float32) * u).astype(np.float32)


def clamped_swiglu_approx(g, u) -> np.ndarray:
    """The vector body and Activations.clampedSwigluApprox alike: x*0.5 * (1 + tanhApprox(0.851x)) * (y + 1)."""
    x = _jmin(g, np.float32(7.0))
    y = _jmin(_jmax(u, np.float32(-7.0)), np.float32(7.0))
    t = tanh_approx((x * np.float32(0.851)).astype(np.float32))
    a = ((x * np.float32(0.5)).astype(np.float32) * (np.float32(1.0) + t).astype(np.float32)).astype(np.float32)
    return (a * (y + np.float32(1.0)).astype(np.float32)).astype(np.float32)


def _by_lanes(g, u, lanes, body, tail):
    g, u = np.asarray(g, np.float32), np.asarray(u, np.float32)
    cols = g.shape[-1]
    bound = cols - cols % lanes
    out = np.empty_like(g)
    out[..., :bound] = body(g[..., :bound], u[..., :bound])
    out[..., bound:] = tail(g[..., bound:], u[..., bound:])
    return out


def silu_mul_vector(g, u, lanes: int) -> np.ndarray:
    return _by_lanes(g, u, lanes, _silu_vec_body, silu_mul)


def clamped_swiglu_vector(g, u, lanes: int) -> np.ndarray:
    return _by_lanes(g, u, lanes, clamped_swiglu_approx, clamped_swiglu_approx)
