"""CPU restatement of the ops jinfer runs right after ``MatMul.gemm``. TEST INFRASTRUCTURE ONLY.

* ``add_row_bias``  -- ``Ops.addRowBiasInPlace`` (jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/
  kernels/Ops.java:375-400): ``x[r][c] += bias[c]`` in f32;
* ``add_in_place``  -- ``Ops.addInPlace`` (Ops.java:326-360): ``x[i] += y[i]`` in f32 (the residual add);
* ``silu_mul``      -- the full-scalar SwiGLU of ``Ops.siluMultiplyInPlace`` (Ops.java:578-583):
  ``(float) (g / (1.0 + Math.exp(-g)) * u)``, the arithmetic in double;
* ``clamped_swiglu`` -- gpt-oss's ``Activations.clampedSwiglu`` (Activations.java:183-187):
  ``x = min(g, 7f)``, ``y = clamp(u, -7f, 7f)``, ``(float) (x / (1.0 + Math.exp(1.702f * -x)) * (y + 1.0))``
  with ``1.702f * -x`` a float product.

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
