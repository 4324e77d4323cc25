"""The epilogue oracle (oracle/epilogue.py) pinned by identities it does not use: the logistic function
through tanh (sigmoid(x) = (1 + tanh(x/2)) / 2), closed-form values, the saturation points of gpt-oss's
clamps, and the zero of (y + 1)."""
import math

import numpy as np

from oracle import epilogue as E


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def test_silu_mul_against_tanh_form():
    g = np.linspace(-16, 16, 4001, dtype=np.float32)   # 1 + tanh(x/2) stays well-conditioned here
    u = np.float32(1.0) + np.zeros_like(g)
    via_tanh = (g.astype(np.float64) * 0.5 * (1.0 + np.tanh(g.astype(np.float64) / 2))).astype(np.float32)
    assert ulps(E.silu_mul(g, u), via_tanh).max() <= 1
    gn = np.linspace(-80, 0, 4001, dtype=np.float32)    # negative tail: sigmoid(x) = e^x / (1 + e^x)
    en = np.exp(gn.astype(np.float64))
    assert ulps(E.silu_mul(gn, np.ones_like(gn)), (gn * en / (1.0 + en)).astype(np.float32)).max() <= 1
    # linear in up, and closed forms
    u3 = np.full_like(g, 3.0)
    assert np.allclose(E.silu_mul(g, u3), 3.0 * E.silu_mul(g, u), rtol=1e-6, atol=0)
    assert E.silu_mul(np.float32([0.0]), np.float32([5.0]))[0] == 0.0
    assert E.silu_mul(np.float32([1.0]), np.float32([1.0]))[0] == np.float32(1.0 / (1.0 + math.exp(-1.0)))
    assert E.silu_mul(np.float32([-100.0]), np.float32([1.0]))[0] == np.float32(-100.0 * math.exp(-100.0) / (1 + math.exp(-100.0)))


def test_clamped_swiglu_identities():
    rng = np.random.default_rng(3)
    g = rng.uniform(-12, 12, 5000).astype(np.float32)
    u = rng.uniform(-12, 12, 5000).astype(np.float32)
    out = E.clamped_swiglu(g, u)
    # quickgelu(x) = x * sigmoid(1.702x), sigmoid through tanh; (y + 1) with y clamped
    x = np.minimum(g, 7.0).astype(np.float64)
    y = np.clip(u, -7.0, 7.0).astype(np.float64)
    ref = x * 0.5 * (1.0 + np.tanh(0.851 * x)) * (y + 1.0)
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-30)
    # gate saturates at 7 (not below), up at +-7; y = -1 gives exactly 0
    assert (E.clamped_swiglu(np.float32([7.0, 9.0, 1e30]), np.float32([2.0] * 3)) ==
            E.clamped_swiglu(np.float32([7.0] * 3), np.float32([2.0] * 3))).all()
    assert E.clamped_swiglu(np.float32([-9.0]), np.float32([0.0]))[0] != E.clamped_swiglu(np.float32([-7.0]), np.float32([0.0]))[0]
    assert (E.clamped_swiglu(np.float32([3.0] * 3), np.float32([7.0, 8.0, 1e9])) == E.clamped_swiglu(np.float32([3.0]), np.float32([7.0]))[0]).all()
    assert (E.clamped_swiglu(np.float32([3.0] * 2), np.float32([-7.0, -50.0])) == E.clamped_swiglu(np.float32([3.0]), np.float32([-7.0]))[0]).all()
    assert E.clamped_swiglu(np.float32([2.5]), np.float32([-1.0]))[0] == 0.0
    # closed form at one point: 7 / (1 + e^(-1.702*7)) * 8 with 1.702f*7 a float product
    t = float(np.float32(1.702) * np.float32(-7.0))
    assert E.clamped_swiglu(np.float32([7.0]), np.float32([7.0]))[0] == np.float32(7.0 / (1.0 + math.exp(t)) * 8.0)
    # NaN propagates as in Math.min / Math.clamp
    assert np.isnan(E.clamped_swiglu(np.float32([np.nan]), np.float32([1.0]))[0])
    assert np.isnan(E.clamped_swiglu(np.float32([1.0]), np.float32([np.nan]))[0])


def test_bias_and_residual_order():
    x = np.float32([[1e8, 1.0]])
    b = np.float32([1.0, 2.0])
    r = E.add_row_bias(x, b)
    assert r.dtype == np.float32 and r[0, 0] == np.float32(1e8) and r[0, 1] == 3.0   # f32 rounding, not f64
    assert (E.add_in_place(np.float32([0.1]), np.float32([0.2])) == np.float32(0.1) + np.float32(0.2)).all()
