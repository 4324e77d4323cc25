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


# ------------------------------------------------------------------ jinfer's Vector API arithmetic
def test_fma32_is_one_rounding():
    """fma32 against exact rational arithmetic, operands spread over 60 binades (so a*b + c often needs more
    than double's 53 bits), and an exact tie that rounds to even."""
    from fractions import Fraction
    rng = np.random.default_rng(8)
    a = rng.standard_normal(3000).astype(np.float32)
    b = rng.standard_normal(3000).astype(np.float32)
    c = (rng.standard_normal(3000) * np.exp2(rng.integers(-30, 30, 3000))).astype(np.float32)
    r = E.fma32(a, b, c)
    for i in range(3000):
        ex = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        f = np.float32(float(ex))
        cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
        best = min(cands, key=lambda v: (abs(Fraction(float(v)) - ex), int(np.array(v).view(np.int32)) & 1))
        assert best == r[i], i
    # 1 + 2^-22 + 2^-24 is the midpoint of 1 + 2^-22 and 1 + 3*2^-23: to even
    one = np.float32(1 + 2.0 ** -23)
    assert E.fma32(one, one, np.float32(2.0 ** -24 - 2.0 ** -46)) == np.float32(1 + 2.0 ** -22)


def test_tanh_approx_pinned():
    """Ops.tanhApprox: within 2e-5 of tanh everywhere (the reference's stated ~1.9e-5), odd bit for bit away
    from zero (at +-0 the final fma's sum gives +0 both ways, as IEEE says), constant beyond the cutoff,
    non-decreasing to within 2e-6 (f32 rounding makes dips of ~20 ulps past |x| = 5), tanh(0) = 0, NaN in -> NaN out. A wrong coefficient, sign or
    dropped term breaks the error bound."""
    x = np.linspace(-12, 12, 200001, dtype=np.float32)
    t = E.tanh_approx(x)
    assert np.abs(t.astype(np.float64) - np.tanh(x.astype(np.float64))).max() <= 2e-5
    nz = x != 0
    assert np.array_equal(E.tanh_approx(-x[nz]).view(np.int32), (-t[nz]).view(np.int32))
    assert E.tanh_approx(np.float32([-0.0])).view(np.int32)[0] == 0
    assert (np.diff(t) >= -2e-6).all()
    far = x[np.abs(x) >= E.TANH_CUTOFF]
    assert (E.tanh_approx(far) == np.where(far > 0, E.tanh_approx(E.TANH_CUTOFF), -E.tanh_approx(E.TANH_CUTOFF))).all()
    assert E.tanh_approx(np.float32([0.0]))[0] == 0.0 and np.isnan(E.tanh_approx(np.float32([np.nan]))[0])


def test_vector_glu_forms():
    """SwiGLU's vector body stays within 4e-5 of silu(g)*u (relative to |g*u|), and the elements past the
    loop bound are the full-scalar form bit for bit; gpt-oss's vector form equals clampedSwigluApprox on
    every element and is within 4e-5 of the exact clamped SwiGLU (relative to |x|*|y+1|), keeps the
    saturation points (gate above 7 = gate 7; up beyond +-7 clamped), and is exactly zero at up = -1."""
    rng = np.random.default_rng(12)
    g = rng.uniform(-15, 15, (4, 37)).astype(np.float32)
    u = rng.uniform(-3, 3, (4, 37)).astype(np.float32)
    v = E.silu_mul_vector(g, u, 16)
    assert np.array_equal(v[:, 32:].view(np.int32), E.silu_mul(g[:, 32:], u[:, 32:]).view(np.int32))
    ex = E.silu_mul(g, u).astype(np.float64)
    assert (np.abs(v[:, :32] - ex[:, :32]) <= 4e-5 * np.abs(g[:, :32] * u[:, :32]).astype(np.float64) + 1e-30).all()
    assert not np.array_equal(v[:, :32], ex[:, :32].astype(np.float32))   # the approximation is really used
    gu = rng.uniform(-12, 12, (3, 40)).astype(np.float32)
    uu = rng.uniform(-12, 12, (3, 40)).astype(np.float32)
    c = E.clamped_swiglu_vector(gu, uu, 8)
    assert np.array_equal(c.view(np.int32), E.clamped_swiglu_approx(gu, uu).view(np.int32))
    xx = np.minimum(gu, 7.0).astype(np.float64)
    yy = np.clip(uu, -7.0, 7.0).astype(np.float64)
    assert (np.abs(c - E.clamped_swiglu(gu, uu)) <= 4e-5 * np.abs(xx) * np.abs(yy + 1) + 1e-30).all()
    assert E.clamped_swiglu_approx(np.float32([9.0]), np.float32([2.0]))[0] == \
        E.clamped_swiglu_approx(np.float32([7.0]), np.float32([2.0]))[0]
    assert E.clamped_swiglu_approx(np.float32([1.0]), np.float32([30.0]))[0] == \
        E.clamped_swiglu_approx(np.float32([1.0]), np.float32([7.0]))[0]
    assert E.clamped_swiglu_approx(np.float32([3.0]), np.float32([-1.0]))[0] == 0.0
