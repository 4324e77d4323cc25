"""GPU: the opt-in native-MX path for MXFP4 weights (jamhip_ctx_set_mx_native).

The scaled fp4 x fp8 MFMA against oracle/mxnative.py: the same MX-FP8 activation values and jam's MXFP4
weight values multiplied in f64, within 2^-13·Σ|w·x~| (TOL_MFMA): the hardware's scaled block dot is not
exact, its results move in steps of about 2^-16 at unit magnitude (measured on MI355X, both modes alike),
and the bound leaves 8x over that while still catching systematic layout, code or scale errors. Against the
f64 product of
the unquantized activations the mode's own tolerance applies (mode 1: 5e-3·Σ|w·a|, mode 2: 5e-2·Σ|w·a|),
and the observed error is reported beside jam's int8 result. Decode-sized calls keep jam's semantics.
"""
import sys

import numpy as np
import pytest

from oracle import mxnative as X
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL_MFMA = 2.0 ** -13


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def acts(seed, n, k, outliers=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k)).astype(np.float32)
    if outliers:
        hit = rng.random((n, k)) < 0.01
        x[hit] = np.where(rng.random(int(hit.sum())) < 0.5, -20.0, 20.0).astype(np.float32)
    return x


def run(hip, w, a, m, n, k):
    from qxotic_amd.jam import JAM, Segment
    c = np.zeros((n, m), np.float32)
    st = hip.mm(Segment.of(w), 0, JAM.MXFP4, k, Segment.of(a), 0, JAM.F32, k, Segment.of(c), 0, JAM.F32, m, m, n, k)
    assert st == JAM.OK, hip.last_error()
    return c


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("m,k,n", [(128, 2880, 64), (256, 1024, 100), (512, 2880, 37), (96, 4096, 512), (64, 6176, 40)])
def test_mx_native_matches_restatement(hip, oracle, mode, m, k, n):
    say(f"mx native mode={mode} m={m} k={k} n={n}")
    w = oracle.quantize(O.MXFP4, oracle.normal(7 + m, (m, k), 0.0, 0.02))
    a = acts(8 + n, n, k)
    wd = oracle.dequant(O.MXFP4, w, k, f64=True)
    assert hip.set_mx_native(mode) == 0
    try:
        c = run(hip, w, a, m, n, k)
    finally:
        assert hip.set_mx_native(0) == 0
    ref, sref = X.mm(wd, a, mode)
    err = np.abs(c - ref)
    say(f"  max |c - restatement| / sum|w.x~| = {float((err / sref).max()):.3g}")
    assert (err <= TOL_MFMA * sref + 1e-30).all(), f"max err / sum {float((err / sref).max()):.3g}"
    # the mode's own tolerance against the unquantized f64 product, and jam's int8 result for scale
    exact = a.astype(np.float64) @ wd.T
    sa = np.abs(a.astype(np.float64)) @ np.abs(wd).T
    rel = float((np.abs(c - exact) / sa).max())
    jam = oracle.mm_int8(O.MXFP4, w, a, m, n, k)
    rel_jam = float((np.abs(jam - exact) / sa).max())
    say(f"  max |c - exact| / sum|w.a| = {rel:.3g} (jam int8: {rel_jam:.3g})")
    assert rel <= (5e-3 if mode == 1 else 5e-2)


def test_mx_native_keeps_decode_semantics(hip, oracle):
    """Calls below the matrix-core threshold (n < 8) are jam's F1 path whether the mode is on or off."""
    m, k = 128, 2880
    w = oracle.quantize(O.MXFP4, oracle.normal(17, (m, k), 0.0, 0.02))
    for n in (1, 3, 7):
        a = acts(18 + n, n, k)
        off = run(hip, w, a, m, n, k)
        assert hip.set_mx_native(1) == 0
        try:
            on = run(hip, w, a, m, n, k)
        finally:
            hip.set_mx_native(0)
        assert np.array_equal(on.view(np.uint32), off.view(np.uint32))


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("E", [7, 24])
def test_mx_native_grouped(hip, oracle, mode, E):
    """jamhip_mm_grouped under the mode. With rows_cap >= 8·n_experts (E = 7: 135 rows) one fused prep derives
    the expert table from the device counts and every expert runs on the native path, those below 8 rows
    included; sparser calls (E = 24) keep jam's F1 path for experts below 8 rows. Each native expert against
    the restatement, each F1 expert against the int8 oracle, rows past the prefix untouched."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, k = 64, 576
    counts = np.zeros(E, np.int32)
    counts[:7] = [3, 0, 12, 70, 1, 9, 40]
    R = int(counts.sum())
    w = oracle.quantize(O.MXFP4, oracle.normal(27, (E * m, k), 0.0, 0.02))
    a = acts(28, R, k)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    counts_d, a_d = dev(counts), dev(a)
    c = torch.full((R, m), 7.0, dtype=torch.float32, device="cuda")
    offs = torch.full((E + 1,), -5, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()   # the inputs are written on torch's stream; the library runs on its own
    assert hip.set_mx_native(mode) == 0
    try:
        st = hip.mm_grouped(Segment.of(w), JAM.MXFP4, k, m, E, counts_d.data_ptr(), a_d.data_ptr(), k,
                            c.data_ptr(), m, k, R, offs.data_ptr())
        torch.cuda.synchronize()
    finally:
        hip.set_mx_native(0)
    assert st == JAM.OK, hip.last_error()
    got = c.cpu().numpy()
    off = np.concatenate([[0], np.cumsum(counts)])
    assert np.array_equal(offs.cpu().numpy(), off)
    for e in range(E):
        rows = slice(off[e], off[e + 1])
        if counts[e] == 0:
            continue
        we = w[e * m:(e + 1) * m]
        if counts[e] >= 8 or R >= 8 * E:
            ref, sref = X.mm(oracle.dequant(O.MXFP4, we, k, f64=True), a[rows], mode)
            assert (np.abs(got[rows] - ref) <= TOL_MFMA * sref + 1e-30).all(), f"expert {e}"
        else:
            ref = oracle.mm_int8(O.MXFP4, we, a[rows], m, int(counts[e]), k)
            _, sa = oracle.mm_ref(O.MXFP4, we, a[rows], m, int(counts[e]), k)
            assert (np.abs(got[rows] - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa).all(), f"expert {e}"


@pytest.mark.parametrize("mode,k", [(2, 2880), (1, 6176)])
def test_mx_native_grouped_many_slots(hip, oracle, mode, k):
    """The fused grouped prep with more real slots than its 1024 workgroups (1530 rows over 6 experts, one
    empty and one of a single row), so that workgroups loop over several slots with the next slot's loads
    issued ahead; k = 6176 (193 blocks) takes two passes per row, the second one partial. Every expert against
    the restatement, the offsets and rows past the prefix untouched."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    say(f"mx native grouped many slots mode={mode} k={k}")
    m, E = 32, 6
    counts = np.array([700, 0, 1, 300, 9, 520], np.int32)
    R = int(counts.sum())
    w = oracle.quantize(O.MXFP4, oracle.normal(37 + k, (E * m, k), 0.0, 0.02))
    a = acts(38 + k, R, k)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    counts_d, a_d = dev(counts), dev(a)
    c = torch.full((R + 3, m), 7.0, dtype=torch.float32, device="cuda")
    offs = torch.full((E + 1,), -5, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    assert hip.set_mx_native(mode) == 0
    try:
        st = hip.mm_grouped(Segment.of(w), JAM.MXFP4, k, m, E, counts_d.data_ptr(), a_d.data_ptr(), k,
                            c.data_ptr(), m, k, R, offs.data_ptr())
        torch.cuda.synchronize()
    finally:
        hip.set_mx_native(0)
    assert st == JAM.OK, hip.last_error()
    got = c.cpu().numpy()
    off = np.concatenate([[0], np.cumsum(counts)])
    assert np.array_equal(offs.cpu().numpy(), off)
    assert (got[R:] == 7.0).all()
    for e in range(E):
        if counts[e] == 0:
            continue
        rows = slice(off[e], off[e + 1])
        ref, sref = X.mm(oracle.dequant(O.MXFP4, w[e * m:(e + 1) * m], k, f64=True), a[rows], mode)
        assert (np.abs(got[rows] - ref) <= TOL_MFMA * sref + 1e-30).all(), f"expert {e}"
