"""Pins the test oracle (oracle/jam_oracle.c) before anything is checked against it.

Each oracle function is checked against something independent of its own formula: numpy's IEEE
conversions, closed forms, the reference's own libjam (compiled from its sources into oracle/_ref), and
the committed fixtures that libjam produced (tests/golden/jam_golden.npz).
"""
from pathlib import Path

import numpy as np
import pytest

from conftest import adversarial_activations
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "jam_golden.npz"


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


# ---------------------------------------------------------------------------------- scalar formats
def test_half2float_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.lib.jo_half2float(int(c)) for c in codes], np.float32)
    want = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_float2half_rne(oracle):
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000).astype(np.float32),
                         np.array([0.0, -0.0, 65504, 65519.9, 65520, 1e-8, 6e-8, 5.96e-8, 2.98e-8, 3e-8, np.inf, -np.inf],
                                  np.float32)])
    got = np.array([oracle.lib.jo_float2half(float(x)) for x in xs], np.uint16)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_e8m0_closed_form(oracle):
    for e in range(256):
        v = oracle.lib.jo_e8m0_half(e)
        want = np.inf if e == 255 else float(np.ldexp(1.0, e - 128))
        assert v == np.float32(want), e


# ---------------------------------------------------------------------------- activation quantizers
def test_quant_closed_forms(oracle):
    x = adversarial_activations(256)
    q, d, s = oracle.quant_f1(x)
    assert (q[0] == 0).all() and (d[0] == 0).all() and (s[0] == 0).all()      # zero block
    assert (q[1] == 127).all() and np.allclose(d[1], np.float32(0.75) / np.float32(127))
    assert (q[2] == -127).all()
    # amax 127 -> d = 1, id = 1: round-half-even on the exact ties
    row = q[4][:8].tolist()
    assert row == [127, 2, -2, 4, 0, 0, 2, -126]
    assert (s[1] == 127 * 32).all()
    q2, d2, s2 = oracle.quant_f2(x)
    assert q2[4][:8].tolist() == [127, 2, -2, 4, 0, 0, 2, -126]
    # F2 sums: exact for small integers
    assert s2[1][0] == np.float32(0.75 * 16)


def test_quant_matches_golden(oracle):
    g = np.load(GOLDEN)
    act = g["act"]
    q, d, s = oracle.quant_f1(act)
    assert np.array_equal(q, g["f1_q"]) and np.array_equal(bits(d), bits(g["f1_d"])) and np.array_equal(s, g["f1_s"])
    q, d, s = oracle.quant_f2(act)
    assert np.array_equal(q, g["f2_q"]) and np.array_equal(bits(d), bits(g["f2_d"]))
    assert np.array_equal(bits(s), bits(g["f2_s"]))


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_quant_matches_libjam(oracle, refjam, seed):
    x = np.concatenate([oracle.outliers(seed, (24, 4096)), adversarial_activations(4096)])
    for ours, theirs in ((oracle.quant_f1, refjam.quant_f1), (oracle.quant_f2, refjam.quant_f2)):
        q, d, s = ours(x)
        qr, dr, sr = theirs(x)
        assert np.array_equal(q, qr)
        assert np.array_equal(bits(d), bits(dr))
        assert np.array_equal(bits(s), bits(sr))


# ----------------------------------------------------------------------------------- dequantization
@pytest.mark.parametrize("dt", O.QUANT_TYPES)
def test_dequant_matches_libjam_float_floor(oracle, refjam_generic, dt):
    """One-hot activations through libjam's portable float floor return single weight columns exactly
    (jam_kernels_generic.c: a float dot with one non-zero term)."""
    m, k = 24, 512
    w = oracle.quantize(dt, oracle.normal(40 + dt, (m, k), 0.0, 0.02))
    deq = oracle.dequant(dt, w, k)
    for t in (0, 1, 17, 31, 32, 255, 256, 300, 511):
        a = np.zeros((1, k), np.float32)
        a[0, t] = 1.0
        col = refjam_generic.mm(dt, w, a, m, 1, k)[0]
        assert np.array_equal(col, deq[:, t]), (O.NAMES[dt], t)   # values (+0 and -0 agree)


def test_dequant_exact_value_blocks(oracle):
    """Hand-built blocks with unit scales: values are the integer codes (QuantWeights.java:108-289)."""
    k = 256
    # Q4_K: d = dmin = 1.0, sub-scales sc = s+1, mins mn = s -> value = (s+1)*nib - s
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    blk[2:4] = blk[0:2]
    sc = np.arange(1, 9)
    mn = np.arange(0, 8)
    b = blk[4:16]
    b[0:4] = (sc[0:4] & 63) | ((sc[4:8] >> 4) << 6)
    b[4:8] = (mn[0:4] & 63) | ((mn[4:8] >> 4) << 6)
    b[8:12] = (sc[4:8] & 15) | ((mn[4:8] & 15) << 4)
    nib = (np.arange(256) * 7) % 16
    for g in range(4):
        blk[16 + 32 * g: 48 + 32 * g] = nib[64 * g: 64 * g + 32] | (nib[64 * g + 32: 64 * g + 64] << 4)
    want = np.array([sc[e // 32] * nib[e] - mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(oracle.dequant(O.Q4_K, blk, k)[0], want)
    # Q6_K: d = 1, scales 1..16 -> value = sc[e // 16] * (code - 32)
    blk = np.zeros(210, np.uint8)
    blk[208:210] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    blk[192:208] = np.arange(1, 17)
    code = (np.arange(256) * 5 + 3) % 64
    for e in range(256):
        h, j, l = e // 128, (e % 128) // 32, e % 32
        blk[64 * h + (j & 1) * 32 + l] |= (code[e] & 15) << (4 if j >= 2 else 0)
        blk[128 + 32 * h + l] |= (code[e] >> 4) << (2 * j)
    want = np.array([(e // 16 + 1) * (code[e] - 32) for e in range(256)], np.float32)
    # scale index 8h + 2j + l/16 equals e // 16 for this element order
    assert np.array_equal(oracle.dequant(O.Q6_K, blk, k)[0], want)
    # MXFP4: e = 128 -> scale 1: value = code table (x2 of E2M1)
    blk = np.zeros(17, np.uint8)
    blk[0] = 128
    blk[1:17] = np.arange(16) | ((15 - np.arange(16)) << 4)
    codes = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    want = np.array([codes[e] for e in range(16)] + [codes[15 - e] for e in range(16)], np.float32)
    assert np.array_equal(oracle.dequant(O.MXFP4, blk, 32)[0], want)


# ------------------------------------------------------------------------------------ int8 pipeline
def tol_int8(ref, sumabs):
    """Same int8 semantics, different f32 accumulation order."""
    return 1e-3 * np.abs(ref) + 1e-5 * sumabs


@pytest.mark.parametrize("dt", O.QUANT_TYPES)
def test_int8_pipeline_matches_golden(oracle, dt):
    g = np.load(GOLDEN)
    w, a = g[f"mm_{O.NAMES[dt]}_w"], g["mm_a"]
    m, k = 32, 512
    for n in (1, 3, 7, 8, 13, 16):
        got = oracle.mm_int8(dt, w, a[:n], m, n, k)
        _, sa = oracle.mm_ref(dt, w, a[:n], m, n, k)
        want = g[f"mm_{O.NAMES[dt]}_n{n}"]
        assert (np.abs(got - want) <= tol_int8(got, sa)).all(), (O.NAMES[dt], n)


@pytest.mark.parametrize("dt", O.QUANT_TYPES)
@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 16, 33])
@pytest.mark.parametrize("m", [96, 104, 77])
def test_int8_pipeline_matches_libjam(oracle, refjam, dt, n, m):
    """m % 16 != 0 included: jam's n>=8 bands leave the last m % 16 rows to a float dot."""
    k = 1024
    w = oracle.quantize(dt, oracle.normal(77 + dt, (m, k), 0.0, 0.02))
    a = oracle.outliers(5 + n, (n, k))
    want = refjam.mm(dt, w, a, m, n, k)
    got = oracle.mm_int8(dt, w, a, m, n, k)
    _, sa = oracle.mm_ref(dt, w, a, m, n, k)
    assert (np.abs(got - want) <= tol_int8(got, sa)).all()


def test_tail_rule_is_discriminating(oracle, refjam):
    """The float-dot tail is observable: computing the last m % 16 rows with F2 int8 instead misses
    libjam's answer there by more than the tolerance (outlier activations make the int8 error large)."""
    m, k, n = 104, 1024, 9
    for dt in O.QUANT_TYPES:
        w = oracle.quantize(dt, oracle.normal(31 + dt, (m, k), 0.0, 0.02))
        a = oracle.outliers(32, (n, k))
        want = refjam.mm(dt, w, a, m, n, k)
        all_int8 = oracle.mm_int8(dt, w, a, m, n, k, flavour=2)
        _, sa = oracle.mm_ref(dt, w, a, m, n, k)
        ok = np.abs(all_int8 - want) <= tol_int8(all_int8, sa)
        assert ok[:, :96].all() and not ok[:, 96:].all(), O.NAMES[dt]


def test_int8_flavour_is_discriminating(oracle, refjam):
    """The pins above can tell the two decompositions apart: the n<8 formula applied at n=8 misses
    libjam's answer for Q4_K/Q6_K by far more than the tolerance."""
    m, k, n = 96, 1024, 8
    for dt in (O.Q4_K, O.Q6_K):
        w = oracle.quantize(dt, oracle.normal(9, (m, k), 0.0, 0.02))
        a = oracle.outliers(10, (n, k))
        want = refjam.mm(dt, w, a, m, n, k)
        wrong = oracle.mm_int8(dt, w, a, m, n, k, flavour=1)
        _, sa = oracle.mm_ref(dt, w, a, m, n, k)
        assert not (np.abs(wrong - want) <= tol_int8(wrong, sa)).all()


@pytest.mark.parametrize("dt", O.QUANT_TYPES)
def test_float_reference_matches_libjam_floor(oracle, refjam_generic, dt):
    m, k, n = 40, 512, 3
    w = oracle.quantize(dt, oracle.normal(3 + dt, (m, k), 0.0, 0.02))
    a = oracle.normal(8, (n, k))
    ref, sa = oracle.mm_ref(dt, w, a, m, n, k)
    floor = refjam_generic.mm(dt, w, a, m, n, k)
    assert (np.abs(floor - ref) <= 1e-5 * sa + 1e-7).all()


@pytest.mark.parametrize("dt", O.QUANT_TYPES)
def test_int8_within_precision_bound(oracle, dt):
    """PRECISION.md:20-26: int8-activation paths stay within 1e-2*sumAbs + 1e-3 of the float reference."""
    m, k = 48, 1024
    w = oracle.quantize(dt, oracle.normal(21 + dt, (m, k), 0.0, 0.02))
    for n in (1, 8):
        a = oracle.outliers(22, (n, k))
        got = oracle.mm_int8(dt, w, a, m, n, k)
        ref, sa = oracle.mm_ref(dt, w, a, m, n, k)
        assert (np.abs(got - ref) <= 1e-2 * sa + 1e-3).all()


def test_span_bytes_matches_geometry(oracle):
    from qxotic_amd import ggml
    for code, t in ggml.BY_CODE.items():
        if code in O.BLOCK:
            be, bb = O.BLOCK[code]
            assert (t.block_elems, t.block_bytes) == (be, bb)
            assert oracle.lib.jo_span_bytes(code, 5, 4 * be * 3, 2 * be) == t.span_bytes(5, 4 * be * 3, 2 * be)
