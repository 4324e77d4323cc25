"""Pins of the oracle's restatement for jam's remaining dtypes (Q5_K, NVFP4, Q1_0 and the dense F32 / F16 /
BF16 paths) against libjam built from the reference sources (oracle/_ref), closed forms and exact-value
blocks. CPU only.

What each check fixes:
* dequantization: libjam's portable float floor with one-hot activations returns single weight columns;
  hand-built blocks whose values are integer closed forms;
* UE4M3 (NVFP4's per-16 scale): all 256 codes through libjam's NVFP4 floor;
* the int8 pipelines: libjam's jam_mm at n in {1..33} and m % 16 != 0 (F1 kernels, F2 bands, float-dot
  tails); the n < 8 decomposition applied at n = 8 and the all-int8 tail both miss libjam (the pins can
  tell them apart);
* the dense paths: libjam's jam_mm within 1e-6·sum|w·a| (only f32 summation order differs), including
  BF16's activation rounding rule, which the same check without rounding misses by 200x.
"""
import numpy as np
import pytest

from oracle import oracle as O


def tol_int8(ref, sumabs):
    return 1e-3 * np.abs(ref) + 1e-5 * sumabs


@pytest.mark.parametrize("dt", O.NEW_QUANT_TYPES + O.DENSE_TYPES)
def test_dequant_matches_libjam_float_floor(oracle, refjam_generic, dt):
    m, k = 24, 512
    w = oracle.quantize(dt, oracle.normal(40 + dt, (m, k), 0.0, 0.02))
    deq = oracle.dequant(dt, w, k)
    for t in (0, 1, 7, 8, 15, 16, 17, 31, 32, 63, 64, 127, 128, 255, 256, 300, 511):
        a = np.zeros((1, k), np.float32)
        a[0, t] = 1.0
        col = refjam_generic.mm(dt, w, a, m, 1, k)[0]
        assert np.array_equal(col, deq[:, t]), (O.NAMES[dt], t)


def test_ue4m3_all_codes_against_libjam(oracle, refjam_generic):
    """Block s of row r carries d[s] = code 4r + s and nibble 2 (kv = 2) everywhere: the one-hot column of
    element 16s is 2·ue4m3(code), for all 256 codes (0x00 and 0x7F read 0, bit 7 ignored otherwise)."""
    m, k = 64, 64
    w = np.zeros((m, 36), np.uint8)
    for r in range(m):
        w[r, 0:4] = [4 * r + s for s in range(4)]
        w[r, 4:36] = 0x22
    for s in range(4):
        a = np.zeros((1, k), np.float32)
        a[0, 16 * s] = 1.0
        col = refjam_generic.mm(O.NVFP4, w, a, m, 1, k)[0]
        want = np.array([2.0 * oracle.lib.jo_ue4m3(4 * r + s) for r in range(m)], np.float32)
        assert np.array_equal(col, want), s
    assert oracle.lib.jo_ue4m3(0x7F) == 0.0 and oracle.lib.jo_ue4m3(0) == 0.0
    assert oracle.lib.jo_ue4m3(0x38) == 1.0 and oracle.lib.jo_ue4m3(0x7E) == 448.0 and oracle.lib.jo_ue4m3(1) == 2.0 ** -9


def test_dequant_exact_value_blocks(oracle):
    # Q5_K: d = dmin = 1, sc = s + 1, mn = s, 5-bit codes q -> (s + 1)·q - s
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    blk[2:4] = blk[0:2]
    sc, mn = np.arange(1, 9), np.arange(0, 8)
    b = blk[4:16]
    b[0:4] = (sc[0:4] & 63) | ((sc[4:8] >> 4) << 6)
    b[4:8] = (mn[0:4] & 63) | ((mn[4:8] >> 4) << 6)
    b[8:12] = (sc[4:8] & 15) | ((mn[4:8] & 15) << 4)
    q5 = (np.arange(256) * 11 + 5) % 32
    for e in range(256):
        s, l = e // 32, e % 32
        blk[48 + 32 * (s // 2) + l] |= (q5[e] & 15) << (4 if s & 1 else 0)
        blk[16 + l] |= (q5[e] >> 4) << s
    want = np.array([sc[e // 32] * q5[e] - mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(oracle.dequant(O.Q5_K, blk, 256)[0], want)
    # NVFP4: ue4m3 0x38 = 1.0: values are the code table; sub-block s byte s*8+j: low -> 16s+j, high -> 16s+8+j
    blk = np.zeros(36, np.uint8)
    blk[0:4] = 0x38
    codes = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    nib = (np.arange(64) * 5 + 1) % 16
    for e in range(64):
        s, j = e // 16, e % 16
        blk[4 + 8 * s + (j & 7)] |= nib[e] << (4 if j >= 8 else 0)
    want = np.array([codes[nib[e]] for e in range(64)], np.float32)
    assert np.array_equal(oracle.dequant(O.NVFP4, blk, 64)[0], want)
    # Q1_0: d = 0.5, bit e (LSB first) -> +-0.5
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    bits = (np.arange(128) * 7 + 3) % 5 < 2
    for e in range(128):
        blk[2 + e // 8] |= int(bits[e]) << (e % 8)
    assert np.array_equal(oracle.dequant(O.Q1_0, blk, 128)[0], np.where(bits, 0.5, -0.5).astype(np.float32))


@pytest.mark.parametrize("dt", O.NEW_QUANT_TYPES)
@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 16, 33])
@pytest.mark.parametrize("m", [96, 104, 77])
def test_int8_pipeline_matches_libjam(oracle, refjam, dt, n, m):
    k = 1024
    w = oracle.quantize(dt, oracle.normal(77 + dt, (m, k), 0.0, 0.02))
    a = oracle.outliers(5 + n, (n, k))
    want = refjam.mm(dt, w, a, m, n, k)
    got = oracle.mm_int8(dt, w, a, m, n, k)
    _, sa = oracle.mm_ref(dt, w, a, m, n, k)
    assert (np.abs(got - want) <= tol_int8(got, sa)).all()


def test_decompositions_are_discriminating(oracle, refjam):
    """The n < 8 formula at n = 8 (Q5_K, Q1_0: jam runs the F2 bands there) and the all-int8 tail (the bands
    leave the last m % 16 rows to a float dot) both miss libjam beyond the tolerance; NVFP4 has no band, so
    its F1 kernel answers at every n (the F2 flavour is refused)."""
    k = 1024
    for dt in (O.Q5_K, O.Q1_0):
        w = oracle.quantize(dt, oracle.normal(9, (96, k), 0.0, 0.02))
        a = oracle.outliers(10, (8, k))
        want = refjam.mm(dt, w, a, 96, 8, k)
        _, sa = oracle.mm_ref(dt, w, a, 96, 8, k)
        wrong = oracle.mm_int8(dt, w, a, 96, 8, k, flavour=1)
        assert not (np.abs(wrong - want) <= tol_int8(wrong, sa)).all(), O.NAMES[dt]
        w = oracle.quantize(dt, oracle.normal(31, (104, k), 0.0, 0.02))
        a = oracle.outliers(32, (9, k))
        want = refjam.mm(dt, w, a, 104, 9, k)
        _, sa = oracle.mm_ref(dt, w, a, 104, 9, k)
        all_int8 = oracle.mm_int8(dt, w, a, 104, 9, k, flavour=2)
        ok = np.abs(all_int8 - want) <= tol_int8(all_int8, sa)
        assert ok[:, :96].all() and not ok[:, 96:].all(), O.NAMES[dt]
    w = oracle.quantize(O.NVFP4, oracle.normal(9, (40, k), 0.0, 0.02))
    with pytest.raises(ValueError):
        oracle.mm_int8(O.NVFP4, w, oracle.normal(1, (8, k)), 40, 8, k, flavour=2)


@pytest.mark.parametrize("dt", O.DENSE_TYPES)
@pytest.mark.parametrize("k", [1024, 1000, 999])
def test_dense_matches_libjam(oracle, refjam, dt, k):
    """k % 32 == 0, k even only, k odd: the three branches of jam's BF16 routing (jam.c:622-652)."""
    m = 40
    w = oracle.quantize(dt, oracle.normal(5 + dt, (m, k), 0.0, 0.02))
    for n in (1, 3, 8, 9, 33):
        a = oracle.normal(6 + n, (n, k))
        want = refjam.mm(dt, w, a, m, n, k)
        got = oracle.mm_dense(dt, w, a, m, n, k)
        _, sa = oracle.mm_ref(dt, w, a, m, n, k)
        assert (np.abs(got - want) <= 1e-6 * sa + 1e-7).all(), (O.NAMES[dt], n, k)


def test_bf16_activation_rounding_is_discriminating(oracle, refjam):
    """Keeping BF16's activations f32 where jam rounds them to bf16 misses libjam by ~2e-4·sum|w·a| (the
    dense check above allows 1e-6); where jam keeps them f32 (n < 8 and k % 32 != 0) rounding would miss."""
    m, k = 40, 1024
    w = oracle.quantize(O.BF16, oracle.normal(5, (m, k), 0.0, 0.02))
    wf = np.ascontiguousarray(oracle.dequant(O.BF16, w, k)).view(np.uint8)
    for n in (3, 9):
        a = oracle.normal(7, (n, k))
        want = refjam.mm(O.BF16, w, a, m, n, k)
        _, sa = oracle.mm_ref(O.BF16, w, a, m, n, k)
        unrounded = oracle.mm_dense(O.F32, wf, a, m, n, k)
        assert (np.abs(unrounded - want) / sa).max() > 1e-5
    assert oracle.lib.jo_bf16_rounds_activations(3, 1024) and oracle.lib.jo_bf16_rounds_activations(9, 1000)
    assert not oracle.lib.jo_bf16_rounds_activations(3, 1000) and not oracle.lib.jo_bf16_rounds_activations(9, 999)
    k = 1000
    w = oracle.quantize(O.BF16, oracle.normal(5, (m, k), 0.0, 0.02))
    a = oracle.normal(7, (3, k))
    want = refjam.mm(O.BF16, w, a, m, 3, k)
    _, sa = oracle.mm_ref(O.BF16, w, a, m, 3, k)
    rounded = np.stack([[oracle.lib.jo_float2bf16(float(v)) for v in row] for row in a]).astype(np.uint32) << 16
    wrong = oracle.mm_dense(O.F32, np.ascontiguousarray(oracle.dequant(O.BF16, w, k)).view(np.uint8),
                            rounded.view(np.float32), m, 3, k)
    assert (np.abs(wrong - want) / sa).max() > 1e-5


def test_float2bf16_rne(oracle):
    """Round to nearest even on the dropped 16 bits, against numpy's exact binary arithmetic: a value just
    above, at and below each halfway point."""
    rng = np.random.default_rng(4)
    hi = rng.integers(0, 1 << 16, 4000, dtype=np.uint32) & 0x7F7F   # finite bf16 patterns
    for lo, up in ((0x7FFF, False), (0x8000, None), (0x8001, True)):
        x = ((hi << 16) | lo).astype(np.uint32).view(np.float32)
        got = np.array([oracle.lib.jo_float2bf16(float(v)) for v in x], np.uint32)
        base = hi & 0xFFFF
        want = base + (1 if up else 0) if up is not None else base + (base & 1)
        assert np.array_equal(got, want), lo


@pytest.mark.parametrize("dt", O.NEW_QUANT_TYPES)
def test_int8_within_precision_bound(oracle, dt):
    """PRECISION.md:20-26: int8-activation paths stay within 1e-2*sumAbs + 1e-3 of the float reference."""
    m, k = 48, 1024
    w = oracle.quantize(dt, oracle.normal(21 + dt, (m, k), 0.0, 0.02))
    for n in (1, 8):
        a = oracle.outliers(22, (n, k))
        got = oracle.mm_int8(dt, w, a, m, n, k)
        ref, sa = oracle.mm_ref(dt, w, a, m, n, k)
        assert (np.abs(got - ref) <= 1e-2 * sa + 1e-3).all()
