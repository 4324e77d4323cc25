"""GPU parity of jam's remaining weight types through the C-ABI: Q5_K, NVFP4 and Q1_0 (jam's int8 pipeline) and
F32, F16, BF16 (jam's dense paths), against the oracle restatement pinned to libjam (tests/test_oracle_dtypes.py).

Bound: tier 1, |gpu - oracle| <= 1e-3*|oracle| + 1e-5*sum|w*a| (the same activation semantics, bit-exact int8
codes or bf16 rounding; only the f32 summation order differs), and jam's own 1e-2*sum|w*a| + 1e-3 against the
float reference on N(0,1) activations. Every n-range jam routes differently is covered: F1 decode (n < 8),
F2 bands with the float-dot tail rows (Q5_K, Q1_0 from n = 8), NVFP4's F1 at every n, the dense GEMV (n <= 8)
and matrix-core GEMM (n > 8), BF16's three activation rules (k % 32 == 0, k even, k odd)."""
import sys

import numpy as np
import pytest

from conftest import parity_report
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NS = [1, 2, 3, 7, 8, 9, 16, 33, 64, 100]


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def tier1(got, ref, sa):
    return np.abs(got - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa


def run_mm(hip, dt, w, a, m, n, k, ldw=None, lda=None, ldc=None, out=None, w_off=0):
    from qxotic_amd.jam import JAM, Segment
    ldw = ldw or k
    lda = lda or a.shape[-1]
    ldc = ldc or m
    c = out if out is not None else np.zeros((n, ldc), np.float32)
    st = hip.mm(Segment.of(w), w_off, dt, ldw, Segment.of(a), 0, JAM.F32, lda, Segment.of(c), 0, JAM.F32, ldc, m, n, k)
    assert st == JAM.OK, (O.NAMES[dt], m, n, k, hip.last_error())
    return c


def shapes(dt):
    be = O.BLOCK[dt][0]
    if be == 1:
        return [(104, 1024), (70, 1000), (33, 999), (130, 4096)]
    return [(m, k) for (m, k) in [(104, 1024), (77, 512), (130, 2048), (48, 256 if be <= 256 else 512)] if k % be == 0]


@pytest.mark.parametrize("dt", O.NEW_QUANT_TYPES + O.DENSE_TYPES)
def test_parity_all_n(hip, oracle, dt):
    for (m, k) in shapes(dt):
        w = oracle.quantize(dt, oracle.normal(0xD7 ^ (m * 31 + k + dt), (m, k), 0.0, 0.02))
        for n in NS:
            say(f"dtype {O.NAMES[dt]} m={m} n={n} k={k}")
            a = oracle.outliers(1000 + n, (n, k))
            got = run_mm(hip, dt, w, a, m, n, k)
            ref = oracle.mm(dt, w, a, m, n, k)
            _, sa = oracle.mm_ref(dt, w, a, m, n, k)
            ok = tier1(got, ref, sa)
            assert ok.all(), (O.NAMES[dt], m, n, k, int((~ok).sum()))
            a = oracle.normal(2000 + n, (n, k))
            got = run_mm(hip, dt, w, a, m, n, k)
            fref, sa = oracle.mm_ref(dt, w, a, m, n, k)
            assert tier1(got, oracle.mm(dt, w, a, m, n, k), sa).all()
            assert (np.abs(got - fref) <= 1e-2 * sa + 1e-3).all(), (O.NAMES[dt], m, n, k)


@pytest.mark.parametrize("dt", O.NEW_QUANT_TYPES + O.DENSE_TYPES)
def test_layout_metamorphic(hip, oracle, dt):
    """ldw > k with padding bytes (0xFF: NaN for the dense types, so columns past k must not be read into a
    product), lda > k, ldc > m with the gap untouched, rerun bit-identical."""
    be = O.BLOCK[dt][0]
    m, k = 48, 512
    ldw = k + (2 * max(be, 256) if be > 1 else 24)
    wfull = oracle.quantize(dt, oracle.normal(5, (m, ldw), 0.0, 0.02))
    rb = O.row_bytes(dt, k)
    wpad = wfull.copy()
    wpad[:, rb:] = 0xFF
    for n in (1, 5, 8, 20):
        say(f"layout {O.NAMES[dt]} n={n}")
        a = np.full((n, k + 40), 7.0, np.float32)
        a[:, :k] = oracle.normal(6 + n, (n, k))
        ldc = m + 9
        c = np.full((n, ldc), -12345.0, np.float32)
        run_mm(hip, dt, wpad, a, m, n, k, ldw=ldw, lda=k + 40, ldc=ldc, out=c)
        assert (c[:, m:] == -12345.0).all()
        ref = run_mm(hip, dt, np.ascontiguousarray(wfull[:, :rb]), np.ascontiguousarray(a[:, :k]), m, n, k)
        assert np.array_equal(bits(c[:, :m]), bits(ref[:, :m])), (O.NAMES[dt], n)
        again = run_mm(hip, dt, wpad, a, m, n, k, ldw=ldw, lda=k + 40)
        assert np.array_equal(bits(again[:, :m]), bits(c[:, :m]))


@pytest.mark.parametrize("dt", O.NEW_QUANT_TYPES + O.DENSE_TYPES)
def test_pinned_matches_staged_and_slices(hip, oracle, dt):
    from qxotic_amd.jam import JAM, Segment
    experts, rows, k = 4, 64, 512
    w = oracle.quantize(dt, oracle.normal(17, (experts * rows, k), 0.0, 0.02))
    rb = O.row_bytes(dt, k)
    a = oracle.normal(18, (40, k))
    staged = [run_mm(hip, dt, np.ascontiguousarray(w[e * rows:(e + 1) * rows]), a[:n], rows, n, k)
              for e in range(experts) for n in (1, 9, 40)]
    assert hip.pin(Segment.of(w), dt, k, experts * rows) == JAM.OK, hip.last_error()
    try:
        i = 0
        for e in range(experts):
            for n in (1, 9, 40):
                say(f"pinned {O.NAMES[dt]} expert={e} n={n}")
                got = run_mm(hip, dt, w, np.ascontiguousarray(a[:n]), rows, n, k, w_off=e * rows * rb)
                assert np.array_equal(bits(got), bits(staged[i])), (O.NAMES[dt], e, n)
                i += 1
    finally:
        assert hip.evict(Segment.of(w)) == JAM.OK


FULL = [(O.Q5_K, 14336, 4096, 1), (O.Q5_K, 4096, 14336, 8), (O.NVFP4, 4096, 4096, 1), (O.NVFP4, 4096, 4096, 16),
        (O.Q1_0, 4096, 4096, 1), (O.Q1_0, 4096, 4096, 16), (O.BF16, 4096, 4096, 1), (O.BF16, 4096, 4096, 64),
        (O.F16, 4096, 4096, 4), (O.F32, 2048, 2880, 33), (O.F16, 14336, 4096, 512), (O.BF16, 4096, 14336, 2),
        (O.F16, 14336, 4096, 8)]


@pytest.mark.parametrize("dt,m,k,n", FULL)
def test_full_size(hip, oracle, dt, m, k, n):
    """Llama-sized matrices: every output finite, a rerun bit-identical, 256 sampled rows against the oracle."""
    from qxotic_amd.jam import JAM, Segment
    say(f"full {O.NAMES[dt]} {m}x{k} n={n}")
    w = oracle.quantize(dt, oracle.normal(0x5A11C0DE ^ dt ^ m, (m, k), 0.0, 0.02))
    a = oracle.normal(0x5A11C0DE ^ 77, (n, k))
    assert hip.pin(Segment.of(w), dt, k, m) == JAM.OK, hip.last_error()
    try:
        got = run_mm(hip, dt, w, a, m, n, k)
        again = run_mm(hip, dt, w, a, m, n, k)
    finally:
        hip.evict(Segment.of(w))
    assert np.isfinite(got).all()
    assert np.array_equal(bits(got), bits(again))
    rows = np.sort(np.random.default_rng(dt + m).choice(m, 256, replace=False))
    ws = np.ascontiguousarray(w[rows])
    ref = oracle.mm(dt, ws, a, len(rows), n, k)
    _, sa = oracle.mm_ref(dt, ws, a, len(rows), n, k)
    parity_report(f"{O.NAMES[dt]} {m}x{k} n={n}", got[:, rows], ref, sa)
    assert tier1(got[:, rows], ref, sa).all()


def test_status_codes_follow_jam(hip, oracle):
    """EUNSUPPORTED exactly where jam's jam_mm refuses (jam.c:662-685, 752): k off the block for every quantized
    type, ldw off the block for Q1_0 (not for NVFP4 and the K-quants, which stride by whole blocks of ldw);
    the dense types take any k."""
    from qxotic_amd.jam import JAM, Segment
    a = oracle.normal(1, (2, 1024))
    c = np.zeros((2, 64), np.float32)

    def st(dt, ldw, k, m=16):
        w = np.zeros(m * max(O.row_bytes(dt, ldw), 4) + 64, np.uint8)
        return hip.mm(Segment.of(w), 0, dt, ldw, Segment.of(a), 0, JAM.F32, 1024, Segment.of(c), 0, JAM.F32, 64, m, 2, k)

    assert st(O.Q5_K, 256, 128) == JAM.EUNSUPPORTED
    assert st(O.Q5_K, 300, 256) == JAM.OK            # row stride = 1 super-block, as jam
    assert st(O.NVFP4, 64, 32) == JAM.EUNSUPPORTED
    assert st(O.NVFP4, 100, 64) == JAM.OK
    assert st(O.Q1_0, 128, 64) == JAM.EUNSUPPORTED
    assert st(O.Q1_0, 200, 128) == JAM.EUNSUPPORTED
    assert st(O.Q1_0, 256, 128) == JAM.OK
    for dt in O.DENSE_TYPES:
        assert st(dt, 7, 7) == JAM.OK and st(dt, 9, 5) == JAM.OK


def test_nvfp4_every_scale_code(hip, oracle):
    """All 256 UE4M3 scale bytes in the weights of every NVFP4 path: one-token decode, the 2..7-token F1 kernel,
    F1 bands, and the matrix cores (n >= 9). jam reads 0x00 and 0x7F as 0 and otherwise ignores bit 7, so 0x80
    reads 0 but 0xFF reads 480 (e = 15, m = 7): a decoder that masks bit 7 first and then treats 0x7F as zero
    gets 0xFF wrong, and this case catches it."""
    m, k = 64, 256   # 16 sub-blocks per row: 1024 scale bytes, each code 4 times
    w = oracle.quantize(O.NVFP4, oracle.normal(0x5CA1E, (m, k), 0.0, 0.02)).reshape(m, -1).copy()
    codes = np.arange(m * 16, dtype=np.uint32) % 256
    for r in range(m):
        for j in range(k // 64):
            w[r, 36 * j:36 * j + 4] = codes[16 * r + 4 * j:16 * r + 4 * j + 4]
    w = np.ascontiguousarray(w)
    for n in (1, 3, 7, 8, 16, 64):
        say(f"nvfp4 every scale code n={n}")
        a = oracle.outliers(0x5CA + n, (n, k))
        got = run_mm(hip, O.NVFP4, w, a, m, n, k)
        ref = oracle.mm(O.NVFP4, w, a, m, n, k)
        _, sa = oracle.mm_ref(O.NVFP4, w, a, m, n, k)
        assert np.isfinite(got).all()
        ok = tier1(got, ref, sa)
        assert ok.all(), (n, int((~ok).sum()))
