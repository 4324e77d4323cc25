"""GPU parity sweep: seeded random shapes over every quantized type and every n-range path (F1 decode at 1..7
tokens, F2 tiles, the matrix cores with and without split K, the activation prep's 8-slot groups from 2048
tokens), each against the int8 oracle on a sample of rows (tier 1: |gpu - oracle| <= 1e-3|oracle| + 1e-5
sum|w*a|), with the ldc gap untouched and a rerun bit-identical."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

KQ = (O.Q4_K, O.Q5_K, O.Q6_K)


def _draws():
    rng = np.random.default_rng(0x5EED5)
    out = []
    for i in range(40):
        dt = O.ALL_QUANT_TYPES[i % len(O.ALL_QUANT_TYPES)]
        step = 256 if dt in KQ else O.BLOCK[dt][0]
        n = int(rng.choice([1, 2, 3, 5, 7, 8, 9, 13, 16, 24, 31, 33, 64, 100, 257, 512, 700, 2100]))
        k = step * int(rng.integers(1, 20480 // step + 1))
        while n * k > 8_000_000 and k > step:      # A at most 32 MB
            k = max(step, k // 2 // step * step)
        m = 16 * int(rng.integers(1, 400))
        while m * k > 16_000_000 and m > 16:       # W at most 16 M elements
            m = max(16, m // 2 // 16 * 16)
        out.append((dt, m, k, n))
    return out


@pytest.mark.parametrize("dt,m,k,n", _draws())
def test_random_shape_parity(hip, oracle, dt, m, k, n):
    from qxotic_amd.jam import JAM, Segment
    print(f"sweep {O.NAMES[dt]} m={m} k={k} n={n}", file=sys.stderr, flush=True)
    w = oracle.quantize(dt, oracle.normal(0x5EED ^ (m * 31 + k) ^ dt, (m, k), 0.0, 0.02))
    a = oracle.outliers(0x5EED ^ n ^ k, (n, k))
    c = np.full((n, m + 2), -3.0, np.float32)

    def run(out):
        st = hip.mm(Segment.of(w), 0, dt, k, Segment.of(a), 0, JAM.F32, k, Segment.of(out), 0, JAM.F32, m + 2, m,
                    n, k)
        assert st == JAM.OK, hip.last_error()
        return out

    got = run(c)
    assert (got[:, m:] == -3.0).all()
    # jam's rule for n >= 8 gives the last m % 16 rows a float dot: sample whole 16-row groups from the rows
    # before them (the oracle on a sample then applies no tail rule) and check the tail rows as a matrix of
    # their own (where the oracle applies it to every row)
    m16 = m - m % 16
    rng = np.random.default_rng(m + k + n)
    rows = np.arange(m16) if m16 <= 32 else np.sort(rng.choice(m16, 32, replace=False))
    for sel in (rows, np.arange(m16, m)):
        if len(sel) == 0:
            continue
        ws = np.ascontiguousarray(w[sel])
        ref = oracle.mm_int8(dt, ws, a, len(sel), n, k)
        _, sa = oracle.mm_ref(dt, ws, a, len(sel), n, k)
        g = got[:, sel]
        ok = np.abs(g - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa
        assert ok.all(), (O.NAMES[dt], m, k, n, int((~ok).sum()), float(np.max(np.abs(g - ref) / (sa + 1e-30))))
    again = run(np.full((n, m + 2), -3.0, np.float32))
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
