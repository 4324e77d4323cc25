"""CPU pins of the native-MX restatement (oracle/mxnative.py): the e4m3 value table against the format's
closed form, encode against brute-force nearest-even, the block exponent rule, and the hi + lo
reconstruction bounds."""
import numpy as np
import pytest

from oracle import mxnative as X


def test_e4m3_table_fixed_points():
    v = X.e4m3_values()
    assert v[0x7E] == 448.0 and v[0x08] == 2.0 ** -6 and v[0x01] == 2.0 ** -9 and v[0x38] == 1.0
    assert v[0x00] == 0.0 and v[0x80] == 0.0 and np.signbit(v[0x80])
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF])
    pos = v[:0x7F]
    assert (np.diff(pos) > 0).all() and len(np.unique(pos)) == 127
    assert np.array_equal(v[0x80:0xFF], -v[:0x7F])


def brute(vals):
    table = X.e4m3_values()
    codes = np.array([c for c in range(256) if not np.isnan(table[c])])
    out = []
    for x in vals:
        d = np.abs(table[codes] - x)
        best = codes[d == d.min()]
        if len(best) > 1:   # a tie between two neighbours (or +0 / -0): the even mantissa, sign of x
            best = [c for c in best if (c & 1) == 0 and ((c & 0x80) != 0) == (x < 0 or (x == 0 and np.signbit(x)))] or best
        out.append(best[0])
    return np.array(out, np.uint8)


def test_encode_is_nearest_even():
    rng = np.random.default_rng(3)
    table = X.e4m3_values()
    pos = table[:0x7F]
    mids = (pos[:-1] + pos[1:]) / 2                           # every exact tie
    vals = np.concatenate([rng.uniform(-448, 448, 2000), rng.uniform(-0.02, 0.02, 500), mids, -mids,
                           pos, -pos[1:], [448.0, -448.0, 2.0 ** -10, 3 * 2.0 ** -10]])
    got = X.e4m3_encode(vals)
    want = brute(vals)
    nz = vals != 0
    assert np.array_equal(got[nz], want[nz])
    # a tie goes to the even code: 1.0625 lies between 1.0 (0x38) and 1.125 (0x39)
    assert X.e4m3_encode(np.array([1.0625]))[0] == 0x38 and X.e4m3_encode(np.array([1.1875]))[0] == 0x3A


def test_block_exponent_rule():
    rng = np.random.default_rng(4)
    amax = np.concatenate([rng.lognormal(0, 8, 4000), 448.0 * 2.0 ** np.arange(-20, 20), np.nextafter(448.0, 0) * 2.0 ** np.arange(-5, 5)])
    E = X.block_exponent(amax).astype(np.float64)
    assert (amax * 2.0 ** -E <= 448.0).all()
    assert (amax * 2.0 ** -(E - 1) > 448.0).all()
    assert X.block_exponent(np.array([0.0]))[0] == -127


@pytest.mark.parametrize("mode,bound", [(1, 2.0 ** -9), (2, 2.0 ** -4)])
def test_reconstruction_bound(mode, bound):
    rng = np.random.default_rng(5 + mode)
    x = rng.standard_normal((16, 4096)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] = 20.0
    xa = X.dequant_act(x, mode)
    blk = np.abs(x).reshape(16, -1, 32).max(axis=2)
    err = np.abs(xa - x).reshape(16, -1, 32).max(axis=2)
    assert (err <= bound * blk).all()
    if mode == 1:   # typically half the bound (about 2^-10.5 of the block maximum)
        assert np.median(err / blk) < 2.0 ** -10


def test_layout_is_blockwise():
    """A block's codes depend on that block only (zeroing another block leaves them unchanged)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 128)).astype(np.float32)
    h0, l0, e0, _ = X.quantize(x)
    y = x.copy()
    y[:, 32:64] = 0
    h1, l1, e1, _ = X.quantize(y)
    keep = np.r_[0:32, 64:128]
    assert np.array_equal(h0[:, keep], h1[:, keep]) and np.array_equal(l0[:, keep], l1[:, keep])
    assert (h1[:, 32:64] == 0).all() and (e1[:, 1] == -127).all()
