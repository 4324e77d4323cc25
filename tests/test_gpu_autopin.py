"""GPU: autopin, the residency an unedited jinfer gets (jamhip_ctx_set_autopin).

jinfer's MatMul.JamMm.mm passes the same mmap'd address for a tensor on every call and never pins
(jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/kernels/MatMul.java:1783-1830); with autopin on, the
backend pins such a W on its N-th sighting and serves later calls from the device copy, after checking two
pages of the host range against the hashes taken at pin time. The arena case of jam's parity test (one
buffer rewritten in place with another tensor's bytes, JamBackendParityTest.java:31) must be detected.
Every result is compared bit for bit with a context that stages W on every call (same kernels), and with
the oracle under the usual tolerance.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


@pytest.fixture
def ctxs():
    from qxotic_amd.jam import HipJAM
    auto, plain = HipJAM(0), HipJAM(0)
    yield auto, plain
    auto.close()
    plain.close()


def mm(hip, dt, w, a, m, n, k, ldw=None):
    from qxotic_amd.jam import JAM, Segment
    c = np.zeros((n, m), np.float32)
    st = hip.mm(Segment.of(w), 0, dt, ldw or k, Segment.of(a), 0, JAM.F32, k, Segment.of(c), 0, JAM.F32, m, m, n, k)
    assert st == JAM.OK, hip.last_error()
    return c


def check_oracle(oracle, dt, w, a, c, m, n, k):
    ref = oracle.mm_int8(dt, w, a, m, n, k)
    _, sa = oracle.mm_ref(dt, w, a, m, n, k)
    assert (np.abs(c - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa).all()


def test_autopin_off_by_default(ctxs, oracle):
    auto, _ = ctxs
    m, k = 64, 512
    w = oracle.quantize(O.Q4_K, oracle.normal(1, (m, k), 0.0, 0.02))
    a = oracle.normal(2, (1, k))
    for _ in range(3):
        mm(auto, O.Q4_K, w, a, m, 1, k)
    assert auto.autopin_stats() == {"pins": 0, "hits": 0, "staged": 0, "invalidated": 0}
    assert auto.pinned_bytes() == 0


@pytest.mark.parametrize("dt,m,k,n", [(O.Q4_K, 160, 2048, 1), (O.Q8_0, 96, 1024, 9), (O.MXFP4, 128, 2880, 3)])
def test_autopin_second_sighting_serves_device_copy(ctxs, oracle, dt, m, k, n):
    """N = 2: the first call stages, the second pins and is served by the pin, the rest hit; every result
    bit-identical to the staging context's."""
    auto, plain = ctxs
    say(f"autopin dt={dt} m={m} k={k} n={n}")
    assert auto.set_autopin(2) == 0
    w = oracle.quantize(dt, oracle.normal(3 + dt, (m, k), 0.0, 0.02))
    a = oracle.normal(4, (n, k))
    want = mm(plain, dt, w, a, m, n, k)
    check_oracle(oracle, dt, w, a, want, m, n, k)
    got = [mm(auto, dt, w, a, m, n, k) for _ in range(4)]
    for g in got:
        assert np.array_equal(bits(g), bits(want))
    assert auto.autopin_stats() == {"pins": 1, "hits": 3, "staged": 1, "invalidated": 0}
    assert auto.pinned_bytes() > 0
    assert plain.pinned_bytes() == 0


def test_autopin_detects_in_place_rewrite(ctxs, oracle):
    """An arena rewritten with another tensor's bytes at the same address: the spot check fails, the pin is
    evicted, the call stages the new bytes (bit-identical to the staging context), and the new content is
    pinned again on its next sighting."""
    auto, plain = ctxs
    m, k, n = 128, 4096, 1
    assert auto.set_autopin(2) == 0
    arena = oracle.quantize(O.Q4_K, oracle.normal(11, (m, k), 0.0, 0.02))
    other = oracle.quantize(O.Q4_K, oracle.normal(12, (m, k), 0.0, 0.02))
    a = oracle.normal(13, (n, k))
    for _ in range(3):
        mm(auto, O.Q4_K, arena, a, m, n, k)
    assert auto.autopin_stats()["pins"] == 1
    arena[...] = other                         # same address, new tensor
    want = mm(plain, O.Q4_K, other, a, m, n, k)
    got = mm(auto, O.Q4_K, arena, a, m, n, k)
    assert np.array_equal(bits(got), bits(want))
    st = auto.autopin_stats()
    assert st["invalidated"] == 1 and st["pins"] == 1
    got2 = mm(auto, O.Q4_K, arena, a, m, n, k)    # second sighting of the new bytes: pinned again
    assert np.array_equal(bits(got2), bits(want))
    st = auto.autopin_stats()
    assert st["pins"] == 2 and st["invalidated"] == 1
    check_oracle(oracle, O.Q4_K, other, a, got2, m, n, k)


def test_autopin_single_page_rewrite_is_swept(ctxs, oracle):
    """A rewrite confined to one 4 KiB page is caught within one sweep of the range's pages (the rotating
    spot check visits every page), never served stale after that."""
    auto, plain = ctxs
    m, k, n = 64, 1024, 1                     # 64 x 576 B = 9 pages
    assert auto.set_autopin(1) == 0
    w = oracle.quantize(O.Q4_K, oracle.normal(21, (m, k), 0.0, 0.02))
    a = oracle.normal(22, (n, k))
    mm(auto, O.Q4_K, w, a, m, n, k)
    assert auto.autopin_stats()["pins"] == 1
    flat = w.reshape(-1)
    flat[5000:5100] ^= 0x5A                    # bytes inside page 1 only
    want = mm(plain, O.Q4_K, w, a, m, n, k)
    pages = (w.nbytes + 4095) // 4096
    for _ in range(pages + 1):
        got = mm(auto, O.Q4_K, w, a, m, n, k)
        if auto.autopin_stats()["invalidated"]:
            break
    assert auto.autopin_stats()["invalidated"] == 1
    assert np.array_equal(bits(mm(auto, O.Q4_K, w, a, m, n, k)), bits(want))


def test_autopin_limits(ctxs, oracle):
    """Never pinned: a range over max_bytes, and a W read with ldw > k (only part of each row); an autopin
    is dropped by jamhip_weight_evict like any pin."""
    from qxotic_amd.jam import Segment
    auto, plain = ctxs
    m, k = 64, 1024
    w = oracle.quantize(O.Q4_K, oracle.normal(31, (m, k), 0.0, 0.02))
    a = oracle.normal(32, (1, k))
    assert auto.set_autopin(1, max_bytes=1024) == 0
    for _ in range(2):
        mm(auto, O.Q4_K, w, a, m, 1, k)
    assert auto.autopin_stats()["pins"] == 0 and auto.pinned_bytes() == 0
    assert auto.set_autopin(1) == 0
    wide = oracle.quantize(O.Q4_K, oracle.normal(33, (m, 2 * k), 0.0, 0.02))
    for _ in range(2):
        got = mm(auto, O.Q4_K, wide, a, m, 1, k, ldw=2 * k)
    assert np.array_equal(bits(got), bits(mm(plain, O.Q4_K, wide, a, m, 1, k, ldw=2 * k)))
    assert auto.autopin_stats()["pins"] == 0
    mm(auto, O.Q4_K, w, a, m, 1, k)
    assert auto.autopin_stats()["pins"] == 1 and auto.pinned_bytes() > 0
    assert auto.evict(Segment.of(w)) == 0
    assert auto.pinned_bytes() == 0


def test_device_entry_points_never_serve_an_autopin(ctxs, oracle):
    """An autopin serves only jamhip_mm calls that pass its spot check. jamhip_mm_device (whose launches a
    caller may capture in a graph) stages W instead: after an in-place rewrite of an autopinned range it
    returns the new bytes' result, and the noalloc entry point (which cannot stage) declines."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    auto, plain = ctxs
    m, k, n = 64, 1024, 2
    assert auto.set_autopin(1) == 0
    w = oracle.quantize(O.Q4_K, oracle.normal(41, (m, k), 0.0, 0.02))
    other = oracle.quantize(O.Q4_K, oracle.normal(42, (m, k), 0.0, 0.02))
    a = oracle.normal(43, (n, k))
    mm(auto, O.Q4_K, w, a, m, n, k)
    assert auto.autopin_stats()["pins"] == 1
    w[...] = other
    a_d = torch.from_numpy(a).cuda()
    c_d = torch.zeros((n, m), dtype=torch.float32, device="cuda")
    assert auto.mm_device(Segment.of(w), O.Q4_K, k, a_d.data_ptr(), k, c_d.data_ptr(), m, m, n, k) == JAM.OK
    auto.synchronize()
    assert np.array_equal(bits(c_d.cpu().numpy()), bits(mm(plain, O.Q4_K, other, a, m, n, k)))
    assert auto.mm_device_noalloc(Segment.of(w), O.Q4_K, k, a_d.data_ptr(), k, c_d.data_ptr(), m, m, n,
                                  k) == JAM.EUNSUPPORTED
    assert auto.autopin_stats()["invalidated"] == 0   # the device entry points never looked at the autopin


def test_offset_call_into_an_autopin_is_staged(ctxs, oracle):
    """A jamhip_mm call at a row offset inside an autopinned range is not served from the autopin (no spot
    check covers it): after an in-place rewrite it returns the new bytes' result."""
    auto, plain = ctxs
    m, k, n = 64, 1024, 1
    assert auto.set_autopin(1) == 0
    w = oracle.quantize(O.Q4_K, oracle.normal(51, (2 * m, k), 0.0, 0.02))
    other = oracle.quantize(O.Q4_K, oracle.normal(52, (2 * m, k), 0.0, 0.02))
    a = oracle.normal(53, (n, k))
    mm(auto, O.Q4_K, w, a, 2 * m, n, k)
    assert auto.autopin_stats()["pins"] == 1
    w[...] = other
    from qxotic_amd.jam import JAM, Segment
    c = np.zeros((n, m), np.float32)
    st = auto.mm(Segment.of(w), m * O.row_bytes(O.Q4_K, k), O.Q4_K, k, Segment.of(a), 0, JAM.F32, k, Segment.of(c),
                 0, JAM.F32, m, m, n, k)
    assert st == JAM.OK, auto.last_error()
    want = mm(plain, O.Q4_K, np.ascontiguousarray(other[m:]), a, m, n, k)
    assert np.array_equal(bits(c), bits(want))


def test_explicit_pin_takes_over_an_autopin(ctxs, oracle):
    """jamhip_weight_pin on an autopinned range (the same extent, or one overlapping it) succeeds: the autopin
    is dropped and the range copied afresh, so the pin holds the bytes at pin time even if the autopin's copy
    predates them. The pin then serves device calls, and stays after further rewrites (an explicit pin is the
    caller's promise)."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    auto, plain = ctxs
    m, k, n = 64, 1024, 1
    assert auto.set_autopin(1) == 0
    w = oracle.quantize(O.Q4_K, oracle.normal(61, (2 * m, k), 0.0, 0.02))
    snap = oracle.quantize(O.Q4_K, oracle.normal(62, (2 * m, k), 0.0, 0.02))
    a = oracle.normal(63, (n, k))
    mm(auto, O.Q4_K, w, a, m, n, k)            # autopin of rows [0, m)
    assert auto.autopin_stats()["pins"] == 1
    w[...] = snap                              # rewritten in place, not yet spot-checked
    assert auto.pin(Segment.of(w), O.Q4_K, k, 2 * m) == JAM.OK, auto.last_error()   # overlaps the autopin
    a_d = torch.from_numpy(a).cuda()
    c_d = torch.zeros((n, 2 * m), dtype=torch.float32, device="cuda")
    w[...] = 0                                 # the pin keeps the bytes it copied
    assert auto.mm_device(Segment.of(w), O.Q4_K, k, a_d.data_ptr(), k, c_d.data_ptr(), 2 * m, 2 * m, n,
                          k) == JAM.OK
    auto.synchronize()
    assert np.array_equal(bits(c_d.cpu().numpy()), bits(mm(plain, O.Q4_K, snap, a, 2 * m, n, k)))
    assert auto.evict(Segment.of(w)) == JAM.OK
    assert auto.pinned_bytes() == 0
    # the same extent as the autopin
    w[...] = snap
    mm(auto, O.Q4_K, w, a, 2 * m, n, k)
    assert auto.autopin_stats()["pins"] == 2
    assert auto.pin(Segment.of(w), O.Q4_K, k, 2 * m) == JAM.OK, auto.last_error()
    w[...] = 0
    assert auto.mm_device(Segment.of(w), O.Q4_K, k, a_d.data_ptr(), k, c_d.data_ptr(), 2 * m, 2 * m, n,
                          k) == JAM.OK
    auto.synchronize()
    assert np.array_equal(bits(c_d.cpu().numpy()), bits(mm(plain, O.Q4_K, snap, a, 2 * m, n, k)))
    assert auto.evict(Segment.of(w)) == JAM.OK
