"""GPU parity sweep of the grouped matmul: seeded random expert counts (empty experts, experts of 1..7 rows,
large ones), expert shapes and weight types, dense enough for the one-launch fused prep or sparse enough for
the offsets + F1 decode path; each expert against the int8 oracle (tier 1), and the gather-folded call
(jamhip_mm_grouped_gather over routes from jamhip_moe_route) bit-identical to gather + grouped call, also in
native-MX mode 2 for MXFP4."""
import sys

import numpy as np
import pytest

from oracle import moe as M
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GROUPED = (O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K, O.MXFP4)


def _draws():
    rng = np.random.default_rng(0x6E0E)
    out = []
    for i in range(16):
        dt = GROUPED[i % len(GROUPED)]
        step = 256 if dt in (O.Q4_K, O.Q6_K) else 32
        E = int(rng.integers(2, 49))
        m = 32 * int(rng.integers(1, 7)) if rng.random() < 0.8 else 16 * int(rng.integers(1, 12)) + 16
        k = step * int(rng.integers(1, 2304 // step + 1))
        dense = rng.random() < 0.6
        seq = int(rng.integers(8 * E // 4 + 1, 12 * E)) if dense else int(rng.integers(1, max(2, 2 * E // 4)))
        out.append((dt, E, m, k, seq, 4))
    return out


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("dt,E,m,k,seq,topk", _draws())
def test_grouped_random_parity(hip, oracle, dt, E, m, k, seq, topk):
    import torch
    from qxotic_amd.jam import JAM, Segment
    print(f"moe sweep {O.NAMES[dt]} E={E} m={m} k={k} seq={seq} topk={topk}", file=sys.stderr, flush=True)
    rng = np.random.default_rng(E * 7919 + m + k + seq)
    pop = rng.random(E) ** 3 + 1e-3                       # skewed expert popularity, some nearly unused
    re = np.stack([rng.choice(E, size=min(topk, E), replace=False, p=pop / pop.sum()) for _ in range(seq)])
    re = re.astype(np.int32).ravel()
    tk = min(topk, E)
    R = seq * tk
    w_e = [oracle.quantize(dt, oracle.normal(0x6E0E ^ (97 * e + dt + k), (m, k), 0.0, 0.02)) for e in range(E)]
    w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
    x = oracle.outliers(0x6E0F ^ seq ^ k, (seq, k))
    i32 = lambda n: torch.zeros(n, dtype=torch.int32, device="cuda")
    counts, off, slot_route, route_slot = i32(E), i32(E + 1), i32(R), i32(R)
    re_d, x_d = _dev(re), _dev(x)
    g = torch.zeros((R, k), dtype=torch.float32, device="cuda")
    ca = torch.full((R, m), -3.0, dtype=torch.float32, device="cuda")
    cb = torch.full((R, m), -3.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
    try:
        assert hip.moe_route(re_d.data_ptr(), seq, tk, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                             route_slot.data_ptr()) == JAM.OK, hip.last_error()
        assert hip.moe_gather(x_d.data_ptr(), k, slot_route.data_ptr(), off.data_ptr(), E, seq, tk, k, g.data_ptr(),
                              k) == JAM.OK, hip.last_error()
        assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts.data_ptr(), g.data_ptr(), k, ca.data_ptr(), m, k,
                              R) == JAM.OK, hip.last_error()
        assert hip.mm_grouped_gather(Segment.of(w), dt, k, m, E, counts.data_ptr(), x_d.data_ptr(), k,
                                     slot_route.data_ptr(), tk, cb.data_ptr(), m, k, R) == JAM.OK, hip.last_error()
        hip.synchronize()
        got, got_b = ca.cpu().numpy(), cb.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), got_b.view(np.uint32))
        cnt = counts.cpu().numpy()
        ga = g.cpu().numpy()
        o = 0
        for e in range(E):
            n = int(cnt[e])
            if n:
                rows = ga[o:o + n]
                ref = oracle.mm_int8(dt, w_e[e], np.ascontiguousarray(rows), m, n, k)
                _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(rows), m, n, k)
                ok = np.abs(got[o:o + n] - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa
                assert ok.all(), (O.NAMES[dt], e, n, float(np.max(np.abs(got[o:o + n] - ref) / (sa + 1e-30))))
            o += n
        if dt == O.MXFP4 and m % 32 == 0:   # native mode 2: the gather-folded call equals the two calls
            assert hip.set_mx_native(2) == JAM.OK
            try:
                cn = torch.full((R, m), -3.0, dtype=torch.float32, device="cuda")
                cg = torch.full((R, m), -3.0, dtype=torch.float32, device="cuda")
                torch.cuda.synchronize()
                assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts.data_ptr(), g.data_ptr(), k, cn.data_ptr(),
                                      m, k, R) == JAM.OK, hip.last_error()
                assert hip.mm_grouped_gather(Segment.of(w), dt, k, m, E, counts.data_ptr(), x_d.data_ptr(), k,
                                             slot_route.data_ptr(), tk, cg.data_ptr(), m, k, R) == JAM.OK
                hip.synchronize()
                a1, a2 = cn.cpu().numpy(), cg.cpu().numpy()
                assert np.isfinite(a1).all()
                assert np.array_equal(a1.view(np.uint32), a2.view(np.uint32))
            finally:
                hip.set_mx_native(0)
    finally:
        assert hip.evict(Segment.of(w)) == JAM.OK
