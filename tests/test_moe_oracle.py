"""Pins the MoE dispatch restatement (oracle/moe.py) with hand-derived answers and invariants."""
import numpy as np

from oracle import moe as M


def test_dispatch_csr_known_answer():
    # seq 3, topk 2, 3 experts: routes r = s*2 + k -> experts [2, 0 | 0, 1 | 2, 1]
    counts, off, slot_route, route_slot = M.dispatch_csr(np.array([2, 0, 0, 1, 2, 1]), 3)
    assert counts.tolist() == [2, 2, 2]
    assert off.tolist() == [0, 2, 4, 6]
    # expert 0 takes routes 1 then 2, expert 1 routes 3 then 5, expert 2 routes 0 then 4 (Moe.java:198-205)
    assert slot_route.tolist() == [1, 2, 3, 5, 0, 4]
    assert route_slot.tolist() == [4, 0, 1, 2, 5, 3]


def test_dispatch_csr_invariants():
    rng = np.random.default_rng(3)
    E, seq, topk = 7, 50, 3
    re = np.stack([rng.permutation(E)[:topk] for _ in range(seq)]).ravel()
    re[5] = -1                      # an invalid id takes no slot
    re[17] = E
    counts, off, slot_route, route_slot = M.dispatch_csr(re, E)
    valid = (re >= 0) & (re < E)
    assert counts.sum() == valid.sum() == off[-1]
    assert sorted(slot_route[:off[-1]].tolist()) == np.flatnonzero(valid).tolist()
    for e in range(E):
        rs = slot_route[off[e]:off[e + 1]]
        assert (re[rs] == e).all() and (np.diff(rs) > 0).all()   # each expert's routes in (s, k) order
    assert (route_slot[~valid] == -1).all()
    assert (slot_route[route_slot[valid]] == np.flatnonzero(valid)).all()


def test_fma32_single_rounding():
    a = np.float32(1 + 2.0 ** -12)
    got = M._fma32(a, np.array([a], np.float32), np.array([-1.0], np.float32))[0]
    assert got == np.float32(2.0 ** -11 + 2.0 ** -24)           # exact: one rounding
    assert np.float32(a * a) - np.float32(1.0) == np.float32(2.0 ** -11)   # two roundings lose 2^-24


def test_combine_expert_order():
    # one token, three routes: route k=0 -> expert 2 (y=1), k=1 -> expert 0 (y=1e8), k=2 -> expert 1 (y=-1e8).
    # Expert order sums 1e8 - 1e8 + 1 = 1; route order would give (1 + 1e8) - 1e8 = 0 in f32.
    y_by_route = np.array([[1.0], [1.0e8], [-1.0e8]], np.float32)
    re = np.array([2, 0, 1])
    prob = np.ones(3, np.float32)
    counts, off, slot_route, route_slot = M.dispatch_csr(re, 3)
    ys = y_by_route[slot_route[:3]]                  # expert outputs in slot (CSR) order
    out = M.combine(ys, re, prob, route_slot, 1, 3, 3)
    assert out[0, 0] == np.float32(1.0)
    assert (np.float32(1.0) + np.float32(1e8)) - np.float32(1e8) == np.float32(0.0)


def test_mm_grouped_is_per_expert_calls(oracle):
    from oracle import oracle as O
    rng_w = [oracle.quantize(O.Q8_0, oracle.normal(40 + e, (32, 64), 0.0, 0.02)) for e in range(3)]
    a = oracle.normal(50, (12, 64))
    counts = [5, 0, 7]
    got = M.mm_grouped(oracle, O.Q8_0, rng_w, a, counts, 32, 64)
    assert np.array_equal(got[:5], oracle.mm_int8(O.Q8_0, rng_w[0], a[:5], 32, 5, 64))
    assert np.array_equal(got[5:12], oracle.mm_int8(O.Q8_0, rng_w[2], a[5:12], 32, 7, 64))
