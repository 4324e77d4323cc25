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


# ------------------------------------------------------------------------------------------ top-k
def test_select_topk_known_answers():
    """Hand-worked rows of Moe.selectTopK (Moe.java:76-127): the first maximum wins on ties, winners are masked
    to -Inf, a row with nothing above -Inf keeps picking expert 0 (best starts at 0), NaN is never taken, and
    counts are the routes per expert."""
    sel = np.array([[1.0, 3.0, 3.0, 2.0],          # tie at 3: expert 1 first, then 2, then 3
                    [-np.inf, -np.inf, -np.inf, -np.inf],   # nothing > -Inf: expert 0 every time
                    [np.nan, 0.5, np.nan, -1.0],   # NaN skipped: 1, then 3, then 0 (nothing left above -Inf)
                    [0.0, 0.0, 0.0, 7.0]], np.float32)
    re, rp, counts, masked = M.select_topk(sel, 3)
    assert re.tolist() == [1, 2, 3, 0, 0, 0, 1, 3, 0, 3, 0, 1]
    assert rp[:3].tolist() == [3.0, 3.0, 2.0]
    assert np.isneginf(rp[3:6]).all()
    assert rp[6:9].tolist()[:2] == [0.5, -1.0] and np.isnan(rp[8])   # expert 0 of row 2 holds NaN
    assert rp[9:12].tolist() == [7.0, 0.0, 0.0]
    assert counts.tolist() == [5, 3, 1, 3]
    assert np.isneginf(masked[0, 1:]).all() and masked[0, 0] == 1.0
    assert np.isneginf(masked[3, [0, 1, 3]]).all() and masked[3, 2] == 0.0


def test_select_topk_two_source_and_k_equals_e():
    """The two-source form reads combine weights from the second array (llama.cpp exp_probs_b); with k = E and
    distinct finite scores every expert is picked once, in descending score order."""
    rng = np.random.default_rng(5)
    sel = rng.standard_normal((6, 8)).astype(np.float32)
    w = rng.random((6, 8)).astype(np.float32)
    re, rp, counts, _ = M.select_topk(sel, 8, weights=w)
    for s in range(6):
        order = np.argsort(-sel[s], kind="stable")
        assert re[8 * s:8 * s + 8].tolist() == order.tolist()
        assert rp[8 * s:8 * s + 8].tolist() == w[s, order].tolist()
    assert counts.tolist() == [6] * 8


def test_select_topk_softmax_and_normalize():
    """gpt-oss's softmax over the k selected logits (GptOss.java:320-345): equal logits give 1/k each (times
    expertWeightsScale), a logit 100 above the rest takes all the weight; normalizeTopP sums to one; the
    expertScale fold multiplies each route's weight by its expert's scale."""
    sel = np.array([[2.0, 2.0, 2.0, 2.0, -5.0], [100.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    _, rp, _, _ = M.select_topk(sel, 4, mode=M.TOPK_SOFTMAX)
    assert rp[:4].tolist() == [0.25] * 4
    assert rp[4] == 1.0 and (rp[5:8] == np.float32(np.exp(-100.0))).all()
    _, rp2, _, _ = M.select_topk(sel, 4, mode=M.TOPK_SOFTMAX, weights_scale=2.0)
    assert rp2[:4].tolist() == [0.5] * 4
    w = np.array([[0.1, 0.2, 0.3, 0.4, 0.0]], np.float32)
    re, rp3, _, _ = M.select_topk(w, 2, mode=M.TOPK_NORMALIZE)
    assert re.tolist() == [3, 2]
    assert rp3.tolist() == [np.float32(np.float32(0.4) / np.float32(np.float32(0.4) + np.float32(0.3))),
                            np.float32(np.float32(0.3) / np.float32(np.float32(0.4) + np.float32(0.3)))]
    scale = np.array([1.0, 1.0, 0.5, 4.0, 1.0], np.float32)
    _, rp4, _, _ = M.select_topk(w, 2, expert_scale=scale)
    assert rp4.tolist() == [np.float32(0.4) * np.float32(4.0), np.float32(0.3) * np.float32(0.5)]


def test_select_topk_invariants():
    """Random rows: the selected scores are non-increasing along k, the experts of a row distinct, counts sum to
    rows*k, the masked array holds -Inf exactly at the picks, and the softmax weights of a row sum to 1 within
    f32 rounding."""
    rng = np.random.default_rng(11)
    sel = rng.standard_normal((64, 32)).astype(np.float32)
    re, rp, counts, masked = M.select_topk(sel, 4)
    re2 = re.reshape(64, 4)
    assert all(len(set(r)) == 4 for r in re2.tolist())
    assert (np.diff(rp.reshape(64, 4), axis=1) <= 0).all()
    assert counts.sum() == 256 and np.array_equal(counts, np.bincount(re, minlength=32))
    picked = np.array([[e in set(r) for e in range(32)] for r in re2.tolist()])
    assert np.array_equal(np.isneginf(masked), picked)
    _, sm, _, _ = M.select_topk(sel, 4, mode=M.TOPK_SOFTMAX)
    assert np.allclose(sm.reshape(64, 4).sum(axis=1), 1.0, atol=4e-7)
