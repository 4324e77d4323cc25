"""GPU parity of the MoE entry points (jamhip_moe_route / _gather / _combine / jamhip_mm_grouped) against the
restatement of jinfer's Moe.dispatch (oracle/moe.py) and per-expert jam matmuls (the int8 oracle).

Routing, gather and combine are bit-exact; the grouped matmul meets the tier-1 bound of the single-matrix
tests (|gpu - oracle| <= 1e-3*|oracle| + 1e-5*sumAbs) on every expert, whichever path (F1 decode, F2 bands
on the matrix cores or on the decode kernels) its row count selects.
"""
import sys

import numpy as np
import pytest

from oracle import moe as M
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def routes(seed, seq, topk, E):
    rng = np.random.default_rng(seed)
    return np.stack([rng.permutation(E)[:topk] for _ in range(seq)]).astype(np.int32).ravel()


def dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def test_route_gather_combine_bit_exact(hip):
    import torch
    # 257..16384 routes with at most 256 experts take the chunked one-launch routing (each chunk counts every
    # route itself), more the chunked two-kernel routing, up to 64 routes over up to 64 experts the one-wave
    # kernel, the rest the single-workgroup kernel (chunks of 1024: the last case takes five); all must give
    # Moe.dispatch's slots
    for seed, seq, topk, E in ((1, 37, 4, 8), (2, 300, 2, 32), (3, 5, 1, 3), (4, 700, 4, 32), (5, 1100, 4, 64),
                               (6, 300, 4, 16), (7, 200, 2, 300), (8, 512, 4, 256), (9, 16, 4, 64), (10, 1, 4, 32),
                               (11, 8, 2, 80), (12, 4200, 4, 32), (13, 4100, 4, 48)):
        say(f"moe route seq={seq} topk={topk} E={E}")
        re = routes(seed, seq, topk, E)
        if seed == 3:
            re[2] = E + 5                        # an id outside [0, E) takes no slot
        if seed == 9:
            re[5], re[63] = -1, E                # the same in the one-wave kernel (its last lane too)
        if seed == 6:                            # the same in the chunked form, in two different chunks
            re[7], re[1000] = -1, E + 3
        if seed == 12:                           # and in the two-kernel form
            re[9], re[16000] = -2, E
        R = seq * topk
        counts = torch.zeros(E, dtype=torch.int32, device="cuda")
        off = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
        slot_route = torch.full((R,), -1, dtype=torch.int32, device="cuda")
        route_slot = torch.zeros(R, dtype=torch.int32, device="cuda")
        re_d = dev(re)
        assert hip.moe_route(re_d.data_ptr(), seq, topk, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                             route_slot.data_ptr()) == 0, hip.last_error()
        hip.synchronize()
        c_o, off_o, sr_o, rs_o = M.dispatch_csr(re, E)
        total = int(off_o[-1])
        assert np.array_equal(counts.cpu().numpy(), c_o)
        assert np.array_equal(off.cpu().numpy(), off_o)
        assert np.array_equal(slot_route.cpu().numpy()[:total], sr_o[:total])
        assert np.array_equal(route_slot.cpu().numpy(), rs_o)

        dim = 96
        x = np.random.default_rng(seed + 10).standard_normal((seq, dim)).astype(np.float32)
        g = torch.zeros((R, dim + 3), dtype=torch.float32, device="cuda")
        x_dv = dev(x)   # held until the kernels that read it have run
        assert hip.moe_gather(x_dv.data_ptr(), dim, slot_route.data_ptr(), off.data_ptr(), E, seq, topk, dim,
                              g.data_ptr(), dim + 3) == 0, hip.last_error()
        hip.synchronize()
        assert np.array_equal(g.cpu().numpy()[:total, :dim], M.gather(x, sr_o, total, topk))

        y = np.random.default_rng(seed + 20).standard_normal((R, dim)).astype(np.float32)
        prob = np.random.default_rng(seed + 30).random(R).astype(np.float32)
        out = torch.full((seq, dim + 1), 7.0, dtype=torch.float32, device="cuda")
        y_dv = dev(y)   # held until the kernels that read it have run
        prob_dv = dev(prob)   # held until the kernels that read it have run
        assert hip.moe_combine(y_dv.data_ptr(), dim, re_d.data_ptr(), prob_dv.data_ptr(), route_slot.data_ptr(),
                               seq, topk, E, dim, out.data_ptr(), dim + 1) == 0, hip.last_error()
        hip.synchronize()
        want = M.combine(y, re, prob, rs_o, seq, topk, E)
        got = out.cpu().numpy()
        assert np.array_equal(got[:, :dim].view(np.uint32), want.view(np.uint32))
        assert (got[:, dim] == 7.0).all()           # the stride gap is untouched

        # contiguous 16-byte-aligned rows (the four-wide copy and fma paths)
        g4 = torch.zeros((R, dim), dtype=torch.float32, device="cuda")
        x_dv = dev(x)   # held until the kernels that read it have run
        assert hip.moe_gather(x_dv.data_ptr(), dim, slot_route.data_ptr(), off.data_ptr(), E, seq, topk, dim,
                              g4.data_ptr(), dim) == 0, hip.last_error()
        out4 = torch.zeros((seq, dim), dtype=torch.float32, device="cuda")
        y_dv = dev(y)   # held until the kernels that read it have run
        prob_dv = dev(prob)   # held until the kernels that read it have run
        assert hip.moe_combine(y_dv.data_ptr(), dim, re_d.data_ptr(), prob_dv.data_ptr(), route_slot.data_ptr(),
                               seq, topk, E, dim, out4.data_ptr(), dim) == 0, hip.last_error()
        hip.synchronize()
        assert np.array_equal(g4.cpu().numpy()[:total], M.gather(x, sr_o, total, topk))
        assert np.array_equal(out4.cpu().numpy().view(np.uint32), want.view(np.uint32))


# (dtype, m rows per expert, k): m % 32 == 0 takes the matrix cores (k % 256 for the K-quants; MXFP4 pads k
# to 256); m = 48 takes the decode kernels' F2 tiles.
GROUPED = [(O.MXFP4, 64, 576), (O.MXFP4, 48, 320), (O.Q4_K, 96, 512), (O.Q6_K, 64, 256), (O.Q8_0, 64, 320),
           (O.Q4_0, 48, 256)]
# Expert row counts. DENSE (rows_cap >= 8 per expert) takes the one-launch prep on the matrix-core shapes, its
# 1..7-row experts quantized with F1 inside the GEMM's slots; SPARSE (fewer rows than 8 per expert) keeps the
# offsets kernel and the F1 decode kernel for its small experts.
COUNTS = [0, 1, 7, 8, 9, 33, 64, 70, 3]
SPARSE = [0, 1, 0, 0, 9, 0, 2, 0, 0, 0, 0, 0, 33, 0]


@pytest.mark.parametrize("counts", [COUNTS, SPARSE], ids=["dense", "sparse"])
@pytest.mark.parametrize("dt,m,k", GROUPED)
def test_mm_grouped_parity(hip, oracle, dt, m, k, counts):
    import torch
    from qxotic_amd.jam import JAM, Segment
    COUNTS = counts
    E = len(COUNTS)
    say(f"grouped {O.NAMES[dt]} m={m} k={k} counts={COUNTS}")
    w_e = [oracle.quantize(dt, oracle.normal(0x5A11C0DE ^ (100 * e + dt), (m, k), 0.0, 0.02)) for e in range(E)]
    w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
    total = sum(COUNTS)
    rows_cap = total + 5
    a = oracle.outliers(77, (rows_cap, k))
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
    try:
        a_d = dev(a)
        c = torch.full((rows_cap, m + 2), -3.0, dtype=torch.float32, device="cuda")
        cnt = dev(np.array(COUNTS, np.int32))
        off = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
        st = hip.mm_grouped(Segment.of(w), dt, k, m, E, cnt.data_ptr(), a_d.data_ptr(), k, c.data_ptr(), m + 2, k,
                            rows_cap, off.data_ptr())
        assert st == JAM.OK, hip.last_error()
        hip.synchronize()
        got = c.cpu().numpy()
        assert np.array_equal(off.cpu().numpy(), np.concatenate([[0], np.cumsum(COUNTS)]))
        ref = M.mm_grouped(oracle, dt, w_e, a, COUNTS, m, k)
        o = 0
        for e, n in enumerate(COUNTS):
            if n:
                _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(a[o:o + n]), m, n, k)
                r = ref[o:o + n]
                ok = np.abs(got[o:o + n, :m] - r) <= 1e-3 * np.abs(r) + 1e-5 * sa
                assert ok.all(), (O.NAMES[dt], e, n, float(np.max(np.abs(got[o:o + n, :m] - r))))
            o += n
        assert (got[:, m:] == -3.0).all()           # ldc gap untouched
        assert (got[total:] == -3.0).all()          # rows past the counts untouched
        # rerun bit-identity
        c2 = torch.zeros_like(c)
        assert hip.mm_grouped(Segment.of(w), dt, k, m, E, cnt.data_ptr(), a_d.data_ptr(), k, c2.data_ptr(), m + 2, k,
                              rows_cap, None) == JAM.OK
        hip.synchronize()
        assert np.array_equal(c2.cpu().numpy()[:total, :m], got[:total, :m])
    finally:
        hip.evict(Segment.of(w))


@pytest.mark.parametrize("seq,topk,E", [(200, 4, 8), (24, 4, 32), (2, 4, 16)], ids=["dense", "mid", "sparse"])
@pytest.mark.parametrize("dt,m,k,native", [(O.MXFP4, 64, 576, 0), (O.MXFP4, 64, 576, 2), (O.Q4_K, 96, 512, 0),
                                           (O.MXFP4, 48, 320, 0), (O.MXFP4, 48, 320, 2)])
def test_mm_grouped_gather_matches_two_calls(hip, oracle, dt, m, k, native, seq, topk, E):
    """jamhip_mm_grouped_gather (CSR row r of A = row slot_route[r] / topk of x) is bit-identical to
    jamhip_moe_gather followed by jamhip_mm_grouped_ex, offsets included: the fused preps reading x themselves
    (dense: rows_cap >= 8 per expert on the matrix cores, jam's path and native MX mode 2) and the paths that
    gather into scratch first (mid: F1 decode + matrix cores; sparse: F1 decode only; m = 48: F2 tiles); x
    with a row pitch above k, expert biases on the dense case."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    say(f"grouped gather {O.NAMES[dt]} m={m} k={k} seq={seq} topk={topk} E={E} native={native}")
    R = seq * topk
    re = routes(0xC0DE + seq + E, seq, topk, E)
    w = oracle.quantize(dt, oracle.normal(0x5A11C0DE ^ (31 * E + dt), (E * m, k), 0.0, 0.02))
    ldx = k + 4
    x = np.zeros((seq, ldx), np.float32)
    x[:, :k] = oracle.outliers(91 + seq, (seq, k))
    bias = oracle.normal(93, (E, m)) if seq == 200 else None
    i32 = lambda n: torch.zeros(n, dtype=torch.int32, device="cuda")
    counts, off, slot_route, route_slot = i32(E), i32(E + 1), i32(R), i32(R)
    re_d, x_d = dev(re), dev(x)
    b_d = dev(bias) if bias is not None else None
    g = torch.zeros((R, k), dtype=torch.float32, device="cuda")
    ca = torch.full((R, m + 1), -3.0, dtype=torch.float32, device="cuda")
    cb = torch.full((R, m + 1), -3.0, dtype=torch.float32, device="cuda")
    offa, offb = i32(E + 1), i32(E + 1)
    torch.cuda.synchronize()   # the inputs are written on torch's stream; the library runs on its own
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
    assert hip.set_mx_native(native) == JAM.OK
    try:
        assert hip.moe_route(re_d.data_ptr(), seq, topk, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                             route_slot.data_ptr()) == JAM.OK, hip.last_error()
        assert hip.moe_gather(x_d.data_ptr(), ldx, slot_route.data_ptr(), off.data_ptr(), E, seq, topk, k,
                              g.data_ptr(), k) == JAM.OK, hip.last_error()
        bp = b_d.data_ptr() if b_d is not None else None
        assert hip.mm_grouped_ex(Segment.of(w), dt, k, m, E, counts.data_ptr(), g.data_ptr(), k, ca.data_ptr(), m + 1,
                                 k, R, offa.data_ptr(), bp) == JAM.OK, hip.last_error()
        assert hip.mm_grouped_gather(Segment.of(w), dt, k, m, E, counts.data_ptr(), x_d.data_ptr(), ldx,
                                     slot_route.data_ptr(), topk, cb.data_ptr(), m + 1, k, R, offb.data_ptr(),
                                     bp) == JAM.OK, hip.last_error()
        hip.synchronize()
        got_a, got_b = ca.cpu().numpy(), cb.cpu().numpy()
        assert np.array_equal(offa.cpu().numpy(), offb.cpu().numpy())
        assert (got_a[:, m:] == -3.0).all() and (got_b[:, m:] == -3.0).all()
        assert np.array_equal(got_a.view(np.uint32), got_b.view(np.uint32))
    finally:
        hip.set_mx_native(0)
        assert hip.evict(Segment.of(w)) == JAM.OK


def test_mm_grouped_counts_past_rows_cap(hip, oracle):
    """Counts whose sum exceeds rows_cap: the rows past rows_cap are neither read nor written."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    dt, m, k, E = O.MXFP4, 32, 256, 3
    w_e = [oracle.quantize(dt, oracle.normal(900 + e, (m, k), 0.0, 0.02)) for e in range(E)]
    w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
    counts = [10, 40, 30]
    rows_cap = 45                                    # expert 1 keeps 35 rows, expert 2 none
    a = oracle.normal(901, (rows_cap, k))
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK
    try:
        c = torch.full((rows_cap, m), -3.0, dtype=torch.float32, device="cuda")
        off = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
        a_dv = dev(a)   # held until the kernels that read it have run
        counts_dv = dev(np.array(counts, np.int32))
        torch.cuda.synchronize()   # torch's fills run on its own stream
        assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts_dv.data_ptr(),
                              a_dv.data_ptr(), k, c.data_ptr(), m, k, rows_cap, off.data_ptr()) == JAM.OK
        hip.synchronize()
        assert off.cpu().numpy().tolist() == [0, 10, 45, 45]
        ref = M.mm_grouped(oracle, dt, w_e, a, [10, 35, 0], m, k)
        got = c.cpu().numpy()
        _, sa = oracle.mm_ref(dt, w_e[1], np.ascontiguousarray(a[10:45]), m, 35, k)
        assert (np.abs(got[10:45] - ref[10:45]) <= 1e-3 * np.abs(ref[10:45]) + 1e-5 * sa).all()
    finally:
        hip.evict(Segment.of(w))


@pytest.mark.parametrize("k,pad", [(512, 0), (5120, 0), (512, 1)])
@pytest.mark.parametrize("dt", [O.MXFP4, O.Q4_K])
def test_mm_grouped_decode_sized(hip, oracle, dt, k, pad):
    """Decode-time MoE: fewer than 8 rows in all (one token, top-4 and a ragged cap), so every expert takes
    jam's F1 and only the F1 decode launch runs; rows and the ldc gap past the counts stay untouched.
    k = 512 with lda = k quantizes the activations inside the decode kernels; k = 5120 (too long for the
    seven-token kernel's fused prologue) and lda = k + 1 (rows not 16-byte aligned) quantize them in a
    separate launch and the kernels read the codes at each expert's CSR offset."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, lda = 64, k + pad
    for counts, rows_cap in (([1, 0, 1, 0, 1, 1], 4), ([0, 3, 0, 2, 0, 0, 1], 7)):
        E = len(counts)
        say(f"grouped decode-sized {O.NAMES[dt]} k={k} lda={lda} counts={counts} rows_cap={rows_cap}")
        w_e = [oracle.quantize(dt, oracle.normal(0xDEC0 + 31 * e + dt, (m, k), 0.0, 0.02)) for e in range(E)]
        w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
        a = oracle.outliers(0xDEC1 + E + k, (rows_cap, k))
        a_pad = np.full((rows_cap, lda), np.nan, np.float32)   # the gap past k is never read
        a_pad[:, :k] = a
        assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
        try:
            c = torch.full((rows_cap + 1, m + 2), -3.0, dtype=torch.float32, device="cuda")
            off = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
            a_dv = dev(a_pad)   # held until the kernels that read it have run
            counts_dv = dev(np.array(counts, np.int32))
            torch.cuda.synchronize()   # torch's fills run on its own stream
            assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts_dv.data_ptr(), a_dv.data_ptr(), lda,
                                  c.data_ptr(), m + 2, k, rows_cap, off.data_ptr()) == JAM.OK, hip.last_error()
            hip.synchronize()
            total = sum(counts)
            assert off.cpu().numpy().tolist() == [0] + np.cumsum(counts).tolist()
            got = c.cpu().numpy()
            ref = M.mm_grouped(oracle, dt, w_e, a, counts, m, k)
            o = 0
            for e, n in enumerate(counts):
                if n:
                    _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(a[o:o + n]), m, n, k)
                    r = ref[o:o + n]
                    assert (np.abs(got[o:o + n, :m] - r) <= 1e-3 * np.abs(r) + 1e-5 * sa).all(), (e, n)
                o += n
            assert (got[:, m:] == -3.0).all()
            assert (got[total:] == -3.0).all()
        finally:
            hip.evict(Segment.of(w))


@pytest.mark.parametrize("E", [150, 300])
def test_mm_grouped_many_experts(hip, oracle, E):
    """More than 64 experts, small and large experts mixed, and counts past rows_cap: offsets are the clamped
    prefix sums, every kept row meets the bound. 150 experts take the one-launch prep (its expert table spans
    the workgroup's four waves); 300 experts (more than the prep's 256) the offsets kernel and the F1 decode
    kernel for the small experts."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    dt, m, k = O.Q4_K, 32, 256
    rng = np.random.default_rng(4242)
    counts = rng.integers(0, 16, E)
    counts[rng.permutation(E)[:30]] = 0
    counts[[3, 77, 140]] = [170, 130, 66]            # several 64-slot blocks each
    counts[[5, 6, 90, 149]] = [1, 7, 2, 5]           # F1 experts (E = 150: the last one loses its rows)
    total = int(counts.sum())
    rows_cap = total - 9                             # the last experts lose rows
    assert (rows_cap >= 8 * E) == (E <= 256)
    kept, o = [], 0
    for n in counts:
        kept.append(max(0, min(int(n), rows_cap - o)))
        o += int(n)
    say(f"grouped many experts E={E} total={total} rows_cap={rows_cap}")
    w_e = [oracle.quantize(dt, oracle.normal(7000 + e, (m, k), 0.0, 0.02)) for e in range(E)]
    w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
    a = oracle.outliers(78, (rows_cap, k))
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
    try:
        c = torch.full((rows_cap, m), -3.0, dtype=torch.float32, device="cuda")
        off = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
        a_dv = dev(a)   # held until the kernels that read it have run
        counts_dv = dev(counts.astype(np.int32))
        torch.cuda.synchronize()   # torch's fills run on its own stream
        assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts_dv.data_ptr(), a_dv.data_ptr(), k, c.data_ptr(), m,
                              k, rows_cap, off.data_ptr()) == JAM.OK, hip.last_error()
        hip.synchronize()
        assert off.cpu().numpy().tolist() == [0] + np.cumsum(kept).tolist()
        ref = M.mm_grouped(oracle, dt, w_e, a, kept, m, k)
        got = c.cpu().numpy()
        o = 0
        for e, n in enumerate(kept):
            if n:
                _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(a[o:o + n]), m, n, k)
                r = ref[o:o + n]
                ok = np.abs(got[o:o + n] - r) <= 1e-3 * np.abs(r) + 1e-5 * sa
                assert ok.all(), (e, n, float(np.max(np.abs(got[o:o + n] - r))))
            o += n
    finally:
        hip.evict(Segment.of(w))


def test_grouped_status_codes(hip):
    import torch
    from qxotic_amd.jam import JAM, Segment
    w = np.zeros(17 * 8 * 40, np.uint8)
    z = torch.zeros(64, dtype=torch.int32, device="cuda")
    f = torch.zeros((64, 64), dtype=torch.float32, device="cuda")
    call = lambda **kw: hip.mm_grouped(Segment.of(w), kw.get("dt", JAM.MXFP4), 256, kw.get("m", 32), kw.get("E", 2),
                                       z.data_ptr(), f.data_ptr(), 256, f.data_ptr(), kw.get("ldc", 32), 256,
                                       kw.get("cap", 4), None)
    assert call(m=24) == JAM.EUNSUPPORTED           # m % 16
    assert call(E=2000) == JAM.EUNSUPPORTED         # more than 1024 experts
    assert call(E=1024, cap=1 << 21) == JAM.EUNSUPPORTED   # n_experts·rows_cap = 2^31: the prefix sums overflow
    assert call(ldc=16) == JAM.EINVAL               # ldc < m
    assert call(cap=-1) == JAM.EINVAL
    assert call(dt=JAM.F16) == JAM.EUNSUPPORTED
    gcall = lambda sr, topk: hip.mm_grouped_gather(Segment.of(w), JAM.MXFP4, 256, 32, 2, z.data_ptr(), f.data_ptr(),
                                                   256, sr, topk, f.data_ptr(), 32, 256, 4, None, None)
    assert gcall(None, 4) == JAM.EINVAL              # no slot_route
    assert gcall(z.data_ptr(), 0) == JAM.EINVAL      # topk < 1


@pytest.mark.parametrize("dt", [O.MXFP4, O.Q4_K])
def test_mm_grouped_decode_counts_derived(hip, oracle, dt):
    """Decode-sized calls without an offsets output: the F1 kernels find their experts and rows from the device
    counts (no offsets launch, at most 64 experts). Each case is run with and without the offsets output (the
    offsets-kernel path); both must give bit-identical C, equal to the oracle on the kept rows, with the
    counts clamped as the offsets kernel clamps them (rows past rows_cap dropped, an expert cut short), 64
    experts (the most a wave holds) and 70 (past it: the offsets kernel runs either way)."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, k = 32, 512
    c64 = np.zeros(64, np.int64)
    c64[[3, 17, 40, 63]] = [1, 2, 1, 3]
    c70 = np.zeros(70, np.int64)
    c70[[2, 65, 69]] = [2, 1, 1]
    for counts, rows_cap in (([2, 0, 5, 1], 5), ([1, 1, 0, 9], 4), (c64.tolist(), 7), (c70.tolist(), 4)):
        E = len(counts)
        c0 = np.clip(np.array(counts), 0, rows_cap)
        o = np.concatenate([[0], np.cumsum(c0)[:-1]])
        kept = np.maximum(0, np.minimum(c0, rows_cap - o)).tolist()
        say(f"grouped decode derived {O.NAMES[dt]} E={E} rows_cap={rows_cap} kept={[x for x in kept if x]}")
        w_e = [oracle.quantize(dt, oracle.normal(0xDE71 + 7 * e + dt, (m, k), 0.0, 0.02)) for e in range(E)]
        w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
        a = oracle.outliers(0xDE72 + E + rows_cap, (rows_cap, k))
        assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
        try:
            a_dv = dev(a)
            counts_dv = dev(np.array(counts, np.int32))
            outs = []
            for with_off in (False, True):
                c = torch.full((rows_cap + 1, m + 2), -3.0, dtype=torch.float32, device="cuda")
                off = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
                torch.cuda.synchronize()
                assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts_dv.data_ptr(), a_dv.data_ptr(), k,
                                      c.data_ptr(), m + 2, k, rows_cap,
                                      off.data_ptr() if with_off else None) == JAM.OK, hip.last_error()
                hip.synchronize()
                outs.append(c.cpu().numpy())
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
            got = outs[0]
            ref = M.mm_grouped(oracle, dt, w_e, a, kept, m, k)
            r0 = 0
            for e, n in enumerate(kept):
                if n:
                    _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(a[r0:r0 + n]), m, n, k)
                    r = ref[r0:r0 + n]
                    assert (np.abs(got[r0:r0 + n, :m] - r) <= 1e-3 * np.abs(r) + 1e-5 * sa).all(), (e, n)
                r0 += n
            assert (got[r0:] == -3.0).all() and (got[:, m:] == -3.0).all()
        finally:
            hip.evict(Segment.of(w))


@pytest.mark.parametrize("dt", [O.MXFP4, O.Q4_K])
def test_mm_grouped_decode_unfused(hip, oracle, dt):
    """The grouped F1 decode kernels reading the quantized copy instead of quantizing in their prologue: k past
    the fused prologue's reach (k = 5120, 14336) and rows not 16-byte aligned (lda = k + 1), with one-row and
    2..7-row experts (the one-token and seven-token launches). Tier 1 on every expert, the ldc gap and the rows
    past the counts untouched."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    m = 32
    for k, lda in ((5120, 5120), (14336, 14336), (2816, 2817)):
        counts, rows_cap = [1, 0, 3, 1, 0, 2], 7
        E = len(counts)
        say(f"grouped unfused {O.NAMES[dt]} k={k} lda={lda} counts={counts}")
        w_e = [oracle.quantize(dt, oracle.normal(0xF1D0 + 13 * e + dt + k, (m, k), 0.0, 0.02)) for e in range(E)]
        w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
        a = oracle.outliers(0xF1D1 + k, (rows_cap, k))
        a_pad = np.zeros((rows_cap, lda), np.float32)
        a_pad[:, :k] = a
        assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
        try:
            c = torch.full((rows_cap + 1, m + 2), -3.0, dtype=torch.float32, device="cuda")
            a_dv = dev(a_pad)
            counts_dv = dev(np.array(counts, np.int32))
            torch.cuda.synchronize()
            assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts_dv.data_ptr(), a_dv.data_ptr(), lda,
                                  c.data_ptr(), m + 2, k, rows_cap, None) == JAM.OK, hip.last_error()
            hip.synchronize()
            got = c.cpu().numpy()
            ref = M.mm_grouped(oracle, dt, w_e, a, counts, m, k)
            o = 0
            for e, n in enumerate(counts):
                if n:
                    _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(a[o:o + n]), m, n, k)
                    r = ref[o:o + n]
                    assert (np.abs(got[o:o + n, :m] - r) <= 1e-3 * np.abs(r) + 1e-5 * sa).all(), (k, e, n)
                o += n
            assert (got[:, m:] == -3.0).all()
            assert (got[sum(counts):] == -3.0).all()
        finally:
            hip.evict(Segment.of(w))


def _topk_case(hip, sel, topk, mode, weights=None, wscale=1.0, escale=None, ld=None):
    import torch
    rows, E = sel.shape
    ld = ld or E
    s_pad = np.full((rows, ld), 5.5, np.float32)
    s_pad[:, :E] = sel
    sd = dev(s_pad)
    wd = None
    if weights is not None:
        w_pad = np.zeros((rows, ld), np.float32)
        w_pad[:, :E] = weights
        wd = dev(w_pad)
    ed = dev(np.asarray(escale, np.float32)) if escale is not None else None
    re = torch.full((rows * topk,), -7, dtype=torch.int32, device="cuda")
    rp = torch.zeros(rows * topk, dtype=torch.float32, device="cuda")
    cnt = torch.full((E,), 99, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    st = hip.moe_select_topk(sd.data_ptr(), None if wd is None else wd.data_ptr(), rows, E, ld, topk, mode,
                             re.data_ptr(), rp.data_ptr(), cnt.data_ptr(), wscale,
                             None if ed is None else ed.data_ptr())
    assert st == 0, hip.last_error()
    hip.synchronize()
    got_sel = sd.cpu().numpy()
    assert (got_sel[:, E:] == 5.5).all()          # the row stride's gap is untouched
    return re.cpu().numpy(), rp.cpu().numpy(), cnt.cpu().numpy(), got_sel[:, :E]


def _topk_check(got, sel, topk, **kw):
    re, rp, cnt, masked = got
    re_o, rp_o, cnt_o, masked_o = M.select_topk(sel, topk, **kw)
    assert np.array_equal(re, re_o)
    # bit for bit, NaN payloads aside (a NaN weight reaching the softmax makes the row's weights NaN, whose payload
    # neither Java nor IEEE arithmetic pins)
    same = (rp.view(np.uint32) == rp_o.view(np.uint32)) | (np.isnan(rp) & np.isnan(rp_o))
    assert same.all(), np.flatnonzero(~same)[:5]
    assert np.array_equal(cnt, cnt_o)
    assert np.array_equal(masked.view(np.uint32), masked_o.view(np.uint32))


def test_select_topk_bit_exact(hip):
    """jamhip_moe_select_topk against oracle/moe.py's select_topk (Moe.selectTopK, gpt-oss's softmax over the
    selected logits, normalizeTopP, the expertScale fold), bit for bit: routes, weights, counts and the
    consumed selection array. Config 5's router (512 tokens x 32 experts, top-4, Zipf(1.1) popularity by
    Gumbel-top-k on log p_e), one- and two-source forms, a row stride above E, and hand-made edge rows
    (ties, all -Inf, NaN); E = 16 with k = 16 (every expert), E = 300 and 1024 (more scores per lane)."""
    rng = np.random.default_rng(0x5A11C0DE ^ 5)
    E, SEQ, TOPK = 32, 512, 4
    logp = -1.1 * np.log(np.arange(1, E + 1))
    logits = (logp[None, :] + rng.gumbel(size=(SEQ, E))).astype(np.float32)
    logits[0, 3] = logits[0, 7] = np.float32(50.0)          # a tie: expert 3 first
    logits[1] = -np.inf                                     # nothing above -Inf: expert 0 each pass
    logits[2, :5] = np.nan                                  # NaN never wins
    logits[3] = np.float32(0.25)                            # all equal
    logits[4] = -np.inf                                     # two scores above -Inf, NaN at expert 0: passes 3
    logits[4, 0], logits[4, 9], logits[4, 20] = np.nan, 1.0, 2.0   # and 4 fall back to expert 0 (NaN, then -Inf)
    logits[5] = -np.inf                                     # expert 0 wins first, then only the fallback
    logits[5, 0] = 3.0
    logits[6, 1], logits[6, 2] = np.float32(-0.0), np.float32(0.0)  # -0 == +0: a tie, the lower expert first
    logits[6, 5:] = -1.0
    logits[6, 0] = -1.0
    logits[6, 3:5] = -1.0
    logits[7, 30], logits[7, 31] = np.inf, np.inf           # +Inf wins, ties by expert
    w = rng.random((SEQ, E)).astype(np.float32)
    scale = (0.5 + rng.random(E)).astype(np.float32)
    for mode in (M.TOPK_RAW, M.TOPK_SOFTMAX, M.TOPK_NORMALIZE):
        say(f"topk config5 mode={mode}")
        _topk_check(_topk_case(hip, logits, TOPK, mode), logits, TOPK, mode=mode)
        _topk_check(_topk_case(hip, logits, TOPK, mode, weights=w, wscale=0.75, escale=scale, ld=E + 3), logits,
                    TOPK, weights=w, mode=mode, weights_scale=0.75, expert_scale=scale)
    re, _, cnt, _ = _topk_case(hip, logits, TOPK, M.TOPK_SOFTMAX)
    c_o, _, _, _ = M.dispatch_csr(re, E)
    assert np.array_equal(cnt, c_o)                        # the counts jamhip_moe_route builds from the routes
    for E2, k2, seq in ((16, 16, 40), (300, 8, 70), (1024, 16, 9)):
        say(f"topk E={E2} k={k2}")
        sel = rng.standard_normal((seq, E2)).astype(np.float32)
        sel[0, E2 - 1] = np.float32(9.0)                  # the last lane's last score
        for mode in (M.TOPK_RAW, M.TOPK_SOFTMAX):
            _topk_check(_topk_case(hip, sel, k2, mode), sel, k2, mode=mode)


def test_select_topk_status_codes(hip):
    import torch
    f = torch.zeros((8, 64), dtype=torch.float32, device="cuda")
    i = torch.zeros(64, dtype=torch.int32, device="cuda")
    call = lambda **kw: hip.moe_select_topk(f.data_ptr(), None, kw.get("rows", 4), kw.get("E", 8), kw.get("ld", 8),
                                            kw.get("k", 2), kw.get("mode", 0), i.data_ptr(), f.data_ptr(), None)
    assert call() == 0
    assert call(ld=7) == 1                      # EINVAL: ld < E
    assert call(mode=3) == 1
    assert call(k=0) == 1
    assert call(k=17) == 2                      # EUNSUPPORTED: topk above 16
    assert call(E=2000, ld=2000) == 2
    hip.synchronize()


@pytest.mark.parametrize("dt", [O.MXFP4, O.Q4_K])
def test_decode_sized_gather_folded(hip, oracle, dt):
    """Decode-sized grouped calls with the gather folded in: the fused F1 prologue reads each slot's token row
    through slot_route / topk itself (one-token and seven-token bodies: 3 tokens top-2 give experts of 1, 2 and
    3 rows; 1 token top-4 gives four 1-row experts). Bit-identical to jamhip_moe_gather + jamhip_mm_grouped."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, k, E = 32, 512, 6
    w_e = [oracle.quantize(dt, oracle.normal(0x6A7E + 5 * e + dt, (m, k), 0.0, 0.02)) for e in range(E)]
    w = np.ascontiguousarray(np.concatenate(w_e, axis=0))
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
    try:
        for re, topk in (([[1, 3], [3, 5], [1, 3]], 2), ([[4, 0, 2, 5]], 4)):
            seq, R = len(re), len(re) * topk
            say(f"decode-sized gather folded {O.NAMES[dt]} seq={seq} topk={topk}")
            x = oracle.outliers(0x6A7F + seq, (seq, k))
            i32 = lambda n: torch.zeros(n, dtype=torch.int32, device="cuda")
            counts, off, slot_route, route_slot = i32(E), i32(E + 1), i32(R), i32(R)
            re_d, x_d = dev(np.array(re, np.int32).ravel()), dev(x)
            g = torch.zeros((R, k), dtype=torch.float32, device="cuda")
            ca = torch.full((R + 1, m), -3.0, dtype=torch.float32, device="cuda")
            cb = torch.full((R + 1, m), -3.0, dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            assert hip.moe_route(re_d.data_ptr(), seq, topk, E, counts.data_ptr(), off.data_ptr(),
                                 slot_route.data_ptr(), route_slot.data_ptr()) == JAM.OK, hip.last_error()
            assert hip.moe_gather(x_d.data_ptr(), k, slot_route.data_ptr(), off.data_ptr(), E, seq, topk, k,
                                  g.data_ptr(), k) == JAM.OK, hip.last_error()
            assert hip.mm_grouped(Segment.of(w), dt, k, m, E, counts.data_ptr(), g.data_ptr(), k, ca.data_ptr(), m, k,
                                  R) == JAM.OK, hip.last_error()
            assert hip.mm_grouped_gather(Segment.of(w), dt, k, m, E, counts.data_ptr(), x_d.data_ptr(), k,
                                         slot_route.data_ptr(), topk, cb.data_ptr(), m, k, R) == JAM.OK, hip.last_error()
            hip.synchronize()
            a_, b_ = ca.cpu().numpy(), cb.cpu().numpy()
            assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32))
            assert (b_[R:] == -3.0).all()
            cnt, ga = counts.cpu().numpy(), g.cpu().numpy()
            o = 0
            for e in range(E):
                n = int(cnt[e])
                if n:
                    ref = oracle.mm_int8(dt, w_e[e], np.ascontiguousarray(ga[o:o + n]), m, n, k)
                    _, sa = oracle.mm_ref(dt, w_e[e], np.ascontiguousarray(ga[o:o + n]), m, n, k)
                    assert (np.abs(b_[o:o + n] - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa).all(), (e, n)
                o += n
    finally:
        hip.evict(Segment.of(w))
