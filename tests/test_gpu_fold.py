"""GPU: block-scale edges of Q8_0 / Q4_0 / MXFP4 / Q1_0 on every path, and jam's Q8_0 saturation suites.

The matrix-core GEMM folds each block's scale into an f16 weight operand relative to a per-group reference
(qxotic_amd/csrc/mma.hip); the repack (qxotic_amd/csrc/prep.hip, repack_kernel) keeps blocks whose products
are all zero out of that reference and flags tensors whose scales span more than f16 holds, or hold a
non-finite scale, so that they never reach the matrix cores (tests/test_fold_model.py models both on the
CPU). Here the edge cases of that model run through the C-ABI on the decode kernel (F1), the F2 decode
kernel, the matrix cores (staged and pinned), the fallback GEMM (a view not on a 32-row boundary), the
grouped matmul and, for MXFP4, the native-MX mode:
  - every finite output meets the tier-1 bound against the oracle; where jam's result is not finite (an
    MXFP4 e = 255 block, which jam-native decodes as +Inf, jam_mxfp4.h:17-24; an fp16 Inf or NaN scale) the
    GPU's is not finite either;
  - a tensor whose groups all fold exactly takes the matrix cores (its result differs in f32 order from the
    F2 decode kernel's), rows at the accepted limit of the scale spread stay at the error floor there (a
    flushed f16 subnormal would show), and a flagged tensor gives exactly the F2 decode kernel's bits.
Also jam's Q8_0 suites (jam/jam-native/tests/jam_test.c:355-420): weights holding -128 (QuantWeights.java:
108-122), every value at +-127, a huge-dynamic-range activation block, and the adversarial activations
(finite output, a zero column for the all-zero token) on every weight type.
"""
import sys

import numpy as np
import pytest

from oracle import mxnative as X
from oracle import oracle as O
from test_fold_model import decode_group, guard, mx_block, mx_cases, q4_block, q8_block, q_cases, rand_nibs

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def mm_host(hip, dt, w, a, m, n, k, w_off=0, ldw=None):
    from qxotic_amd.jam import JAM, Segment
    c = np.zeros((n, m), np.float32)
    st = hip.mm(Segment.of(w), w_off, dt, ldw or k, Segment.of(a), 0, JAM.F32, k, Segment.of(c), 0, JAM.F32, m, m,
                n, k)
    assert st == JAM.OK, hip.last_error()
    return c


def check(got, ref, sa, label, floor_rows=None):
    """Non-finite where jam is non-finite, tier 1 elsewhere; at floor_rows also the error floor."""
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin), (label, np.argwhere(np.isfinite(got) != fin)[:4].tolist())
    err = np.abs(got.astype(np.float64) - ref)
    ok = err[fin] <= 1e-3 * np.abs(ref[fin]) + 1e-5 * sa[fin]
    assert ok.all(), (label, np.argwhere(fin)[~ok][:4].tolist())
    if floor_rows is not None and len(floor_rows):
        e = err[:, floor_rows] / np.maximum(sa[:, floor_rows], 1e-300)
        assert e.max() <= 4e-6, (label, float(e.max()))


# ------------------------------------------------------------------------------------ edge tensors
def normal_group(dt, rng):
    if dt == O.MXFP4:
        return np.concatenate([mx_block(118 + int(rng.integers(0, 5)), rand_nibs(rng)) for _ in range(8)])
    if dt == O.Q8_0:
        return np.concatenate([q8_block(np.float16(rng.uniform(1e-4, 3e-4)).view(np.uint16),
                                        rng.integers(-127, 128, 32)) for _ in range(8)])
    return np.concatenate([q4_block(np.float16(rng.uniform(2e-3, 6e-3)).view(np.uint16), rand_nibs(rng))
                           for _ in range(8)])


def extra_cases(dt):
    """Non-finite fp16 scales (Q8_0 / Q4_0), beside the model's cases."""
    if dt == O.MXFP4:
        return {}
    rng = np.random.default_rng(99 + dt)
    blk = q8_block if dt == O.Q8_0 else q4_block
    cds = (lambda: rng.integers(-127, 128, 32)) if dt == O.Q8_0 else (lambda: rand_nibs(rng))
    small = np.float16(1e-4 if dt == O.Q8_0 else 3e-3).view(np.uint16)
    return {"Inf scale": (np.concatenate([blk(0x7C00, cds())] + [blk(small, cds()) for _ in range(7)]), ()),
            "NaN scale": (np.concatenate([blk(0x7E00, cds())] + [blk(small, cds()) for _ in range(7)]), ())}


def at_limit(dt):
    """Groups whose small blocks sit exactly at the accepted spread limit (reference block 0)."""
    rng = np.random.default_rng(5 + dt)
    if dt == O.MXFP4:
        return [np.concatenate([mx_block(125, rand_nibs(rng))] + [mx_block(111, rand_nibs(rng)) for _ in range(7)])]
    blk, lim = (q8_block, 36) if dt == O.Q8_0 else (q4_block, 39)
    out = []
    for F in (15, 22):   # fp16 exponent field of the reference scale
        ref = np.float16(2.0 ** (F - 15) * 1.5).view(np.uint16)
        small = np.float16(2.0 ** (F - lim) * 1.99).view(np.uint16)   # 11 significant bits, just above 2^(F-lim)
        cds = (lambda: rng.integers(-128, 128, 32)) if dt == O.Q8_0 else (lambda: rand_nibs(rng))
        out.append(np.concatenate([blk(ref, cds())] + [blk(small, cds()) for _ in range(7)]))
    return out


def edge_tensor(dt, flagged_too):
    """[64, 512-element rows]: each row's group 0 an edge case, group 1 an ordinary group; rows past the
    cases ordinary. Returns (W, limit rows, flagged row count)."""
    rng = np.random.default_rng(0xED6E ^ dt)
    cases = dict(mx_cases() if dt == O.MXFP4 else q_cases(dt))
    cases.update(extra_cases(dt))
    rows, limit, nflag = [], [], 0
    for name, (g0, _) in cases.items():
        scale, codes, nib = decode_group(dt, g0)
        flagged = guard(dt, scale, codes, nib, "new")[2]
        if flagged and not flagged_too:
            continue
        nflag += flagged
        rows.append(np.concatenate([g0, normal_group(dt, rng)]))
    for g0 in at_limit(dt):
        scale, codes, nib = decode_group(dt, g0)
        assert not guard(dt, scale, codes, nib, "new")[2]
        limit.append(len(rows))
        rows.append(np.concatenate([g0, normal_group(dt, rng)]))
    while len(rows) < 64:
        rows.append(np.concatenate([normal_group(dt, rng), normal_group(dt, rng)]))
    return np.ascontiguousarray(np.stack(rows[:64])), limit, nflag


def activation_sets(oracle, n, k, seed):
    """A: N(0,1); B: the same with block 0 and the whole second group zero, so that each case row's result is
    its small blocks alone."""
    a = oracle.normal(seed, (n, k))
    b = a.copy()
    b[:, 0:32] = 0.0
    b[:, 256:] = 0.0
    return {"A": a, "B": np.ascontiguousarray(b)}


@pytest.mark.parametrize("dt", [O.MXFP4, O.Q8_0, O.Q4_0])
def test_fold_edges_every_path(hip, oracle, dt, monkeypatch):
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, k = 64, 512
    for flagged_too in (False, True):
        w, limit, nflag = edge_tensor(dt, flagged_too)
        assert (nflag > 0) == flagged_too
        tag = f"{O.NAMES[dt]} {'with flagged rows' if flagged_too else 'all rows fold exactly'}"
        floor = limit if not flagged_too else None
        for n, force in ((1, None), (3, None), (12, "100000"), (40, "8")):
            for an, a in activation_sets(oracle, n, k, 0xF0 + n).items():
                say(f"fold edges {tag} n={n} mma_min_n={force} acts={an}")
                if force:
                    monkeypatch.setenv("JAM_HIP_MMA_MIN_N", force)
                else:
                    monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
                got = mm_host(hip, dt, w, a, m, n, k)
                ref = oracle.mm_int8(dt, w, a, m, n, k)
                _, sa = oracle.mm_ref(dt, w, a, m, n, k)
                check(got, ref, sa, (tag, n, an), floor if n == 40 else None)
                if n == 40 and an == "A":   # the matrix cores when every group folds, else the F2 decode kernel's bits
                    monkeypatch.setenv("JAM_HIP_NO_MMA", "1")
                    f2 = mm_host(hip, dt, w, a, m, n, k)
                    monkeypatch.delenv("JAM_HIP_NO_MMA")
                    same = np.array_equal(bits(got), bits(f2))
                    assert same == flagged_too, (tag, an, "routing")
        # pinned: the flag kept with the pin; a view at row 16 (not on a 32-row tile) takes the fallback GEMM
        wide = np.ascontiguousarray(np.concatenate([w, w[:16]], axis=0))   # 80 rows
        assert hip.pin(Segment.of(wide), dt, k, 80) == JAM.OK, hip.last_error()
        try:
            rb = O.row_bytes(dt, k)
            for an, a in activation_sets(oracle, 40, k, 0xF7).items():
                monkeypatch.setenv("JAM_HIP_MMA_MIN_N", "8")
                say(f"fold edges {tag} pinned n=40 acts={an}")
                got = mm_host(hip, dt, wide, a, m, 40, k)
                ref = oracle.mm_int8(dt, w, a, m, 40, k)
                _, sa = oracle.mm_ref(dt, w, a, m, 40, k)
                check(got, ref, sa, (tag, "pinned", an), floor)
            monkeypatch.delenv("JAM_HIP_MMA_MIN_N")
            for an, a in activation_sets(oracle, 100, k, 0xF8).items():
                say(f"fold edges {tag} view at row 16, n=100 acts={an}")
                got = mm_host(hip, dt, wide, a, m, 100, k, w_off=16 * rb)
                ws = np.ascontiguousarray(wide[16:80])
                ref = oracle.mm_int8(dt, ws, a, m, 100, k)
                _, sa = oracle.mm_ref(dt, ws, a, m, 100, k)
                check(got, ref, sa, (tag, "view", an))
        finally:
            assert hip.evict(Segment.of(wide)) == JAM.OK
        # grouped: two experts of 32 rows, 40 and 3 rows routed (the one-launch prep: expert 1 quantized with F1
        # into the GEMM's slots)
        assert hip.pin(Segment.of(w), dt, k, m) == JAM.OK, hip.last_error()
        try:
            counts = [40, 3]
            for an, a in activation_sets(oracle, 43, k, 0xF9).items():
                say(f"fold edges {tag} grouped counts={counts} acts={an}")
                c = torch.full((43, 32), -3.0, dtype=torch.float32, device="cuda")
                a_d = dev(a)
                cnt = dev(np.array(counts, np.int32))
                torch.cuda.synchronize()
                assert hip.mm_grouped(Segment.of(w), dt, k, 32, 2, cnt.data_ptr(), a_d.data_ptr(), k, c.data_ptr(),
                                      32, k, 43, None) == JAM.OK, hip.last_error()
                hip.synchronize()
                got = c.cpu().numpy()
                for e, (o, nr) in enumerate(((0, 40), (40, 3))):
                    we = np.ascontiguousarray(w[32 * e:32 * e + 32])
                    ae = np.ascontiguousarray(a[o:o + nr])
                    ref = oracle.mm_int8(dt, we, ae, 32, nr, k)
                    _, sa = oracle.mm_ref(dt, we, ae, 32, nr, k)
                    check(got[o:o + nr], ref, sa, (tag, "grouped", e, an))
        finally:
            assert hip.evict(Segment.of(w)) == JAM.OK
        if dt == O.MXFP4:   # native MX: its own semantics (hardware block scales), non-finite where W is
            wd = oracle.dequant(O.MXFP4, w, k, f64=True)
            for mode in (1, 2):
                a = oracle.normal(0xFA + mode, (40, k))
                say(f"fold edges {tag} native MX mode={mode}")
                assert hip.set_mx_native(mode) == 0
                try:
                    got = mm_host(hip, dt, w, a, m, 40, k)
                finally:
                    assert hip.set_mx_native(0) == 0
                with np.errstate(all="ignore"):
                    ref, sref = X.mm(wd, a, mode)
                fin = np.isfinite(ref)
                assert np.array_equal(np.isfinite(got), fin), (tag, mode)
                assert (np.abs(got[fin] - ref[fin]) <= 2.0 ** -13 * sref[fin] + 1e-30).all(), (tag, mode)


def test_all_e0_mxfp4_groups(hip, oracle, monkeypatch):
    """MXFP4 groups whose every exponent is 0 (2^-128, an f32 subnormal scale) and exponents 0..3 mixed, with
    activations large enough that the outputs are normal f32 values: every path meets tier 1."""
    m, k = 32, 256
    rng = np.random.default_rng(0xE0)
    rows = [np.concatenate([mx_block(int(rng.integers(0, 4)) if r % 2 else 0, rand_nibs(rng)) for _ in range(8)])
            for r in range(m)]
    w = np.ascontiguousarray(np.stack(rows))
    for n, force in ((1, None), (12, "100000"), (40, "8")):
        say(f"all-e0 MXFP4 n={n}")
        if force:
            monkeypatch.setenv("JAM_HIP_MMA_MIN_N", force)
        a = (oracle.normal(0xE1 + n, (n, k)) * np.float32(2.0 ** 100)).astype(np.float32)
        got = mm_host(hip, O.MXFP4, w, a, m, n, k)
        ref = oracle.mm_int8(O.MXFP4, w, a, m, n, k)
        _, sa = oracle.mm_ref(O.MXFP4, w, a, m, n, k)
        assert (np.abs(ref) > 2.0 ** -126).mean() > 0.9
        check(got, ref, sa, ("all e0", n))


# ---------------------------------------------------------------------------- jam's Q8_0 suites
def q8_exact_int_weights(m, k, seed):
    """Scale 1.0 and int8 codes over the whole range, -128 included (QuantWeights.java:108-122)."""
    rng = np.random.default_rng(seed)
    nb = k // 32
    blk = np.zeros((m, nb, 34), np.uint8)
    blk[:, :, 0:2] = np.array([np.float16(1.0).view(np.uint16)], np.uint16).view(np.uint8)
    q = rng.integers(-128, 128, (m, nb, 32)).astype(np.int8)
    q[:, :, 0] = -128
    blk[:, :, 2:] = q.view(np.uint8)
    return np.ascontiguousarray(blk.reshape(m, nb * 34))


def test_q8_0_minus128_every_path(hip, oracle, monkeypatch):
    """Q8_0 weights holding -128 (legal in jam; its CPU kernels clamp the repacked byte, PRECISION.md:28-36):
    decode, F2 tiles, the matrix cores and the fallback GEMM all meet tier 1 against the oracle, and jam's own
    bound against the double reference."""
    from qxotic_amd.jam import JAM, Segment
    m, k = 96, 1024
    w = q8_exact_int_weights(m + 16, k, 0x128)
    for n, force in ((1, None), (3, None), (7, None), (8, "100000"), (13, "100000"), (16, "8"), (40, "8")):
        monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
        if force:
            monkeypatch.setenv("JAM_HIP_MMA_MIN_N", force)
        a = oracle.normal(0x129 + n, (n, k))
        say(f"Q8_0 -128 n={n} mma_min_n={force}")
        got = mm_host(hip, O.Q8_0, w, a, m + 16, n, k)
        ref = oracle.mm_int8(O.Q8_0, w, a, m + 16, n, k)
        fref, sa = oracle.mm_ref(O.Q8_0, w, a, m + 16, n, k)
        check(got, ref, sa, ("-128", n))
        assert (np.abs(got - fref) <= 1e-2 * sa + 1e-3).all()
    monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
    assert hip.pin(Segment.of(w), O.Q8_0, k, m + 16) == JAM.OK
    try:
        a = oracle.normal(0x12A, (100, k))
        say("Q8_0 -128 fallback GEMM (view at row 16) n=100")
        got = mm_host(hip, O.Q8_0, w, a, m, 100, k, w_off=16 * O.row_bytes(O.Q8_0, k))
        ws = np.ascontiguousarray(w[16:])
        ref = oracle.mm_int8(O.Q8_0, ws, a, m, 100, k)
        _, sa = oracle.mm_ref(O.Q8_0, ws, a, m, 100, k)
        check(got, ref, sa, ("-128", "fallback"))
    finally:
        assert hip.evict(Segment.of(w)) == JAM.OK


def f1_requant_ref(wq_rows, b, k):
    """jam_test.c:355-390's reference: the double dot of the weights' int8 codes and scales with B requantized
    by F1's formula (d = amax/127, id = 1/d, lrintf, clamp)."""
    m = wq_rows.shape[0]
    nb = k // 32
    blk = wq_rows.reshape(m, nb, 34)
    d = blk[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    bb = b.reshape(b.shape[0], nb, 32).astype(np.float32)
    amax = np.abs(bb).max(axis=2)
    dB = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(dB > 0, np.float32(1.0) / dB, np.float32(0.0)).astype(np.float32)
    qb = np.clip(np.rint((bb * idv[:, :, None]).astype(np.float32)), -128, 127).astype(np.float64)
    s = np.einsum("mbe,nbe->nmb", q, qb)
    return (s * (d.astype(np.float64)[None, :, :] * dB.astype(np.float64)[:, None, :])).sum(axis=2)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("m,n,k", [(37, 16, 256), (33, 1, 512), (64, 4, 128), (64, 40, 512)])
def test_q8_0_extreme_suite(hip, oracle, monkeypatch, mode, m, n, k):
    """jam_test.c:355-390 on every path: |W| = 8 everywhere (every code +-127), B at +-8 (mode 0: codes +-127)
    or one 1e4 and 31 values of 1e-3 per block (mode 1: the requant clamp's dynamic range). jam's bound
    (1e-2 + 1e-3*|ref|) against its requant reference, no NaN, and tier 1 against the oracle."""
    i = np.arange(m * k)
    W = np.where(((i ^ (i >> 3)) & 1) != 0, -8.0, 8.0).astype(np.float32).reshape(m, k)
    j = np.arange(n * k)
    if mode == 0:
        B = np.where(((j ^ (j >> 2)) & 1) != 0, -8.0, 8.0).astype(np.float32).reshape(n, k)
    else:
        B = np.where(j % 32 == 0, 1.0e4, 1.0e-3).astype(np.float32).reshape(n, k)
    wq = oracle.quantize(O.Q8_0, W)
    assert (np.abs(wq.reshape(m, k // 32, 34)[:, :, 2:].view(np.int8)) == 127).all()
    forces = ("8", "100000") if n >= 8 else (None,)
    for force in forces:
        monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
        if force:
            monkeypatch.setenv("JAM_HIP_MMA_MIN_N", force)
        say(f"Q8_0 extreme mode={mode} {m}x{n}x{k} mma_min_n={force}")
        got = mm_host(hip, O.Q8_0, wq, B, m, n, k)
        assert np.isfinite(got).all()
        R = f1_requant_ref(wq, B, k)
        assert (np.abs(got - R) <= 1e-2 + 1e-3 * np.abs(R)).all(), float(np.abs(got - R).max())
        ref = oracle.mm_int8(O.Q8_0, wq, B, m, n, k)
        _, sa = oracle.mm_ref(O.Q8_0, wq, B, m, n, k)
        check(got, ref, sa, ("extreme", mode, m, n, k, force))


@pytest.mark.parametrize("dt,k", [(O.Q8_0, 64), (O.Q4_0, 64), (O.MXFP4, 64), (O.NVFP4, 128), (O.Q4_K, 256),
                                  (O.Q5_K, 256), (O.Q6_K, 256), (O.Q1_0, 128), (O.F16, 80), (O.BF16, 80),
                                  (O.F32, 80)])
def test_adversarial_suite(hip, oracle, dt, k, monkeypatch):
    """jam_test.c:392-420 at its shape (37 rows, 8 tokens) and on the matrix cores (m = 64): token 0 all zero,
    token 1 all equal, token 2 a tiny scale, the rest exact .5 ties at dA = 1. Every output finite, token 0's
    column exactly zero."""
    for m, force in ((37, None), (64, "8")):
        monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
        if force:
            monkeypatch.setenv("JAM_HIP_MMA_MIN_N", force)
        n = 8
        B = np.zeros((n, k), np.float32)
        B[1] = 3.0
        B[2] = 1e-6
        e = np.arange(k)
        for jj in range(3, n):
            B[jj] = np.where(e % 32 == 0, 127.0, ((e + jj) % 32) - 16 + 0.5)
        w = oracle.quantize(dt, oracle.normal(0xAD + dt, (m, k), 0.0, 0.02))
        say(f"adversarial {O.NAMES[dt]} m={m} k={k} mma_min_n={force}")
        got = mm_host(hip, dt, w, B, m, n, k)
        assert np.isfinite(got).all()
        assert (got[0] == 0.0).all()


def q1_block(d_bits, rng):
    """One Q1_0 block (18 bytes): the fp16 d, then 128 random sign bits (jam_q1_0.h)."""
    return np.concatenate([np.array([d_bits & 0xFF, d_bits >> 8], np.uint8), rng.integers(0, 256, 16, np.uint8)])


def test_q1_0_scales_every_path(hip, oracle, monkeypatch):
    """Q1_0 (one fp16 d per 128 elements, each element +d or -d): d subnormal, at the smallest normal, at the
    fp16 maximum, zero and negative beside ordinary d in one row. The matrix cores apply 2^14·d in f32 once
    per block and -d as an f16 operand of the sums term, so every finite d takes them and stays at the error
    floor; a non-finite d (+-Inf, NaN) flags the tensor, which then gives the F2 decode kernel's bits and is
    non-finite where jam's result is. Decode (n = 1, 3), the F2 decode kernel (n = 12) and the matrix cores
    (n = 40), staged and pinned."""
    from qxotic_amd.jam import JAM, Segment
    m, k = 64, 512
    special = [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x0000, 0x8001, 0xFBFF, 0x8400]
    nonfinite = [0x7C00, 0xFC00, 0x7E00]
    for flagged in (False, True):
        rng = np.random.default_rng(0x0110 + flagged)
        rows = []
        for r in range(m):
            ds = [int(np.float16(rng.uniform(0.01, 0.03) * rng.choice([-1, 1])).view(np.uint16)) for _ in range(4)]
            if r < 2 * len(special):
                ds[r % 4] = special[r % len(special)]
            if flagged and r < len(nonfinite):
                ds[1] = nonfinite[r]
            rows.append(np.concatenate([q1_block(d, rng) for d in ds]))
        w = np.ascontiguousarray(np.stack(rows))
        tag = f"Q1_0 {'with non-finite d' if flagged else 'finite d'}"
        for n, force in ((1, None), (3, None), (12, "100000"), (40, "8")):
            for an, a in activation_sets(oracle, n, k, 0x1F0 + n).items():
                say(f"q1_0 scales {tag} n={n} mma_min_n={force} acts={an}")
                if force:
                    monkeypatch.setenv("JAM_HIP_MMA_MIN_N", force)
                else:
                    monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
                with np.errstate(all="ignore"):
                    ref = oracle.mm_int8(O.Q1_0, w, a, m, n, k)
                    _, sa = oracle.mm_ref(O.Q1_0, w, a, m, n, k)
                got = mm_host(hip, O.Q1_0, w, a, m, n, k)
                check(got, ref, sa, (tag, n, an), None if flagged or n != 40 else list(range(m)))
                if n == 40 and an == "A":
                    monkeypatch.setenv("JAM_HIP_NO_MMA", "1")
                    f2 = mm_host(hip, O.Q1_0, w, a, m, n, k)
                    monkeypatch.delenv("JAM_HIP_NO_MMA")
                    assert np.array_equal(bits(got), bits(f2)) == flagged, (tag, "routing")
        assert hip.pin(Segment.of(w), O.Q1_0, k, m) == JAM.OK, hip.last_error()
        try:
            monkeypatch.setenv("JAM_HIP_MMA_MIN_N", "8")
            a = oracle.normal(0x1F7, (40, k))
            say(f"q1_0 scales {tag} pinned n=40")
            got = mm_host(hip, O.Q1_0, w, a, m, 40, k)
            with np.errstate(all="ignore"):
                ref = oracle.mm_int8(O.Q1_0, w, a, m, 40, k)
                _, sa = oracle.mm_ref(O.Q1_0, w, a, m, 40, k)
            check(got, ref, sa, (tag, "pinned"), None if flagged else list(range(m)))
            monkeypatch.setenv("JAM_HIP_NO_MMA", "1")
            f2 = mm_host(hip, O.Q1_0, w, a, m, 40, k)
            monkeypatch.delenv("JAM_HIP_NO_MMA")
            assert np.array_equal(bits(got), bits(f2)) == flagged, (tag, "pinned routing")
        finally:
            monkeypatch.delenv("JAM_HIP_MMA_MIN_N", raising=False)
            assert hip.evict(Segment.of(w)) == JAM.OK
