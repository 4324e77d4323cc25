"""GPU: fused epilogues through the C-ABI.

jamhip_mm_device_ex applies C = [C +] (W·A^T [+ bias]) in the matmul's own final store. Every kernel path
(decode F1 / F2, K-split decode and its reduce, matrix-core GEMM with and without split K, the fallback
GEMM, the float-dot tail rows) must give, bit for bit, what the separate passes give in f32 on the plain
jamhip_mm_device result (oracle/epilogue.py: Ops.addRowBiasInPlace then Ops.addInPlace), and leave the ldc
gap untouched. jamhip_glu_device must match the full-scalar SwiGLU / gpt-oss clamped SwiGLU within 1 ulp
(the device exp in double against numpy's)."""
import sys

import numpy as np
import pytest

from oracle import epilogue as EP
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


CASES = [   # (m, k, n): decode F1, split-K decode, F2 decode, matrix cores (+ split K), tail rows, and matrix
    # cores whose last round runs as half tiles (1024 x 4150: 65 tiles per XCD)
    (104, 1024, 1), (100, 9216, 4), (104, 1024, 8), (100, 1024, 16), (100, 1024, 100), (4096, 4096, 64),
    (1024, 256, 4150),
]


@pytest.mark.parametrize("dt", O.QUANT_TYPES)
@pytest.mark.parametrize("m,k,n", CASES)
def test_mm_epilogue_bit_exact(hip, oracle, dt, m, k, n):
    import torch
    from qxotic_amd.jam import JAM, Segment
    say(f"epilogue {O.NAMES[dt]} m={m} k={k} n={n}")
    w = oracle.quantize(dt, oracle.normal(0xE1 + dt + m, (m, k), 0.0, 0.02))
    a = oracle.outliers(0xE2 + n, (n, k))
    ldc = m + 3
    bias = np.random.default_rng(m + n).standard_normal(m).astype(np.float32)
    c0 = np.random.default_rng(k + n).standard_normal((n, ldc)).astype(np.float32)
    assert hip.pin(Segment.of(w), dt, k, m) == JAM.OK, hip.last_error()
    try:
        a_d = torch.from_numpy(a).cuda()
        b_d = torch.from_numpy(bias).cuda()
        plain = torch.zeros((n, ldc), dtype=torch.float32, device="cuda")
        assert hip.mm_device(Segment.of(w), dt, k, a_d.data_ptr(), k, plain.data_ptr(), ldc, m, n, k) == JAM.OK
        hip.synchronize()
        p = plain.cpu().numpy()[:, :m]
        for bias_on, acc in ((True, False), (False, True), (True, True)):
            c = torch.from_numpy(c0.copy()).cuda()
            st = hip.mm_device_ex(Segment.of(w), dt, k, a_d.data_ptr(), k, c.data_ptr(), ldc, m, n, k,
                                  b_d.data_ptr() if bias_on else None, acc)
            assert st == JAM.OK, hip.last_error()
            hip.synchronize()
            got = c.cpu().numpy()
            want = EP.add_row_bias(p, bias) if bias_on else p
            if acc:
                want = EP.add_in_place(c0[:, :m], want)
            assert np.array_equal(got[:, :m].view(np.uint32), want.view(np.uint32)), (bias_on, acc)
            assert np.array_equal(got[:, m:].view(np.uint32), c0[:, m:].view(np.uint32))   # gap untouched
    finally:
        hip.evict(Segment.of(w))


def test_mm_epilogue_rejects_bad_accumulate(hip, oracle):
    from qxotic_amd.jam import JAM, Segment
    w = oracle.quantize(O.Q8_0, oracle.normal(1, (32, 64), 0.0, 0.02))
    st = hip.mm_device_ex(Segment.of(w), O.Q8_0, 64, 1 << 20, 64, 1 << 20, 32, 32, 1, 64, None, 2)
    assert st == JAM.EINVAL


@pytest.mark.parametrize("act", [1, 2])
def test_glu(hip, act):
    import torch
    rows, cols, ldg, ldu = 7, 3001, 3005, 3003
    rng = np.random.default_rng(act)
    g = (rng.standard_normal((rows, ldg)) * 6).astype(np.float32)
    u = (rng.standard_normal((rows, ldu)) * 6).astype(np.float32)
    g[0, :8] = [7.0, 7.0001, -7.0, 40.0, -40.0, 0.0, -0.0, 1e-30]
    u[0, :8] = [7.0, -7.0001, -1.0, 100.0, -100.0, 3.0, 3.0, 1.0]
    say(f"glu act={act}")
    g_d = torch.from_numpy(g).cuda()
    u_d = torch.from_numpy(u).cuda()
    assert hip.glu_device(act, g_d.data_ptr(), ldg, u_d.data_ptr(), ldu, rows, cols) == 0, hip.last_error()
    hip.synchronize()
    got = g_d.cpu().numpy()
    f = EP.silu_mul if act == 1 else EP.clamped_swiglu
    want = f(g[:, :cols], u[:, :cols])
    d = np.abs(got[:, :cols].view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert d.max() <= 1, int(d.max())
    assert np.array_equal(got[:, cols:].view(np.uint32), g[:, cols:].view(np.uint32))   # gap untouched
    assert np.array_equal(u_d.cpu().numpy(), u)


GROUPED_COUNTS = [3, 0, 12, 70, 1, 9, 40]   # F1 experts (1..7 rows), F2 bands (8..15), matrix cores (>= 16)


@pytest.mark.parametrize("dt", O.QUANT_TYPES)
def test_grouped_expert_bias_bit_exact(hip, oracle, dt):
    """jamhip_mm_grouped_ex: expert e's rows get bias[e·m + i] in the store, bit for bit the f32 add of
    Ops.addRowBiasInPlace on the plain grouped result; rows past the routed total stay untouched."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    E, m, k = len(GROUPED_COUNTS), 64, 512
    say(f"grouped bias {O.NAMES[dt]} counts={GROUPED_COUNTS}")
    w = np.ascontiguousarray(np.concatenate(
        [oracle.quantize(dt, oracle.normal(0xB1 + 7 * e + dt, (m, k), 0.0, 0.02)) for e in range(E)]))
    total = sum(GROUPED_COUNTS)
    cap = total + 4
    a_d = torch.from_numpy(oracle.outliers(0xB2, (cap, k))).cuda()
    bias = np.random.default_rng(dt).standard_normal((E, m)).astype(np.float32)
    b_d = torch.from_numpy(bias).cuda()
    cnt = torch.tensor(GROUPED_COUNTS, dtype=torch.int32, device="cuda")
    assert hip.pin(Segment.of(w), dt, k, E * m) == JAM.OK, hip.last_error()
    try:
        outs = []
        for b in (None, b_d.data_ptr()):
            c = torch.full((cap, m + 1), -5.0, dtype=torch.float32, device="cuda")
            st = hip.mm_grouped_ex(Segment.of(w), dt, k, m, E, cnt.data_ptr(), a_d.data_ptr(), k, c.data_ptr(),
                                   m + 1, k, cap, None, b)
            assert st == JAM.OK, hip.last_error()
            hip.synchronize()
            outs.append(c.cpu().numpy())
        plain, fused = outs
        o = 0
        for e, n in enumerate(GROUPED_COUNTS):
            want = EP.add_row_bias(plain[o:o + n, :m], bias[e])
            assert np.array_equal(fused[o:o + n, :m].view(np.uint32), want.view(np.uint32)), (e, n)
            o += n
        assert (fused[total:] == -5.0).all() and (fused[:, m] == -5.0).all()
    finally:
        hip.evict(Segment.of(w))


@pytest.mark.parametrize("act", [1, 2])
@pytest.mark.parametrize("lanes", [8, 16])
def test_glu_vector(hip, act, lanes):
    """jamhip_glu_device_vector: jinfer's default Vector API arithmetic (njuffa's rational tanh in f32 with
    fused multiply-adds) against oracle/epilogue.py, bit for bit on the vector body; the elements past each
    row's loop bound take the scalar tail (SwiGLU: the double formula, within 1 ulp, the double exp differing
    by implementation; gpt-oss: clampedSwigluApprox, bit for bit). Clamp edges, +-0, NaN, the row gap."""
    import torch
    rows, cols, ldg, ldu = 5, 2885, 2889, 2887          # 2885 = 180*16 + 5 = 360*8 + 5
    rng = np.random.default_rng(act * 100 + lanes)
    g = (rng.standard_normal((rows, ldg)) * 6).astype(np.float32)
    u = (rng.standard_normal((rows, ldu)) * 6).astype(np.float32)
    g[0, :9] = [7.0, 7.0001, -7.0, 40.0, -40.0, 0.0, -0.0, 1e-30, np.nan]
    u[0, :9] = [7.0, -7.0001, -1.0, 100.0, -100.0, 3.0, 3.0, 1.0, 2.0]
    g[1, cols - 3:cols] = [11.5, -0.25, 6.0]            # the scalar tail
    say(f"glu vector act={act} lanes={lanes}")
    g_d = torch.from_numpy(g).cuda()
    u_d = torch.from_numpy(u).cuda()
    assert hip.glu_device_vector(act, g_d.data_ptr(), ldg, u_d.data_ptr(), ldu, rows, cols, lanes) == 0, \
        hip.last_error()
    hip.synchronize()
    got = g_d.cpu().numpy()[:, :cols]
    f = EP.silu_mul_vector if act == 1 else EP.clamped_swiglu_vector
    want = f(g[:, :cols], u[:, :cols], lanes)
    bound = cols - cols % lanes
    assert np.array_equal(np.isnan(got), np.isnan(want))
    got, want = np.where(np.isnan(got), 0, got), np.where(np.isnan(want), 0, want)   # NaN payloads may differ
    assert np.array_equal(got[:, :bound].view(np.uint32), want[:, :bound].view(np.uint32))
    d = np.abs(got[:, bound:].view(np.int32).astype(np.int64) - want[:, bound:].view(np.int32).astype(np.int64))
    assert d.max() <= (1 if act == 1 else 0), int(d.max())
    assert np.array_equal(g_d.cpu().numpy()[:, cols:].view(np.uint32), g[:, cols:].view(np.uint32))
    assert hip.glu_device_vector(act, g_d.data_ptr(), ldg, u_d.data_ptr(), ldu, rows, cols, -1) == 1   # EINVAL
