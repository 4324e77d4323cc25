"""GPU: jamhip_mm_device_noalloc (no allocation on its path; scratch from the GPU's static array) against
jamhip_mm_device on the same inputs: bit-identical results on every path that takes scratch (split-K decode,
F1 copy, F2 tiles, matrix-core prep and its split K), on two calls in a row, the second with a smaller
input; device memory in use unchanged across the calls; EUNSUPPORTED, with C untouched, for an unpinned W
and for a call whose scratch exceeds the static maximum."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

# (dtype, m, k, [n of the first call, n of the second, smaller call], lda pad)
CASES = [
    (O.Q4_K, 14336, 4096, [1, 1], 0),      # fused decode: no scratch
    (O.Q4_0, 4096, 14336, [7, 4], 0),      # split-K decode partials
    (O.Q8_0, 256, 4096, [5, 3], 1),        # rows not 16-byte aligned: F1 copy, then the decode kernel
    (O.Q4_K, 256, 1024, [24, 12], 0),      # F2 tiles on the decode kernel
    (O.Q4_K, 4096, 4096, [96, 40], 0),     # matrix cores: prep layout (and split K on the small grid)
    (O.Q6_K, 4096, 14336, [512, 64], 0),   # config 4's prefill shape: prep layout plus split K
    (O.MXFP4, 2880, 2880, [100, 17], 0),
]


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def test_noalloc_matches_mm_device(hip, oracle):
    import torch
    from qxotic_amd.jam import JAM, Segment
    ws, runs = [], []
    for dt, m, k, ns, pad in CASES:
        w = oracle.quantize(dt, oracle.normal(0x0A11 ^ m ^ dt, (m, k), 0.0, 0.02))
        assert hip.pin(Segment.of(w), dt, k, m) == JAM.OK, hip.last_error()
        ws.append(w)
        for n in ns:
            a = oracle.outliers(0x0A12 + n + dt, (n, k + pad))
            runs.append((dt, w, m, k, n, pad, torch.from_numpy(a).cuda()))
    try:
        # the allocating entry point first: its answers are the reference, and it loads every kernel's code
        # object, so that nothing the runtime loads lazily is counted against the allocation-free calls
        refs = []
        for (dt, w, m, k, n, pad, a) in runs:
            say(f"mm_device reference {O.NAMES[dt]} m={m} k={k} n={n}")
            ref = torch.full((n, m + 3), -7.0, dtype=torch.float32, device="cuda")
            assert hip.mm_device(Segment.of(w), dt, k, a.data_ptr(), k + pad, ref.data_ptr(), m + 3, m, n, k) == JAM.OK
            refs.append(ref)
        outs = [torch.full((n, m + 3), -7.0, dtype=torch.float32, device="cuda") for (_, _, m, _, n, _, _) in runs]
        hip.synchronize()
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        for (dt, w, m, k, n, pad, a), c in zip(runs, outs):
            say(f"noalloc {O.NAMES[dt]} m={m} k={k} n={n} lda={k + pad}")
            st = hip.mm_device_noalloc(Segment.of(w), dt, k, a.data_ptr(), k + pad, c.data_ptr(), m + 3, m, n, k)
            assert st == JAM.OK, hip.last_error()
        hip.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0, f"device memory in use changed by {free0 - free1} bytes"
        for (dt, w, m, k, n, pad, a), c, ref in zip(runs, outs, refs):
            assert torch.equal(c, ref), (O.NAMES[dt], m, k, n)
            assert bool((c[:, m:] == -7.0).all())
        # one case also against the oracle (the entry point's answer, not only its agreement)
        dt, w, m, k, n, pad, a = runs[7]
        an = a.cpu().numpy()[:, :k].copy()
        ref = oracle.mm_int8(dt, w, an, m, n, k)
        _, sa = oracle.mm_ref(dt, w, an, m, n, k)
        got = outs[7].cpu().numpy()[:, :m]
        assert (np.abs(got - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa).all()
    finally:
        for w, (dt, m, k, _, _) in zip(ws, CASES):
            hip.evict(Segment.of(w))


def test_noalloc_refusals(hip, oracle):
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, k = 512, 14336
    w = oracle.quantize(O.Q6_K, oracle.normal(0x0A13, (m, k), 0.0, 0.02))
    a = torch.from_numpy(oracle.normal(0x0A14, (2048, k))).cuda()
    c = torch.full((2048, m), 5.0, dtype=torch.float32, device="cuda")
    say("noalloc: unpinned W")
    assert hip.mm_device_noalloc(Segment.of(w), O.Q6_K, k, a.data_ptr(), k, c.data_ptr(), m, m, 8, k) == JAM.EUNSUPPORTED
    assert "not resident" in hip.last_error()
    assert hip.pin(Segment.of(w), O.Q6_K, k, m) == JAM.OK
    try:
        say("noalloc: 2048 tokens x 14336 exceed the static scratch")
        st = hip.mm_device_noalloc(Segment.of(w), O.Q6_K, k, a.data_ptr(), k, c.data_ptr(), m, m, 2048, k)
        assert st == JAM.EUNSUPPORTED and "static scratch maximum" in hip.last_error(), (st, hip.last_error())
        hip.synchronize()
        assert bool((c == 5.0).all())     # nothing was queued
        # the same call through the allocating entry point runs
        assert hip.mm_device(Segment.of(w), O.Q6_K, k, a.data_ptr(), k, c.data_ptr(), m, m, 2048, k) == JAM.OK
        hip.synchronize()
        assert bool(torch.isfinite(c).all())
    finally:
        hip.evict(Segment.of(w))
