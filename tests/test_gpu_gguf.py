"""GPU: the GGUF device weight registry (jamhip_gguf_pin / jamhip_gguf_evict) through the C-ABI.

A file holding five jam weight dtypes (2-D Q4_K, Q6_K and Q4_0 tensors, a stacked MXFP4 expert tensor
[k, rows, experts], a Q8_0 tensor with a partial row tile) and an F16 token embedding beside a 1-D F32 bias
(skipped) is opened and pinned in one call. Every jam call on a registry address
must (1) meet the tier-1 bound against the int8 oracle, (2) equal bit for bit the same call on an unpinned
heap copy of the same bytes (the staged path runs the same kernels), and (3) read the device copy: when
the caller's own mapping is pinned and then overwritten, results do not change. Expert slices of the
stacked tensor and the grouped call on it resolve inside the one pin (GptOss.java:673-684)."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

K = 512
E, ER = 4, 64            # experts, rows per expert


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def tier1(got, ref, sa):
    return np.abs(got - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa


def mm_at(hip, address, nbytes, owner, dt, a, m, n):
    from qxotic_amd.jam import JAM, Segment
    c = np.zeros((n, m), np.float32)
    st = hip.mm(Segment(address, nbytes, True, owner), 0, dt, K, Segment.of(a), 0, JAM.F32, K, Segment.of(c), 0,
                JAM.F32, m, m, n, K)
    assert st == JAM.OK, hip.last_error()
    return c


def mm_heap(hip, w, dt, a, m, n):
    w = np.ascontiguousarray(w).copy()
    return mm_at(hip, w.ctypes.data, w.nbytes, w, dt, a, m, n)


@pytest.fixture(scope="module")
def model(oracle, tmp_path_factory):
    from qxotic_amd import gguf as G
    w = {
        "blk.0.ffn_up.weight": (O.Q4_K, 96, oracle.quantize(O.Q4_K, oracle.normal(0x6601, (96, K), 0.0, 0.02))),
        "blk.0.ffn_gate_exps.weight": (O.MXFP4, E * ER,
                                       oracle.quantize(O.MXFP4, oracle.normal(0x6602, (E * ER, K), 0.0, 0.02))),
        "blk.0.attn_q.weight": (O.Q8_0, 40, oracle.quantize(O.Q8_0, oracle.normal(0x6603, (40, K), 0.0, 0.02))),
        "output.weight": (O.Q6_K, 72, oracle.quantize(O.Q6_K, oracle.normal(0x6604, (72, K), 0.0, 0.02))),
        "blk.0.attn_k.weight": (O.Q4_0, 48, oracle.quantize(O.Q4_0, oracle.normal(0x6605, (48, K), 0.0, 0.02))),
    }
    bias = np.arange(96, dtype=np.float32)
    tensors = [("blk.0.ffn_up.weight", O.Q4_K, (K, 96), w["blk.0.ffn_up.weight"][2]),
               ("blk.0.ffn_up.bias", 0, (96,), bias),
               ("blk.0.ffn_gate_exps.weight", O.MXFP4, (K, ER, E), w["blk.0.ffn_gate_exps.weight"][2]),
               ("blk.0.attn_q.weight", O.Q8_0, (K, 40), w["blk.0.attn_q.weight"][2]),
               ("token_embd.weight", 1, (K, 8), np.zeros(8 * K, np.float16)),
               ("output.weight", O.Q6_K, (K, 72), w["output.weight"][2]),
               ("blk.0.attn_k.weight", O.Q4_0, (K, 48), w["blk.0.attn_k.weight"][2])]
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    G.write(path, tensors, [("general.architecture", "string", "test")], alignment=64)
    return path, w


def test_registry_pin_lookup_evict(hip, oracle, model):
    from qxotic_amd import gguf as G
    path, w = model
    before = hip.pinned_bytes()
    with G.GGUF(path) as g:
        say("gguf registry: pin from the handle's mapping")
        st, cnt, nbytes = g.pin(hip)
        assert st == 0, hip.last_error()
        # every 2-D tensor of a jam weight type is pinned (the F16 token embedding included: tied-embedding
        # models multiply by it); the 1-D F32 bias is skipped
        emb = g.tensors["token_embd.weight"]
        assert cnt == 6 and nbytes == sum(x[2].nbytes for x in w.values()) + emb.byte_size
        assert hip.pinned_bytes() > before
        assert g.pin(hip)[:2] == (0, 6)                        # idempotent
        a = oracle.normal(0x55, (3, K))
        got = mm_at(hip, emb.address, emb.byte_size, g, O.F16, a, 8, 3)
        assert np.array_equal(got, np.zeros((3, 8), np.float32))   # the embedding rows are zeros
        try:
            for name, (dt, m, wq) in w.items():
                e = g.tensors[name]
                assert g.data(name).tobytes() == wq.tobytes()
                for n in (1, 4, 16):
                    a = oracle.outliers(0x77 + n + dt, (n, K))
                    say(f"  {name} {O.NAMES[dt]} m={m} n={n}")
                    got = mm_at(hip, e.address, e.byte_size, g, dt, a, m, n)
                    ref = oracle.mm_int8(dt, wq, a, m, n, K)
                    _, sa = oracle.mm_ref(dt, wq, a, m, n, K)
                    assert tier1(got, ref, sa).all(), (name, n)
                    assert np.array_equal(got.view(np.uint32), mm_heap(hip, wq, dt, a, m, n).view(np.uint32)), (name, n)
            # expert slices of the stacked tensor: row e·ER of the one pin
            e = g.tensors["blk.0.ffn_gate_exps.weight"]
            wq = w["blk.0.ffn_gate_exps.weight"][2]
            rb = wq.nbytes // (E * ER)
            for x in range(E):
                for n in (1, 16):
                    a = oracle.outliers(0x99 + x + n, (n, K))
                    got = mm_at(hip, e.address + x * ER * rb, ER * rb, g, O.MXFP4, a, ER, n)
                    sl = np.ascontiguousarray(wq[x * ER:(x + 1) * ER])
                    assert np.array_equal(got.view(np.uint32), mm_heap(hip, sl, O.MXFP4, a, ER, n).view(np.uint32)), (x, n)
        finally:
            assert g.evict(hip) == 6
    assert hip.pinned_bytes() == before


def test_registry_keys_caller_mapping(hip, oracle, model):
    """data_base = the caller's own copy of the data region: calls on the caller's addresses hit the pin,
    and overwriting the caller's bytes after the pin leaves results unchanged (the device copy is used)."""
    import torch
    from qxotic_amd import gguf as G
    from qxotic_amd.jam import JAM, Segment
    path, w = model
    with G.GGUF(path) as g:
        region = np.fromfile(path, dtype=np.uint8, offset=g.tensor_data_offset)
        base = region.ctypes.data
        say("gguf registry: pin the caller's mapping")
        st, cnt, _ = g.pin(hip, base)
        assert st == 0 and cnt == 6, hip.last_error()
        try:
            region[:] = 0
            for name, (dt, m, wq) in w.items():
                e = g.tensors[name]
                a = oracle.outliers(0x55 + dt, (8, K))
                got = mm_at(hip, base + e.offset, e.byte_size, region, dt, a, m, 8)
                assert np.array_equal(got.view(np.uint32), mm_heap(hip, wq, dt, a, m, 8).view(np.uint32)), name
            # grouped MoE call on the stacked expert tensor (m = rows per expert)
            e = g.tensors["blk.0.ffn_gate_exps.weight"]
            wq = w["blk.0.ffn_gate_exps.weight"][2]
            counts = [5, 0, 19, 40]
            rows = sum(counts)
            a = oracle.outliers(0x31, (rows, K))
            a_d = torch.from_numpy(a).cuda()
            c = torch.zeros((rows, ER), dtype=torch.float32, device="cuda")
            cnt_d = torch.tensor(counts, dtype=torch.int32, device="cuda")
            st = hip.mm_grouped(Segment(base + e.offset, e.byte_size, True, region), O.MXFP4, K, ER, E,
                                cnt_d.data_ptr(), a_d.data_ptr(), K, c.data_ptr(), ER, K, rows)
            assert st == JAM.OK, hip.last_error()
            hip.synchronize()
            got = c.cpu().numpy()
            o = 0
            for x, n in enumerate(counts):
                if n:
                    sl = np.ascontiguousarray(wq[x * ER:(x + 1) * ER])
                    ref = oracle.mm_int8(O.MXFP4, sl, np.ascontiguousarray(a[o:o + n]), ER, n, K)
                    _, sa = oracle.mm_ref(O.MXFP4, sl, np.ascontiguousarray(a[o:o + n]), ER, n, K)
                    assert tier1(got[o:o + n], ref, sa).all(), x
                o += n
        finally:
            assert g.evict(hip, base) == 6


def test_registry_rejects_partial_row_blocks(hip, tmp_path):
    """A jam-typed tensor whose row extent is not a whole number of blocks (allowed by GGUF when the total
    element count is) cannot be a jam weight: pin refuses the file with EUNSUPPORTED before pinning
    anything and names the tensor."""
    from qxotic_amd import gguf as G
    from qxotic_amd.jam import JAM
    ok = np.zeros(2 * 34, np.uint8)                            # Q8_0 [64, 1]
    bad = np.zeros(3 * 34, np.uint8)                           # Q8_0 [48, 2]: 96 elements, rows of 1.5 blocks
    path = tmp_path / "bad.gguf"
    G.write(path, [("a.weight", O.Q8_0, (64, 1), ok), ("b.weight", O.Q8_0, (48, 2), bad)])
    before = hip.pinned_bytes()
    with G.GGUF(path) as g:
        st, cnt, _ = g.pin(hip)
        assert st == JAM.EUNSUPPORTED and cnt == 0
        assert "b.weight" in hip.last_error()
    assert hip.pinned_bytes() == before
    # a row extent below one block ([16, 2] Q8_0, [128, 2] Q4_K: 32 and 256 elements in all) has a zero row
    # size; the check runs before any division by it (evict walks the same table)
    for dt, dims, nbytes in ((O.Q8_0, (16, 2), 34), (O.Q4_K, (128, 2), 144)):
        path = tmp_path / f"short_{dt}.gguf"
        G.write(path, [("a.weight", O.Q8_0, (64, 1), ok), ("c.weight", dt, dims, np.zeros(nbytes, np.uint8))])
        with G.GGUF(path) as g:
            st, cnt, _ = g.pin(hip)
            assert st == JAM.EUNSUPPORTED and cnt == 0, (dt, st)
            assert "c.weight" in hip.last_error()
            with pytest.raises(RuntimeError):
                g.evict(hip)
    assert hip.pinned_bytes() == before


def test_registry_runs_fused_call(hip, oracle, tmp_path):
    """q|k|v and gate|up stored back to back share one device range: each tensor alone, and one call over
    the run (W = the first tensor, m = the rows of all), meet the tier-1 bound, the run's rows equal the
    concatenation of the tensors' own results, and a tensor after a padding gap or of another dtype stays
    its own range."""
    from qxotic_amd import gguf as G
    from qxotic_amd.jam import JAM, Segment
    q = oracle.quantize(O.Q4_K, oracle.normal(0x7101, (64, K), 0.0, 0.02))
    kk = oracle.quantize(O.Q4_K, oracle.normal(0x7102, (32, K), 0.0, 0.02))
    v = oracle.quantize(O.Q4_K, oracle.normal(0x7103, (32, K), 0.0, 0.02))
    o = oracle.quantize(O.Q8_0, oracle.normal(0x7104, (64, K), 0.0, 0.02))
    tensors = [("blk.0.attn_q.weight", O.Q4_K, (K, 64), q), ("blk.0.attn_k.weight", O.Q4_K, (K, 32), kk),
               ("blk.0.attn_v.weight", O.Q4_K, (K, 32), v), ("blk.0.attn_output.weight", O.Q8_0, (K, 64), o)]
    path = tmp_path / "runs.gguf"
    G.write(path, tensors)
    qkv = np.concatenate([q, kk, v])
    before = hip.pinned_bytes()
    with G.GGUF(path) as g:
        e = {n: g.tensors[n] for n, *_ in tensors}
        assert e["blk.0.attn_k.weight"].offset == e["blk.0.attn_q.weight"].offset + q.nbytes   # back to back
        st, cnt, _ = g.pin(hip)
        assert st == 0 and cnt == 4, hip.last_error()
        try:
            for n in (1, 4, 16):
                a = oracle.outliers(0x7200 + n, (n, K))
                say(f"registry run q|k|v n={n}")
                fused = mm_at(hip, e["blk.0.attn_q.weight"].address, qkv.nbytes, g, O.Q4_K, a, 128, n)
                ref = oracle.mm_int8(O.Q4_K, qkv, a, 128, n, K)
                _, sa = oracle.mm_ref(O.Q4_K, qkv, a, 128, n, K)
                assert tier1(fused, ref, sa).all(), n
                parts = [mm_at(hip, e[nm].address, w.nbytes, g, O.Q4_K, a, w.shape[0], n)
                         for nm, w in (("blk.0.attn_q.weight", q), ("blk.0.attn_k.weight", kk), ("blk.0.attn_v.weight", v))]
                for got, w in zip(parts, (q, kk, v)):
                    r = oracle.mm_int8(O.Q4_K, w, a, w.shape[0], n, K)
                    _, sw = oracle.mm_ref(O.Q4_K, w, a, w.shape[0], n, K)
                    assert tier1(got, r, sw).all(), n
                # the output tensor (Q8_0) is a range of its own
                got = mm_at(hip, e["blk.0.attn_output.weight"].address, o.nbytes, g, O.Q8_0, a, 64, n)
                assert np.array_equal(got.view(np.uint32), mm_heap(hip, o, O.Q8_0, a, 64, n).view(np.uint32))
        finally:
            assert g.evict(hip) == 4
    assert hip.pinned_bytes() == before
