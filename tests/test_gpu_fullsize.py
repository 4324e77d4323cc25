"""GPU parity at BASELINE.json's full sizes, and the paths only a forced condition reaches.

* config 2: Q4_0 14336x4096 and 4096x14336 at M in {1, 4, 8}, every output against the int8 oracle;
* config 3: the 128256x4096 Q6_K output head at n = 1 (431 MB, 4008 row bands) and the registry's fused
  q|k|v (6144x4096) and gate|up (28672x4096) runs of one Llama-3-8B block, on sampled rows;
* config 5: one gpt-oss-20B MoE layer at its real shape (32 experts, 5760x2880 gate_up and 2880x2880 down in
  MXFP4, 512 tokens routed top-4 by Zipf(1.1) popularity) through route -> gather -> grouped gate_up ->
  grouped down -> combine, against oracle/moe.py on a seeded sample of 96 output rows per grouped call;
* the fallback GEMM (gemm_kernel), which the matrix-core path leaves to views not aligned to 32 rows and to
  JAM_HIP_NO_MMA=1, on all five dtypes.

Bound: tier 1, |gpu - oracle| <= 1e-3*|oracle| + 1e-5*sum|w*a| (same int8 semantics, f32 order differs). Each
case prints its largest relative error (parity_report).
"""
import json
import os
import sys

import numpy as np
import pytest

from conftest import parity_report, random_blocks
from oracle import moe as M
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def tier1(got, ref, sa):
    return np.abs(got - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa


def run_mm(hip, dt, w, a, m, n, k, w_off=0, ldw=None):
    from qxotic_amd.jam import JAM, Segment
    c = np.zeros((n, m), np.float32)
    st = hip.mm(Segment.of(w), w_off, dt, ldw or k, Segment.of(a), 0, JAM.F32, k, Segment.of(c), 0, JAM.F32, m, m,
                n, k)
    assert st == JAM.OK, hip.last_error()
    return c


# ------------------------------------------------------------------------------------------ config 2
@pytest.mark.parametrize("m,k", [(14336, 4096), (4096, 14336)])
def test_config2_q4_0_decode_full(hip, oracle, m, k):
    w = oracle.quantize(O.Q4_0, oracle.normal(0x5A11C0DE ^ 2 ^ m, (m, k), 0.0, 0.02))
    for n in (1, 4, 8):
        say(f"config 2 Q4_0 {m}x{k} M={n}")
        a = oracle.normal(0x5A11C0DE ^ 2 ^ n, (n, k))
        got = run_mm(hip, O.Q4_0, w, a, m, n, k)
        ref = oracle.mm_int8(O.Q4_0, w, a, m, n, k)
        _, sa = oracle.mm_ref(O.Q4_0, w, a, m, n, k)
        parity_report(f"config2 Q4_0 {m}x{k} M={n}", got, ref, sa)
        assert tier1(got, ref, sa).all()


# ------------------------------------------------------------------------------------------ config 3
def test_config3_output_head(hip, oracle):
    """The 128256x4096 Q6_K head at n = 1, pinned; 256 sampled rows against the oracle, every output finite,
    a rerun bit-identical."""
    from qxotic_amd.jam import JAM, Segment
    m, k = 128256, 4096
    w = random_blocks(O.Q6_K, m, k, 0x5A11C0DE ^ 3)
    a = oracle.normal(0x5A11C0DE ^ 33, (1, k))
    assert hip.pin(Segment.of(w), JAM.Q6_K, k, m) == JAM.OK, hip.last_error()
    try:
        say("config 3 head Q6_K 128256x4096 n=1")
        got = run_mm(hip, O.Q6_K, w, a, m, 1, k)
        again = run_mm(hip, O.Q6_K, w, a, m, 1, k)
    finally:
        hip.evict(Segment.of(w))
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    rows = np.sort(np.random.default_rng(3).choice(m, 256, replace=False))
    rows[-1] = m - 1
    ws = np.ascontiguousarray(w[rows])
    ref = oracle.mm_int8(O.Q6_K, ws, a, len(rows), 1, k)
    _, sa = oracle.mm_ref(O.Q6_K, ws, a, len(rows), 1, k)
    parity_report("config3 head Q6_K 128256x4096 n=1", got[:, rows], ref, sa)
    assert tier1(got[:, rows], ref, sa).all()


def test_config3_fused_registry_runs(hip, oracle, tmp_path):
    """One Llama-3-8B block's q|k|v (4096 + 1024 + 1024 rows) and gate|up (2 x 14336 rows) Q4_K tensors back to
    back in a GGUF file: pinned as two runs, each run called once at n = 1 (m = 6144, m = 28672) from the
    first tensor's address; 192 sampled rows of each run against the oracle, and the run's rows equal the
    member tensors' own calls bit for bit."""
    from qxotic_amd import gguf as G
    from qxotic_amd.jam import JAM, Segment
    k = 4096
    shapes = [("attn_q", 4096), ("attn_k", 1024), ("attn_v", 1024), ("ffn_gate", 14336), ("ffn_up", 14336)]
    ws = {name: random_blocks(O.Q4_K, rows, k, 0x5A11C0DE ^ rows ^ len(name)) for name, rows in shapes}
    path = tmp_path / "llama_block.gguf"
    G.write(path, [(f"blk.0.{n}.weight", O.Q4_K, (k, r), ws[n]) for n, r in shapes])
    a = oracle.normal(0x5A11C0DE ^ 34, (1, k))
    with G.GGUF(path) as g:
        st, cnt, _ = g.pin(hip)
        assert st == JAM.OK and cnt == 5, hip.last_error()
        try:
            for first, members in (("attn_q", ["attn_q", "attn_k", "attn_v"]), ("ffn_gate", ["ffn_gate", "ffn_up"])):
                e0 = g.tensors[f"blk.0.{first}.weight"]
                m = sum(r for n, r in shapes if n in members)
                say(f"config 3 fused run {'|'.join(members)} m={m}")
                c = np.zeros((1, m), np.float32)
                st = hip.mm(Segment(e0.address, m * O.row_bytes(O.Q4_K, k), True, g), 0, JAM.Q4_K, k, Segment.of(a), 0,
                            JAM.F32, k, Segment.of(c), 0, JAM.F32, m, m, 1, k)
                assert st == JAM.OK, hip.last_error()
                wrun = np.concatenate([ws[n] for n in members])
                rows = np.sort(np.random.default_rng(m).choice(m, 192, replace=False))
                wsmp = np.ascontiguousarray(wrun[rows])
                ref = oracle.mm_int8(O.Q4_K, wsmp, a, len(rows), 1, k)
                _, sa = oracle.mm_ref(O.Q4_K, wsmp, a, len(rows), 1, k)
                parity_report(f"config3 fused {'|'.join(members)} 1x{m}x{k}", c[:, rows], ref, sa)
                assert tier1(c[:, rows], ref, sa).all()
                o = 0
                for n in members:
                    e = g.tensors[f"blk.0.{n}.weight"]
                    r = dict(shapes)[n]
                    cm = np.zeros((1, r), np.float32)
                    assert hip.mm(Segment(e.address, e.byte_size, True, g), 0, JAM.Q4_K, k, Segment.of(a), 0, JAM.F32,
                                  k, Segment.of(cm), 0, JAM.F32, r, r, 1, k) == JAM.OK
                    assert np.array_equal(cm.view(np.uint32), c[:, o:o + r].view(np.uint32)), n
                    o += r
        finally:
            g.evict(hip)


# ------------------------------------------------------------------------------------------ config 5
def test_config5_gptoss_moe_layer(hip, oracle):
    """gpt-oss-20B's MoE layer at its real shape: 32 distinct MXFP4 experts (5760x2880 gate_up, 2880x2880
    down, random valid blocks), 512 tokens of N(0,1), top-4 by Zipf(1.1) popularity (Gumbel-top-k on
    log p_e, p_e ~ e^-1.1, the bench's generator). Route, gather and combine bit-exact; each grouped call
    against per-expert jam matmuls on 96 sampled output rows, all routed rows."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    E, TOPK, SEQ, D, FF = 32, 4, 512, 2880, 5760
    wg = random_blocks(O.MXFP4, E * FF, D, 0xC0F5)
    wd = random_blocks(O.MXFP4, E * D, D, 0xD0F5)
    rng = np.random.default_rng(0x5A11C0DE ^ 5)
    logp = -1.1 * np.log(np.arange(1, E + 1))
    sel = np.argsort(-(logp[None, :] + rng.gumbel(size=(SEQ, E))), axis=1)[:, :TOPK].astype(np.int32)
    re_h = sel.ravel()
    R = SEQ * TOPK
    prob_h = rng.random(R).astype(np.float32)
    x_h = rng.standard_normal((SEQ, D)).astype(np.float32)
    hid_h = rng.standard_normal((R, D)).astype(np.float32)
    dev = lambda v: torch.from_numpy(np.ascontiguousarray(v)).cuda()
    i32 = lambda nel: torch.zeros(nel, dtype=torch.int32, device="cuda")
    counts, off, slot_route, route_slot = i32(E), i32(E + 1), i32(R), i32(R)
    re_d, prob, x, hid = dev(re_h), dev(prob_h), dev(x_h), dev(hid_h)
    g = torch.empty((R, D), device="cuda")
    h = torch.empty((R, FF), device="cuda")
    y = torch.empty((R, D), device="cuda")
    out = torch.empty((SEQ, D), device="cuda")
    assert hip.pin(Segment.of(wg), JAM.MXFP4, D, E * FF) == JAM.OK, hip.last_error()
    assert hip.pin(Segment.of(wd), JAM.MXFP4, D, E * D) == JAM.OK, hip.last_error()
    try:
        say("config 5 gpt-oss MoE layer: route, gather, grouped gate_up, grouped down, combine")
        assert hip.moe_route(re_d.data_ptr(), SEQ, TOPK, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                             route_slot.data_ptr()) == JAM.OK
        assert hip.moe_gather(x.data_ptr(), D, slot_route.data_ptr(), off.data_ptr(), E, SEQ, TOPK, D, g.data_ptr(),
                              D) == JAM.OK
        assert hip.mm_grouped(Segment.of(wg), JAM.MXFP4, D, FF, E, counts.data_ptr(), g.data_ptr(), D, h.data_ptr(),
                              FF, D, R, None) == JAM.OK, hip.last_error()
        assert hip.mm_grouped(Segment.of(wd), JAM.MXFP4, D, D, E, counts.data_ptr(), hid.data_ptr(), D, y.data_ptr(),
                              D, D, R, None) == JAM.OK, hip.last_error()
        assert hip.moe_combine(y.data_ptr(), D, re_d.data_ptr(), prob.data_ptr(), route_slot.data_ptr(), SEQ, TOPK, E,
                               D, out.data_ptr(), D) == JAM.OK
        assert hip.synchronize() == JAM.OK
    finally:
        hip.evict(Segment.of(wg))
        hip.evict(Segment.of(wd))
    c_o, off_o, sr_o, rs_o = M.dispatch_csr(re_h, E)
    assert np.array_equal(counts.cpu().numpy(), c_o)
    assert np.array_equal(off.cpu().numpy(), off_o)
    assert np.array_equal(route_slot.cpu().numpy(), rs_o)
    assert (c_o < 64).sum() >= 8 and c_o.max() >= 128, c_o     # ragged: small and large experts
    g_h = M.gather(x_h, sr_o, R, TOPK)
    assert np.array_equal(g.cpu().numpy(), g_h)
    y_h = y.cpu().numpy()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), M.combine(y_h, re_h, prob_h, rs_o, SEQ, TOPK, E).view(np.uint32))
    srng = np.random.default_rng(55)
    for name, w, m, a_h, got_all in (("gate_up", wg, FF, g_h, h.cpu().numpy()), ("down", wd, D, hid_h, y_h)):
        rows = np.sort(srng.choice(m, 96, replace=False))
        worst = {"max_rel": 0.0, "max_err_per_sumabs": 0.0}
        for e in range(E):
            n = int(c_o[e])
            if n == 0:
                continue
            ws = np.ascontiguousarray(w[e * m + rows])
            ae = np.ascontiguousarray(a_h[off_o[e]:off_o[e] + n])
            ref = oracle.mm_int8(O.MXFP4, ws, ae, len(rows), n, D)
            _, sa = oracle.mm_ref(O.MXFP4, ws, ae, len(rows), n, D)
            got = got_all[off_o[e]:off_o[e] + n][:, rows]
            ok = tier1(got, ref, sa)
            assert ok.all(), (name, e, n, int((~ok).sum()))
            err = np.abs(got.astype(np.float64) - ref)
            big = np.abs(ref) > 1e-3 * np.abs(ref).max()
            if big.any():
                worst["max_rel"] = max(worst["max_rel"], float((err[big] / np.abs(ref[big])).max()))
            worst["max_err_per_sumabs"] = max(worst["max_err_per_sumabs"], float((err / sa).max()))
        say(f"parity config5 {name} (32 experts, 96 sampled rows each): max_rel {worst['max_rel']:.3e}  "
            f"max_err/sumAbs {worst['max_err_per_sumabs']:.3e}")
        log = os.environ.get("JAM_PARITY_LOG")
        if log:
            with open(log, "a") as f:
                f.write(json.dumps({"case": f"config5 MoE grouped {name} MXFP4 (32 experts, 96 sampled rows each)",
                                    "outputs": int(R * 96), **worst}) + "\n")


# ---------------------------------------------------------------------------------- fallback GEMM
@pytest.mark.parametrize("dt", O.QUANT_TYPES)
def test_fallback_gemm_kernel(hip, oracle, dt, monkeypatch):
    """gemm_kernel runs where the matrix-core path declines, for n from its crossover (64 tokens for Q8_0,
    96 otherwise): (1) JAM_HIP_NO_MMA=1 on a staged weight; (2) a pinned tensor's slice starting at row 16 (not
    a 32-row tile boundary of the device copy). Both against the oracle; (2) also bit-identical to (1) on the
    same rows, since both run the same kernel on the same operands."""
    from qxotic_amd.jam import JAM, Segment
    be = O.BLOCK[dt][0]
    m, k = 128, (1024 if be == 256 else 992)
    w = oracle.quantize(dt, oracle.normal(0xFA11 ^ dt, (16 + m, k), 0.0, 0.02))
    rb = O.row_bytes(dt, k)
    for n in ((64, 100) if dt == O.Q8_0 else (96, 130)):
        a = oracle.outliers(0xFA12 + n, (n, k))
        ws = np.ascontiguousarray(w[16:])
        ref = oracle.mm_int8(dt, ws, a, m, n, k)
        _, sa = oracle.mm_ref(dt, ws, a, m, n, k)
        monkeypatch.setenv("JAM_HIP_NO_MMA", "1")
        say(f"fallback gemm {O.NAMES[dt]} JAM_HIP_NO_MMA=1 m={m} n={n} k={k}")
        forced = run_mm(hip, dt, ws, a, m, n, k)
        monkeypatch.delenv("JAM_HIP_NO_MMA")
        parity_report(f"fallback gemm {O.NAMES[dt]} n={n} (no-mma)", forced, ref, sa)
        assert tier1(forced, ref, sa).all()
        assert hip.pin(Segment.of(w), dt, k, 16 + m) == JAM.OK, hip.last_error()
        try:
            say(f"fallback gemm {O.NAMES[dt]} slice at row 16 m={m} n={n} k={k}")
            sliced = run_mm(hip, dt, w, a, m, n, k, w_off=16 * rb)
        finally:
            assert hip.evict(Segment.of(w)) == JAM.OK
        assert tier1(sliced, ref, sa).all()
        assert np.array_equal(sliced.view(np.uint32), forced.view(np.uint32))
