"""Benchmark of the MI355X jam backend on BASELINE.json's headline metric.

Step = one decode matmul of jam's hot path: Q4_K GEMV 14336x4096, M=1 (Llama-3-8B gate/up projection),
activation quantization (jam's F1) included, through the C-ABI device entry point; one kernel launch per
step. Weights are resident in HBM before timing: 32 distinct copies (1.06 GB, > the 256 MB Infinity Cache)
rotate so no step is served from cache. The K timed steps are one captured HIP graph of K launches on the
library's stream, timed with HIP events recorded on that stream, between a synchronize on each side.

The same JSON line carries
  * ``roofline``: the GEMV kernel's algorithmic bytes per launch over its event-timed average duration,
    against MI355X's 8 TB/s, plus the HBM bytes per launch that rocprofv3's FETCH_SIZE/WRITE_SIZE counters
    measured for this command (read from the committed summary under profiles/);
  * ``moe``: config 5, a gpt-oss-20B-shaped MoE layer (device routing, gather, two grouped MXFP4 matmuls,
    combine) in TOPS and weight GB/s with their fractions of the int8 / fp4 MFMA and HBM peaks;
  * ``prefill``: the metric's second half, M=512 prefill TOPS of Q4_K 14336x4096 and Q6_K 4096x14336
    (activations 99% N(0,1) + 1% outliers at +-20, F2-quantized in the timed calls) against MI355X's dense
    int8 and f16 MFMA peaks;
  * ``decode_step``: config 3, a whole Llama-3-8B decode step's 225 matmuls (32 layers + output head,
    4.8 GB of weights) as one graph, in µs per token and HBM fraction;
  * ``epilogue``: a fused bias + residual epilogue against the separate passes (gpt-oss attention output
    projection at decode);
  * ``registry``: model load through the GGUF device weight registry (open + pin of a synthetic
    gpt-oss-20B-shaped file) in GB/s of jam weights made resident;
  * ``cpu_baseline``: the reference's own libjam (oracle/_ref, built from the reference C sources) on the
    same decode workload on this machine's host cores.

    python bench.py [--gpus 1] [--steps 2048] [--warmup 64] [--no-cpu] [--no-prefill] [--no-moe] [--no-step] [--no-epilogue] [--no-registry]
    profiling runs: --no-graph (plain stream launches) --calibrate-copy (three 256 MiB device copies first,
    the known-size reference for the FETCH_SIZE/WRITE_SIZE scale factors)
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

M, K, N = 14336, 4096, 1
COPIES = 32
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16 MFMA
# Algorithmic bytes per step, each operand once (jam_bench.c:46-75): W + A (f32) + C (f32).
STEP_BYTES = M * (K // 256) * 144 + N * K * 4 + N * M * 4   # 33,103,872
METRIC = "GB/s (%HBM peak) Q4_K GEMV 14336x4096 M=1; TOPS (%MFMA) M=512 prefill"
TRAFFIC_SUMMARY = ROOT / "profiles" / "q4k_gemv_14336x4096_traffic.txt"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def quantized(name: str, m: int, k: int, seed: int) -> np.ndarray:
    from qxotic_amd import ggml
    x = np.random.default_rng(seed).normal(0.0, 0.02, (m, k)).astype(np.float32)
    return ggml.quantize(name, x)


def synthetic(name: str, m: int, k: int, seed: int) -> np.ndarray:
    """[m, row_bytes] weights for the types qxotic_amd.ggml does not quantize: Q5_K, NVFP4 and Q1_0 as random
    valid blocks (random quant bytes; block scales drawn so the decoded values are of the N(0, 0.02) order),
    F16 / BF16 as N(0, 0.02) draws rounded to the type. The kernels' work does not depend on the values."""
    rng = np.random.default_rng(seed)
    if name in ("F16", "BF16"):
        x = rng.normal(0.0, 0.02, (m, k)).astype(np.float32)
        if name == "F16":
            return np.ascontiguousarray(x.astype(np.float16).view(np.uint8))
        u = x.view(np.uint32)
        return np.ascontiguousarray(((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8))
    be, bb = {"Q5_K": (256, 176), "NVFP4": (64, 36), "Q1_0": (128, 18)}[name]
    nb = k // be
    blk = rng.integers(0, 256, (m, nb, bb), dtype=np.uint8)
    f16 = lambda lo, hi: rng.uniform(lo, hi, (m, nb)).astype(np.float16).view(np.uint8).reshape(m, nb, 2)
    if name == "Q5_K":
        blk[:, :, 0:2] = f16(2e-5, 8e-5)          # d
        blk[:, :, 2:4] = f16(1e-4, 5e-4)          # dmin
    elif name == "NVFP4":
        blk[:, :, 0:4] = rng.integers(0x20, 0x30, (m, nb, 4), dtype=np.uint8)   # UE4M3 sub-block scales
    else:
        blk[:, :, 0:2] = f16(0.01, 0.03)
    return np.ascontiguousarray(blk.reshape(m, nb * bb))


def calibrate_copy(torch) -> None:
    """Three device-to-device copies of 256 MiB: 256 MiB read + 256 MiB written per dispatch."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def gpu_leg(args, w: np.ndarray, hip, torch, stream) -> dict:
    from qxotic_amd.jam import JAM, Segment

    copies = [w.copy() for _ in range(COPIES)]
    for cp in copies:
        st = hip.pin(Segment.of(cp), JAM.Q4_K, K, M)
        assert st == JAM.OK, hip.last_error()
    a = torch.randn((N, K), dtype=torch.float32, device="cuda")
    c = torch.empty((COPIES, N, M), dtype=torch.float32, device="cuda")

    def step(i):
        st = hip.mm_device(Segment.of(copies[i % COPIES]), JAM.Q4_K, K, a.data_ptr(), K,
                           c[i % COPIES].data_ptr(), M, M, N, K)
        if st != JAM.OK:
            raise RuntimeError(hip.last_error())

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        graph = None
        if not args.no_graph:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(args.steps):
                    step(i)
            graph.replay()   # warm replay
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        if graph is not None:
            graph.replay()
        else:
            for i in range(args.steps):
                step(i)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1)
    # the last output of the timed region against a direct call
    ref = torch.empty((N, M), dtype=torch.float32, device="cuda")
    last = (args.steps - 1) % COPIES
    with torch.cuda.stream(stream):
        st = hip.mm_device(Segment.of(copies[last]), JAM.Q4_K, K, a.data_ptr(), K, ref.data_ptr(), M, M, N, K)
    torch.cuda.synchronize()
    assert st == JAM.OK and torch.equal(ref, c[last]), "timed output disagrees with a direct call"
    # the host-pointer entry point (jamhip_mm: A staged host -> device, C copied back, synchronized), the
    # PCIe-inclusive latency a caller passing host buffers sees; pinned weights, wall clock per call
    a_h = a.cpu().numpy()
    c_h = np.empty((N, M), np.float32)
    for i in range(8):
        hip.mm_contiguous(Segment.of(copies[i % COPIES]), Segment.of(a_h), Segment.of(c_h), JAM.Q4_K, M, N, K)
    calls = 256
    t0 = time.perf_counter()
    for i in range(calls):
        st = hip.mm_contiguous(Segment.of(copies[i % COPIES]), Segment.of(a_h), Segment.of(c_h), JAM.Q4_K, M, N, K)
        if st != JAM.OK:
            raise RuntimeError(hip.last_error())
    host_us = (time.perf_counter() - t0) / calls * 1e6
    # the same call on a weight nobody pinned: staged every call (autopin off), then with autopin (pinned on
    # its second sighting, the first staged) -- the residency an unedited jinfer gets
    fresh = w.copy()
    t0 = time.perf_counter()
    for i in range(8):
        hip.mm_contiguous(Segment.of(fresh), Segment.of(a_h), Segment.of(c_h), JAM.Q4_K, M, N, K)
    staged_us = (time.perf_counter() - t0) / 8 * 1e6
    assert hip.set_autopin(2) == JAM.OK
    for i in range(2):
        hip.mm_contiguous(Segment.of(fresh), Segment.of(a_h), Segment.of(c_h), JAM.Q4_K, M, N, K)
    t0 = time.perf_counter()
    for i in range(calls):
        hip.mm_contiguous(Segment.of(fresh), Segment.of(a_h), Segment.of(c_h), JAM.Q4_K, M, N, K)
    auto_us = (time.perf_counter() - t0) / calls * 1e6
    ap = hip.autopin_stats()
    assert ap["pins"] >= 1 and ap["hits"] >= calls, ap
    assert hip.set_autopin(0) == JAM.OK and hip.evict(Segment.of(fresh)) == JAM.OK
    with torch.cuda.stream(stream):
        st = hip.mm_device(Segment.of(copies[(calls - 1) % COPIES]), JAM.Q4_K, K, a.data_ptr(), K, ref.data_ptr(),
                           M, M, N, K)
    torch.cuda.synchronize()
    assert st == JAM.OK and np.array_equal(c_h, ref.cpu().numpy()), "host-pointer call disagrees"
    for cp in copies:
        hip.evict(Segment.of(cp))
    return {"event_ms": ev_ms, "wall_s": wall, "host_us": host_us, "staged_us": staged_us, "auto_us": auto_us}


def read_floor_leg(args, hip, torch, stream) -> dict:
    """The same harness as the decode leg (COPIES rotating buffers, one graph of args.steps launches) around
    jamhip_read_floor: a plain streaming read of the weight copy's bytes with the decode kernel's load shape,
    nothing computed or written. Its rate is the practical floor the decode GEMV is measured against."""
    nbytes = M * (K // 256) * 144
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(COPIES)]
    for b in bufs:
        b.random_(0, 255)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")

    def step(i):
        if hip.read_floor(bufs[i % COPIES].data_ptr(), nbytes, sink.data_ptr()) != 0:
            raise RuntimeError(hip.last_error())

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        graph = None
        if not args.no_graph:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(args.steps):
                    step(i)
            graph.replay()
            torch.cuda.synchronize()
        e0.record(stream)
        if graph is not None:
            graph.replay()
        else:
            for i in range(args.steps):
                step(i)
        e1.record(stream)
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    del bufs
    return {"us": round(us, 3), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes,
            "note": "streaming read of the Q4_K weight bytes, decode load shape, same graph harness; no compute, "
                    "no output"}


def shapes_leg(hip, torch, stream, steps: int = 512) -> dict:
    """The other BASELINE decode shapes, in the headline's harness: config 1 (Q8_0 4096x4096, M = 1), config 2
    (Q4_0 14336x4096 and 4096x14336, M in {1, 4, 8}) and config 3's down projection (Q6_K 4096x14336, M = 1).
    Each shape rotates over enough pinned copies to pass 1 GB (beyond the 256 MB Infinity Cache) inside one
    captured graph of `steps` launches on the library's stream, timed with HIP events; GB/s counts each
    operand once (jam_bench.c:46-75)."""
    from qxotic_amd.jam import JAM, Segment

    out = {}
    for label, name, dt, m, k, ns in (("config1", "Q8_0", JAM.Q8_0, 4096, 4096, (1,)),
                                      ("config2", "Q4_0", JAM.Q4_0, 14336, 4096, (1, 4, 8)),
                                      ("config2", "Q4_0", JAM.Q4_0, 4096, 14336, (1, 4, 8)),
                                      ("config3 down", "Q6_K", JAM.Q6_K, 4096, 14336, (1,)),
                                      ("dtype", "Q5_K", JAM.Q5_K, 14336, 4096, (1,)),
                                      ("dtype", "NVFP4", JAM.NVFP4, 14336, 4096, (1,)),
                                      ("dtype", "Q1_0", JAM.Q1_0, 14336, 4096, (1,)),
                                      ("dtype", "F16", JAM.F16, 14336, 4096, (1,)),
                                      ("dtype", "BF16", JAM.BF16, 14336, 4096, (1,))):
        w = (quantized(name, m, k, 0x5A11C0DE ^ dt ^ m) if name in ("Q8_0", "Q4_0", "Q6_K")
             else synthetic(name, m, k, 0x5A11C0DE ^ dt ^ m))
        ncp = max(32, -(-1_070_000_000 // w.nbytes))
        copies = [w.copy() for _ in range(ncp)]
        for cp in copies:
            assert hip.pin(Segment.of(cp), dt, k, m) == JAM.OK, hip.last_error()
        for n in ns:
            a = torch.randn((n, k), dtype=torch.float32, device="cuda")
            c = torch.empty((ncp, n, m), dtype=torch.float32, device="cuda")

            def step(i):
                if hip.mm_device(Segment.of(copies[i % ncp]), dt, k, a.data_ptr(), k, c[i % ncp].data_ptr(), m, m, n,
                                 k) != JAM.OK:
                    raise RuntimeError(hip.last_error())

            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                for i in range(ncp):
                    step(i)
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for i in range(steps):
                        step(i)
                graph.replay()
                torch.cuda.synchronize()
                e0.record(stream)
                graph.replay()
                e1.record(stream)
                torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / steps
            nbytes = w.nbytes + n * k * 4 + n * m * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            out[f"{label} {name} {m}x{k} M={n}"] = {"us": round(us, 3), "GBs": round(gbs, 1),
                                                    "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes,
                                                    "copies": ncp}
            del graph, a, c
        for cp in copies:
            hip.evict(Segment.of(cp))
        del copies
    out["note"] = ("graph-timed like the headline: one captured graph of %d launches over >= 1.07 GB of rotating "
                   "pinned copies; bytes = W + A + C once; 'dtype' rows: jam's other weight types (random valid "
                   "blocks / N(0,0.02) rounded)" % steps)
    return out


def prefill_leg(hip, torch, stream, reps: int = 10) -> dict:
    """M=512 prefill on the two BASELINE prefill shapes (config 4), then jam's other weight types at 14336x4096;
    each timed call quantizes its activations (F2; NVFP4: F1, jam's only path for it)."""
    from qxotic_amd.jam import JAM, Segment

    out = {}
    n = 512
    for name, dt, m, k in (("Q4_K", JAM.Q4_K, 14336, 4096), ("Q6_K", JAM.Q6_K, 4096, 14336),
                           ("Q5_K", JAM.Q5_K, 14336, 4096), ("Q4_0", JAM.Q4_0, 14336, 4096),
                           ("Q8_0", JAM.Q8_0, 14336, 4096), ("MXFP4", JAM.MXFP4, 14336, 4096),
                           ("NVFP4", JAM.NVFP4, 14336, 4096), ("Q1_0", JAM.Q1_0, 14336, 4096),
                           ("F16", JAM.F16, 14336, 4096)):
        w = (quantized(name, m, k, 0x5EED ^ dt) if name in ("Q4_K", "Q6_K", "Q4_0", "Q8_0", "MXFP4")
             else synthetic(name, m, k, 0x5EED ^ dt))
        assert hip.pin(Segment.of(w), dt, k, m) == JAM.OK, hip.last_error()
        rng = np.random.default_rng(11)
        x = rng.standard_normal((n, k)).astype(np.float32)
        hit = rng.random((n, k)) < 0.01
        x[hit] = np.where(rng.random(int(hit.sum())) < 0.5, -20.0, 20.0).astype(np.float32)
        a = torch.from_numpy(x).to("cuda")
        c = torch.empty((n, m), dtype=torch.float32, device="cuda")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            for _ in range(2):
                assert hip.mm_device(Segment.of(w), dt, k, a.data_ptr(), k, c.data_ptr(), m, m, n, k) == JAM.OK
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(reps):
                hip.mm_device(Segment.of(w), dt, k, a.data_ptr(), k, c.data_ptr(), m, m, n, k)
            e1.record(stream)
            torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
        assert bool(torch.isfinite(c).all()), "prefill output not finite"
        # the host-pointer entry point on the same call (jamhip_mm: 8 / 28 MiB of A up, C down, synchronized)
        host_us = None
        if name in ("Q4_K", "Q6_K"):
            c_h = np.empty((n, m), np.float32)
            hip.mm_contiguous(Segment.of(w), Segment.of(x), Segment.of(c_h), dt, m, n, k)
            t0 = time.perf_counter()
            for _ in range(5):
                assert hip.mm_contiguous(Segment.of(w), Segment.of(x), Segment.of(c_h), dt, m, n, k) == JAM.OK
            host_us = round((time.perf_counter() - t0) / 5 * 1e6, 1)
        out[f"{name} {m}x{k} M=512"] = {"us": round(us, 2), "TOPS": round(tops, 2),
                                        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                        "frac_f16_peak": round(tops / F16_PEAK_TFLOPS, 4),
                                        "host_pointer_us": host_us}
        hip.evict(Segment.of(w))
        del a, c
    out["note"] = ("jam's F2 quantization + int8 products computed exactly on f16 MFMA (integer operands "
                   "<= 2048); peaks are MI355X dense int8 5.0 POP/s and f16 2.5 PFLOP/s; host_pointer_us = the "
                   "same call through jamhip_mm with host A and C (PCIe both ways, synchronized), wall clock")
    return out


def moe_leg(hip, torch, stream, steps: int = 10, no_graph: bool = False) -> dict:
    """Config 5: a gpt-oss-20B-shaped MoE layer on the device: 32 experts with an MXFP4 gate_up 5760x2880
    and down 2880x2880, 512 tokens routed top-4 by Zipf(1.1) popularity (Gumbel-top-k on log p_e,
    p_e ~ e^-1.1). One step = jamhip_moe_select_topk + _route + _gather + grouped gate_up + grouped down + _combine
    (the down projection reads a synthetic 2880-wide hidden of the routed rows; the activation between
    the two matmuls is not part of jam's path). The layer starts from the router's logits on the device:
    jamhip_moe_select_topk (Moe.selectTopK + gpt-oss's softmax over the selected logits) gives the routes."""
    from qxotic_amd.jam import JAM, Segment

    E, TOPK, SEQ, D, FF = 32, 4, 512, 2880, 5760
    distinct = 2   # distinct expert matrices quantized from N(0,0.02); the 32 experts cycle through them
    gu = [quantized("MXFP4", FF, D, 0xC0F5 + s) for s in range(distinct)]
    dn = [quantized("MXFP4", D, D, 0xD0F5 + s) for s in range(distinct)]
    copies = 2    # 2 x 423 MB of weights, over the 256 MB Infinity Cache
    wg = [np.ascontiguousarray(np.concatenate([gu[e % distinct] for e in range(E)])) for _ in range(copies)]
    wd = [np.ascontiguousarray(np.concatenate([dn[e % distinct] for e in range(E)])) for _ in range(copies)]
    for x in wg:
        assert hip.pin(Segment.of(x), JAM.MXFP4, D, E * FF) == JAM.OK, hip.last_error()
    for x in wd:
        assert hip.pin(Segment.of(x), JAM.MXFP4, D, E * D) == JAM.OK, hip.last_error()
    rng = np.random.default_rng(0x5A11C0DE ^ 5)
    logp = -1.1 * np.log(np.arange(1, E + 1))
    logits_h = (logp[None, :] + rng.gumbel(size=(SEQ, E))).astype(np.float32)   # router logits: Zipf(1.1) top-4
    sel = np.argsort(-logits_h, axis=1, kind="stable")[:, :TOPK].astype(np.int32)
    counts_h = np.bincount(sel.ravel(), minlength=E)
    R = SEQ * TOPK
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to("cuda")
    logits0 = dev(logits_h)
    logits = torch.empty_like(logits0)
    re = dev(sel.ravel())
    prob = dev(rng.random(R).astype(np.float32))
    x = dev(rng.standard_normal((SEQ, D)).astype(np.float32))
    hid = dev(rng.standard_normal((R, D)).astype(np.float32))
    i32 = lambda nel: torch.zeros(nel, dtype=torch.int32, device="cuda")
    counts, off, slot_route, route_slot = i32(E), i32(E + 1), i32(R), i32(R)
    g = torch.empty((R, D), device="cuda")
    h = torch.empty((R, FF), device="cuda")
    y = torch.empty((R, D), device="cuda")
    out = torch.empty((SEQ, D), device="cuda")

    def layer(i):
        cg, cd = wg[i % copies], wd[i % copies]
        logits.copy_(logits0)   # the router's output (selectTopK consumes it)
        ok = hip.moe_select_topk(logits.data_ptr(), None, SEQ, E, E, TOPK, hip.TOPK_SOFTMAX, re.data_ptr(),
                                 prob.data_ptr()) == JAM.OK
        ok &= hip.moe_route(re.data_ptr(), SEQ, TOPK, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                            route_slot.data_ptr()) == JAM.OK
        ok &= hip.moe_gather(x.data_ptr(), D, slot_route.data_ptr(), off.data_ptr(), E, SEQ, TOPK, D, g.data_ptr(),
                             D) == JAM.OK
        ok &= hip.mm_grouped(Segment.of(cg), JAM.MXFP4, D, FF, E, counts.data_ptr(), g.data_ptr(), D, h.data_ptr(),
                             FF, D, R, None) == JAM.OK
        ok &= hip.mm_grouped(Segment.of(cd), JAM.MXFP4, D, D, E, counts.data_ptr(), hid.data_ptr(), D, y.data_ptr(),
                             D, D, R, None) == JAM.OK
        ok &= hip.moe_combine(y.data_ptr(), D, re.data_ptr(), prob.data_ptr(), route_slot.data_ptr(), SEQ, TOPK, E, D,
                              out.data_ptr(), D) == JAM.OK
        if not ok:
            raise RuntimeError(hip.last_error())

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn=layer, n=steps, warm=3) -> tuple:
        """(graph, stream) µs per layer: the median of 3 replays of one captured graph of `n` layers (the layer's
        launches are all device-side: routing, offsets and slot maps come from device counts), and the median
        of 3 runs of `n` layers launched on the stream (one run varies by 2-3% between runs on one box). The
        stream runs come first and allocate every scratch buffer the capture then reuses."""
        runs, gruns = [], []
        with torch.cuda.stream(stream):
            for i in range(warm):
                fn(i)
            torch.cuda.synchronize()
            for _ in range(3):
                e0.record(stream)
                for i in range(n):
                    fn(i)
                e1.record(stream)
                torch.cuda.synchronize()
                runs.append(e0.elapsed_time(e1) * 1e3 / n)
        if no_graph:
            return sorted(runs)[1], sorted(runs)[1]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                fn(i)
        with torch.cuda.stream(stream):
            g.replay()   # warm replay
            torch.cuda.synchronize()
            for _ in range(3):
                e0.record(stream)
                g.replay()
                e1.record(stream)
                torch.cuda.synchronize()
                gruns.append(e0.elapsed_time(e1) * 1e3 / n)
        del g
        return sorted(gruns)[1], sorted(runs)[1]

    def layer_gf(i):
        # the same layer with the gather folded into the gate_up call (jamhip_mm_grouped_gather): its activation
        # prep reads each routed row from x through slot_route; bit-identical results (tests/test_gpu_moe.py)
        cg, cd = wg[i % copies], wd[i % copies]
        logits.copy_(logits0)
        ok = hip.moe_select_topk(logits.data_ptr(), None, SEQ, E, E, TOPK, hip.TOPK_SOFTMAX, re.data_ptr(),
                                 prob.data_ptr()) == JAM.OK
        ok &= hip.moe_route(re.data_ptr(), SEQ, TOPK, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                            route_slot.data_ptr()) == JAM.OK
        ok &= hip.mm_grouped_gather(Segment.of(cg), JAM.MXFP4, D, FF, E, counts.data_ptr(), x.data_ptr(), D,
                                    slot_route.data_ptr(), TOPK, h.data_ptr(), FF, D, R, None) == JAM.OK
        ok &= hip.mm_grouped(Segment.of(cd), JAM.MXFP4, D, D, E, counts.data_ptr(), hid.data_ptr(), D, y.data_ptr(),
                             D, D, R, None) == JAM.OK
        ok &= hip.moe_combine(y.data_ptr(), D, re.data_ptr(), prob.data_ptr(), route_slot.data_ptr(), SEQ, TOPK, E, D,
                              out.data_ptr(), D) == JAM.OK
        if not ok:
            raise RuntimeError(hip.last_error())

    us, us_stream = timed()
    assert np.array_equal(counts.cpu().numpy(), counts_h), "device routing counts disagree with the host's"
    assert np.array_equal(re.cpu().numpy(), sel.ravel()), "device top-k disagrees with the host's"
    assert bool(torch.isfinite(out).all()), "moe output not finite"
    out_ref = out.clone()
    us_gf, _ = timed(layer_gf)
    assert torch.equal(out, out_ref), "the gather-folded layer differs from jam's path"
    ops = 2.0 * R * (FF * D + D * D)
    # the opt-in native-MX mode (not jam's activation semantics): the same layer with the experts' matrix-core
    # calls on the scaled fp4 x fp8 MFMA, MX-FP8 activations hi + lo (mode 1) or hi only (mode 2)
    native = {}
    for mode in (1, 2):
        assert hip.set_mx_native(mode) == JAM.OK
        u, u_stream = timed()
        u_gf, _ = timed(layer_gf)
        assert hip.set_mx_native(0) == JAM.OK
        assert bool(torch.isfinite(out).all()), "moe output not finite"
        native[f"mode{mode}"] = {"us_per_layer": round(u, 1), "us_per_layer_stream": round(u_stream, 1),
                                 "us_per_layer_gather_folded": round(u_gf, 1),
                                 "TOPS": round(ops / (u * 1e-6) / 1e12, 2),
                                 "frac_fp4_peak": round(ops / (u * 1e-6) / 1e12 / 10070.0, 4)}
    native["note"] = ("opt-in jamhip_ctx_set_mx_native: MXFP4 weights as fp4 on v_mfma_scale_f32_32x32x64_f8f6f4, "
                      "activations MX-FP8 hi + lo (mode 1, ~8 bits) or hi only (mode 2, ~4 bits); not jam's "
                      "int8 activation semantics")
    # decode-time layer: one token routed top-4, a different random expert set per layer (64 sets), the two
    # weight copies alternating; jam's F1 decode path (every expert holds one row)
    NL, NDEC = 64, 200
    res = [dev(rng.permutation(E)[:TOPK].astype(np.int32)) for _ in range(NL)]

    def dec_layer(i):
        cg, cd, rd = wg[i % copies], wd[i % copies], res[i % NL]
        ok = hip.moe_route(rd.data_ptr(), 1, TOPK, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                           route_slot.data_ptr()) == JAM.OK
        ok &= hip.moe_gather(x.data_ptr(), D, slot_route.data_ptr(), off.data_ptr(), E, 1, TOPK, D, g.data_ptr(),
                             D) == JAM.OK
        ok &= hip.mm_grouped(Segment.of(cg), JAM.MXFP4, D, FF, E, counts.data_ptr(), g.data_ptr(), D, h.data_ptr(),
                             FF, D, TOPK, None) == JAM.OK
        ok &= hip.mm_grouped(Segment.of(cd), JAM.MXFP4, D, D, E, counts.data_ptr(), hid.data_ptr(), D, y.data_ptr(),
                             D, D, TOPK, None) == JAM.OK
        ok &= hip.moe_combine(y.data_ptr(), D, rd.data_ptr(), prob.data_ptr(), route_slot.data_ptr(), 1, TOPK, E, D,
                              out.data_ptr(), D) == JAM.OK
        if not ok:
            raise RuntimeError(hip.last_error())

    dus, dus_stream = timed(dec_layer, NDEC, 8)
    assert bool(torch.isfinite(out[:1]).all()), "decode moe output not finite"
    ref_h = h.clone()

    def dec_layer_gf(i):   # the gather folded into the gate_up call (jamhip_mm_grouped_gather)
        cg, cd, rd = wg[i % copies], wd[i % copies], res[i % NL]
        ok = hip.moe_route(rd.data_ptr(), 1, TOPK, E, counts.data_ptr(), off.data_ptr(), slot_route.data_ptr(),
                           route_slot.data_ptr()) == JAM.OK
        ok &= hip.mm_grouped_gather(Segment.of(cg), JAM.MXFP4, D, FF, E, counts.data_ptr(), x.data_ptr(), D,
                                    slot_route.data_ptr(), TOPK, h.data_ptr(), FF, D, TOPK) == JAM.OK
        ok &= hip.mm_grouped(Segment.of(cd), JAM.MXFP4, D, D, E, counts.data_ptr(), hid.data_ptr(), D, y.data_ptr(),
                             D, D, TOPK, None) == JAM.OK
        ok &= hip.moe_combine(y.data_ptr(), D, rd.data_ptr(), prob.data_ptr(), route_slot.data_ptr(), 1, TOPK, E, D,
                              out.data_ptr(), D) == JAM.OK
        if not ok:
            raise RuntimeError(hip.last_error())

    dus_gf, _ = timed(dec_layer_gf, NDEC, 8)
    dec_layer(NDEC - 1)
    torch.cuda.synchronize()
    ref_h.copy_(h)
    dec_layer_gf(NDEC - 1)
    torch.cuda.synchronize()
    assert torch.equal(ref_h.view(torch.int32), h.view(torch.int32)), "decode gather-folded gate_up differs"
    dbytes = TOPK * (FF + D) * (D // 32) * 17
    decode = {"us_per_layer": round(dus, 1), "us_per_layer_stream": round(dus_stream, 1),
              "us_per_layer_gather_folded": round(dus_gf, 1),
              "weights_GBs": round(dbytes / (dus * 1e-6) / 1e9, 1),
              "note": "1 token top-4 (a random expert set per layer), route + gather + two grouped calls + combine, "
                      "one captured graph of 200 layers (median of 3 replays; us_per_layer_stream: the same 200 "
                      "layers launched on the stream; us_per_layer_gather_folded: gate_up through "
                      "jamhip_mm_grouped_gather, no gather launch, bit-identical); weights = 4 experts' gate_up + down "
                      "(52.9 MB)"}
    # the same layer the way an unedited jinfer runs it through the host-pointer entry point: Moe.dispatch's host
    # loop (Moe.java:178-232) gathering each expert's rows, one jamhip_mm per expert and matrix on a row view of
    # the pinned stacked tensors (GptOss.java:677-717), the probability-weighted scatter on the host
    rb = (D // 32) * 17
    re_h, x_h, hid_h, prob_h = sel.ravel(), x.cpu().numpy(), hid.cpu().numpy(), prob.cpu().numpy()
    by_e = np.argsort(re_h, kind="stable")
    off_h = np.concatenate([[0], np.cumsum(counts_h)])
    hb = [np.empty((int(c_), FF), np.float32) for c_ in counts_h]
    yb = [np.empty((int(c_), D), np.float32) for c_ in counts_h]

    def host_layer():
        acc = np.zeros((SEQ, D), np.float32)
        for e in range(E):
            r = by_e[off_h[e]:off_h[e + 1]]
            ne = len(r)
            if ne == 0:
                continue
            xe, he = np.ascontiguousarray(x_h[r // TOPK]), np.ascontiguousarray(hid_h[r])
            ok = hip.mm(Segment.of(wg[0]), e * FF * rb, JAM.MXFP4, D, Segment.of(xe), 0, JAM.F32, D, Segment.of(hb[e]),
                        0, JAM.F32, FF, FF, ne, D) == JAM.OK
            ok &= hip.mm(Segment.of(wd[0]), e * D * rb, JAM.MXFP4, D, Segment.of(he), 0, JAM.F32, D, Segment.of(yb[e]),
                         0, JAM.F32, D, D, ne, D) == JAM.OK
            if not ok:
                raise RuntimeError(hip.last_error())
            acc[r // TOPK] += prob_h[r, None] * yb[e]
        return acc

    host_layer()
    t0 = time.perf_counter()
    for _ in range(3):
        host_layer()
    host_us = (time.perf_counter() - t0) / 3 * 1e6
    for xx in wg + wd:
        hip.evict(Segment.of(xx))
    wbytes = E * (FF + D) * (D // 32) * 17
    tops = ops / (us * 1e-6) / 1e12
    gbs = wbytes / (us * 1e-6) / 1e9
    return {"us_per_layer": round(us, 1), "us_per_layer_stream": round(us_stream, 1), "TOPS": round(tops, 2),
            "us_per_layer_gather_folded": round(us_gf, 1),
            "weights_GBs": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "frac_fp4_peak": round(tops / 10070.0, 4), "routed_rows": R,
            "counts": counts_h.tolist(), "mx_native": native, "decode": decode,
            "host_pointer_layer_us": round(host_us, 1),
            "host_pointer_note": "the layer as 64 jamhip_mm calls with host A and C (one per expert and matrix, on row "
                                 "views of the pinned stacked experts) plus the host-side gather and weighted scatter, "
                                 "wall clock, mean of 3",
            "note": "32 experts x (5760x2880 + 2880x2880) MXFP4 (423 MB, 2 rotating copies; experts cycle through "
                    "2 distinct N(0,0.02) quantizations), 512 tokens top-4 Zipf(1.1); ops = 2*routed_rows*"
                    "(5760*2880 + 2880*2880); us_per_layer: one captured graph of the timed layers, median of 3 "
                    "replays; us_per_layer_stream: the same layers launched on the stream; "
                    "us_per_layer_gather_folded: the same layer with jamhip_moe_gather folded into the gate_up call "
                    "(jamhip_mm_grouped_gather, bit-identical output)"}


def decode_step_leg(hip, torch, stream, w_gate: np.ndarray, reps: int = 8) -> dict:
    """Config 3: a Llama-3-8B Q4_K_M-style decode step, matmuls only. Per layer q 4096x4096, k / v
    1024x4096, o 4096x4096, gate / up 14336x4096 in Q4_K and down 4096x14336 in Q6_K; 32 layers and the
    128256x4096 Q6_K output head: 4.84 GB of weights, each layer's in its own HBM allocations. One token
    (n = 1, jam's F1 decode path); every layer reads the same synthetic activations (matmuls only, as the
    config says). Weight values: one N(0,0.02) quantization per shape, copied into every layer (the
    kernels' work does not depend on the values). Two schedules of the same bytes:
      separate  7 calls per layer, as jinfer issues them (225 launches);
      fused     q|k|v and gate|up as one call each over weights laid out back to back (the way a GGUF file
                stores a block's tensors), 4 calls per layer (129 launches): the same rows, outputs
                concatenated.
    Timed: `reps` replays of one captured graph per schedule, HIP events on the library's stream."""
    from qxotic_amd.jam import JAM, Segment

    layers, D, KV, FF, V = 32, 4096, 1024, 14336, 128256
    dd, kv = quantized("Q4_K", D, D, 0xD301), quantized("Q4_K", KV, D, 0xD302)
    down = quantized("Q6_K", D, FF, 0xD303)
    blk = quantized("Q6_K", 4096, D, 0xD304)
    head = np.ascontiguousarray(np.concatenate([blk] * ((V + 4095) // 4096))[:V])
    plans = {"separate": [], "fused": []}   # (weight, dtype, m, k)
    for _ in range(layers):
        plans["separate"] += [(dd.copy(), JAM.Q4_K, D, D), (kv.copy(), JAM.Q4_K, KV, D), (kv.copy(), JAM.Q4_K, KV, D),
                              (dd.copy(), JAM.Q4_K, D, D), (w_gate.copy(), JAM.Q4_K, FF, D),
                              (w_gate.copy(), JAM.Q4_K, FF, D), (down.copy(), JAM.Q6_K, D, FF)]
        plans["fused"] += [(np.concatenate([dd, kv, kv]), JAM.Q4_K, D + 2 * KV, D), (dd.copy(), JAM.Q4_K, D, D),
                           (np.concatenate([w_gate, w_gate]), JAM.Q4_K, 2 * FF, D), (down.copy(), JAM.Q6_K, D, FF)]
    for p in plans.values():
        p.append((head, JAM.Q6_K, V, D))
    wbytes = sum(x[0].nbytes for x in plans["separate"])
    assert wbytes == sum(x[0].nbytes for x in plans["fused"])
    x_d = torch.randn((1, D), device="cuda")
    h_d = torch.randn((1, FF), device="cuda")
    out = {}
    for name, plan in plans.items():
        for w, dt, m, k in plan:
            assert hip.pin(Segment.of(w), dt, k, m) == JAM.OK, hip.last_error()
        outs = {m: torch.empty((1, m), device="cuda") for m in {x[2] for x in plan}}

        def step():
            for w, dt, m, k in plan:
                a = h_d if k == FF else x_d
                st = hip.mm_device(Segment.of(w), dt, k, a.data_ptr(), k, outs[m].data_ptr(), m, m, 1, k)
                if st != JAM.OK:
                    raise RuntimeError(hip.last_error())

        with torch.cuda.stream(stream):
            step()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        io = sum(4 * (k + m) for _, _, m, k in plan)
        gbs = (wbytes + io) / (us * 1e-6) / 1e9
        out[name] = {"us_per_token": round(us, 1), "tokens_per_s": round(1e6 / us, 1), "launches": len(plan),
                     "GBs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        if name == "separate":   # the same 225 calls through jamhip_mm with host A and C, as an unedited jinfer
            a_h, h_h = x_d.cpu().numpy(), h_d.cpu().numpy()
            outs_h = {m: np.empty((1, m), np.float32) for m in outs}

            def host_step():
                for w, dt, m, k in plan:
                    if hip.mm_contiguous(Segment.of(w), Segment.of(h_h if k == FF else a_h), Segment.of(outs_h[m]), dt,
                                         m, 1, k) != JAM.OK:
                        raise RuntimeError(hip.last_error())

            host_step()
            t0 = time.perf_counter()
            for _ in range(3):
                host_step()
            out[name]["host_pointer_us_per_token"] = round((time.perf_counter() - t0) / 3 * 1e6, 1)
        for w, _, _, _ in plan:
            if w is not head or name == "fused":
                hip.evict(Segment.of(w))
        del g
    out["weights_GB"] = round(wbytes / 1e9, 3)
    out["note"] = ("config 3: 32 Llama-3-8B layers (q/k/v/o/gate/up Q4_K, down Q6_K) + Q6_K output head, n = 1, "
                   "matmuls only, one captured graph per schedule; GB/s = weights + activations + outputs; "
                   "host_pointer_us_per_token = the 225 calls through jamhip_mm with host A and C, wall clock")
    return out


def epilogue_leg(hip, torch, stream, steps: int = 512) -> dict:
    """Fused epilogue on gpt-oss-20B's attention output projection at decode (Q8_0 2880x4096, n = 1, with
    bias, then the residual add): separate = jamhip_mm_device + bias add + residual add (jinfer's order:
    MatMul.gemm, Ops.addRowBiasInPlace, Ops.addInPlace; 3 launches), fused = jamhip_mm_device_ex (1 launch).
    Each timed as a captured graph of `steps` steps over 32 rotating weight copies (400 MB)."""
    from qxotic_amd.jam import JAM, Segment

    m, k, copies = 2880, 4096, 32
    w = quantized("Q8_0", m, k, 0xA77E)
    ws = [w.copy() for _ in range(copies)]
    for x in ws:
        assert hip.pin(Segment.of(x), JAM.Q8_0, k, m) == JAM.OK, hip.last_error()
    a = torch.randn((1, k), device="cuda")
    bias = torch.randn((m,), device="cuda")
    tmp = torch.empty((1, m), device="cuda")
    res = {v: torch.randn((1, m), device="cuda") for v in ("separate", "fused")}
    res["fused"].copy_(res["separate"])

    def step(variant, i):
        x = Segment.of(ws[i % copies])
        r = res[variant]
        if variant == "fused":
            st = hip.mm_device_ex(x, JAM.Q8_0, k, a.data_ptr(), k, r.data_ptr(), m, m, 1, k, bias.data_ptr(), True)
        else:
            st = hip.mm_device(x, JAM.Q8_0, k, a.data_ptr(), k, tmp.data_ptr(), m, m, 1, k)
            tmp.add_(bias)
            r.add_(tmp)
        if st != JAM.OK:
            raise RuntimeError(hip.last_error())

    out = {}
    with torch.cuda.stream(stream):
        for v in ("separate", "fused"):   # one step each from the same residual: identical f32 operations
            step(v, 0)
        torch.cuda.synchronize()
        assert torch.equal(res["separate"], res["fused"]), "fused epilogue disagrees with the separate passes"
        for v in ("separate", "fused"):
            for i in range(16):
                step(v, i)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(steps):
                    step(v, i)
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            out[v] = e0.elapsed_time(e1) * 1e3 / steps
    for x in ws:
        hip.evict(Segment.of(x))
    return {"separate_us": round(out["separate"], 2), "fused_us": round(out["fused"], 2),
            "saved_us": round(out["separate"] - out["fused"], 2),
            "note": "gpt-oss-20B attn_output Q8_0 2880x4096, n=1, bias + residual; graph-timed, 32 rotating "
                    "weight copies; separate = matmul + bias add + residual add (3 launches), fused = 1 launch"}


def registry_leg(hip, layers: int = 2) -> dict:
    """Model load through the GGUF device weight registry: a synthetic GGUF holding `layers` gpt-oss-20B
    layers' jam weights (attention q/k/v/o in Q8_0, stacked gate/up/down experts 32 x 2880 x 2880 in MXFP4,
    f32 norms and biases), random bytes, freshly written (so page-cache warm). Timed: jamhip_gguf_open +
    jamhip_gguf_pin (parse, map, H2D of every jam tensor, repack to the device layout) on the wall clock;
    twice, the second after jamhip_gguf_evict."""
    import tempfile
    from qxotic_amd import gguf as G
    from qxotic_amd.ggml import BY_NAME

    q8, mx, f32 = BY_NAME["Q8_0"], BY_NAME["MXFP4"], BY_NAME["F32"]
    D, E, HQ, HKV = 2880, 32, 4096, 512
    rng = np.random.default_rng(0x6E6E)
    blob = lambda t, rows, cols: rng.integers(0, 256, rows * t.row_bytes(cols), dtype=np.uint8)
    tensors = []
    for l in range(layers):
        p = f"blk.{l}."
        tensors += [(p + "attn_norm.weight", f32.ggml, (D,), np.ones(D, np.float32)),
                    (p + "attn_q.weight", q8.ggml, (D, HQ), blob(q8, HQ, D)),
                    (p + "attn_k.weight", q8.ggml, (D, HKV), blob(q8, HKV, D)),
                    (p + "attn_v.weight", q8.ggml, (D, HKV), blob(q8, HKV, D)),
                    (p + "attn_output.weight", q8.ggml, (HQ, D), blob(q8, D, HQ))]
        for name in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
            tensors += [(p + name + ".weight", mx.ggml, (D, D, E), blob(mx, E * D, D)),
                        (p + name + ".bias", f32.ggml, (D, E), np.zeros(D * E, np.float32))]
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "model.gguf"
        G.write(path, tensors, [("general.architecture", "string", "gpt-oss")])
        del tensors
        size = path.stat().st_size
        runs = []
        for _ in range(2):
            t0 = time.perf_counter()
            g = G.GGUF(path)
            st, cnt, nbytes = g.pin(hip)
            dt = time.perf_counter() - t0
            assert st == 0, hip.last_error()
            runs.append(dt)
            assert g.evict(hip) == cnt
            g.close()
    best = min(runs)
    return {"file_GB": round(size / 1e9, 3), "pinned_tensors": cnt, "pinned_GB": round(nbytes / 1e9, 3),
            "s": [round(r, 4) for r in runs], "GBs": round(nbytes / best / 1e9, 2),
            "note": f"{layers} gpt-oss-20B layers' jam weights (Q8_0 attention, 3 stacked 32-expert MXFP4 "
                    "tensors per layer), page-cache-warm file; open + pin on the wall clock, best of 2"}


def cpu_leg(w: np.ndarray, budget_s: float = 4.0) -> dict | None:
    """The reference's own libjam (oracle/_ref), same workload, 32 rotating host copies (1.06 GB, far
    above any L3), one thread per allotted core."""
    try:
        from oracle import oracle as O
    except Exception as e:   # pragma: no cover
        log(f"cpu baseline unavailable: {e}")
        return None
    if not O.ref_available():
        log("cpu baseline unavailable: oracle/_ref/libjam.so not built")
        return None
    threads = O.default_threads()
    ref = O.RefJam(nthreads=threads)
    copies = [w.copy() for _ in range(COPIES)]
    a = np.random.default_rng(7).standard_normal((N, K)).astype(np.float32)
    c = np.zeros((N, M), np.float32)
    for cp in copies[:2]:
        ref.mm(O.Q4_K, cp, a, M, N, K, out=c)
    calls = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        ref.mm(O.Q4_K, copies[calls % COPIES], a, M, N, K, out=c)
        calls += 1
    dt = time.perf_counter() - t0
    ref.close()
    return {"value": round(calls * STEP_BYTES / dt / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "reference",
            "sample": f"libjam jam_mm (reference C sources, isa avx512_vnni dispatch) Q4_K 14336x4096 M=1, "
                      f"{calls} calls over {COPIES} rotating host copies in {dt:.1f} s"}


def cpu_gemm_leg(budget_s: float = 4.0) -> dict | None:
    """libjam (oracle/_ref) at the GEMM shapes, one thread per allotted core, on bounded row samples of the
    same weights (jam_bench.c:77-90 times M x N x K the same way): config 4's Q4_K 14336x4096 and Q6_K
    4096x14336 at M = 512 (F2 bands, jam.c:489-499), and config 5's 32 MXFP4 experts with their routed
    counts (gate_up 5760x2880 and down 2880x2880 per expert, jam's per-expert calls as Moe.dispatch makes
    them). Each sample is repeated for `budget_s` seconds; ops = 2·rows·n·k per call."""
    try:
        from oracle import oracle as O
    except Exception as e:   # pragma: no cover
        log(f"cpu gemm baseline unavailable: {e}")
        return None
    if not O.ref_available():
        return None
    threads = O.default_threads()
    ref = O.RefJam(nthreads=threads)
    out = {}

    def timed(calls_fn):
        calls_fn()                              # warm
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < budget_s:
            calls_fn()
            reps += 1
        return reps, time.perf_counter() - t0

    n = 512
    for name, dt, m, k, rows in (("Q4_K", O.Q4_K, 14336, 4096, 1024), ("Q6_K", O.Q6_K, 4096, 14336, 512)):
        w = quantized(name, rows, k, 0x5EED ^ dt)        # the GPU leg's distribution, a row sample
        a = np.random.default_rng(11).standard_normal((n, k)).astype(np.float32)
        c = np.zeros((n, rows), np.float32)
        reps, dt_s = timed(lambda: ref.mm(dt, w, a, rows, n, k, out=c))
        tops = reps * 2.0 * rows * n * k / dt_s / 1e12
        out[f"{name} {m}x{k} M=512"] = {"TOPS": round(tops, 3), "sample": f"rows 0..{rows - 1} of {m}, "
                                        f"{reps} calls in {dt_s:.1f} s"}
    E, D, FF, frac = 32, 2880, 5760, 8
    counts = [388, 268, 191, 124, 112, 115, 76, 67, 61, 57, 52, 50, 44, 42, 27, 39, 28, 30, 26, 25, 26, 18, 19,
              19, 19, 30, 15, 20, 14, 21, 11, 14]   # the GPU leg's Zipf(1.1) top-4 routing of 512 tokens
    gu = quantized("MXFP4", FF // frac, D, 0xC0F5)
    dn = quantized("MXFP4", D // frac, D, 0xD0F5)
    xs = [np.random.default_rng(e).standard_normal((c_, D)).astype(np.float32) for e, c_ in enumerate(counts)]
    cg = [np.zeros((c_, FF // frac), np.float32) for c_ in counts]
    cd = [np.zeros((c_, D // frac), np.float32) for c_ in counts]

    def layer():
        for e in range(E):
            ref.mm(O.MXFP4, gu, xs[e], FF // frac, counts[e], D, out=cg[e])
            ref.mm(O.MXFP4, dn, xs[e], D // frac, counts[e], D, out=cd[e])
    reps, dt_s = timed(layer)
    ops = 2.0 * sum(counts) * (FF // frac + D // frac) * D
    out["MoE config 5 layer"] = {"TOPS": round(reps * ops / dt_s / 1e12, 3),
                                 "us_per_layer_scaled": round(dt_s / reps * frac * 1e6, 1),
                                 "sample": f"1/{frac} of every expert's rows (gate_up {FF // frac}, down {D // frac}) "
                                           f"at the routed counts, 64 jam_mm calls per layer, {reps} layers in "
                                           f"{dt_s:.1f} s; us_per_layer_scaled = x{frac}"}
    ref.close()
    out.update({"cores": threads, "kind": "reference", "unit": "TOPS",
                "note": "libjam jam_mm (reference C sources, isa avx512_vnni dispatch), int8 ops counted as 2*M*N*K"})
    return out


def traffic_from_profiles() -> int | None:
    """HBM bytes per GEMV launch, measured by rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (calibrated)."""
    try:
        m = re.search(r"^bytes_per_launch:\s*(\d+)", TRAFFIC_SUMMARY.read_text(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-registry", action="store_true")
    ap.add_argument("--no-epilogue", action="store_true")
    ap.add_argument("--no-step", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--no-read-floor", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (every GPU box here has one; the matmul would "
              "shard by weight rows, one process per GPU); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    from qxotic_amd.jam import HipJAM

    torch.cuda.set_device(0)
    if args.calibrate_copy:
        calibrate_copy(torch)
    hip = HipJAM(0)
    stream = torch.cuda.Stream()
    hip.set_stream(stream.cuda_stream)
    log("bench: quantizing weights")
    w = quantized("Q4_K", M, K, 0x5A11C0DE ^ 3)
    log("bench: decode leg")
    g = gpu_leg(args, w, hip, torch, stream)
    ms = g["event_ms"] / args.steps
    gbs = STEP_BYTES / (ms * 1e-3) / 1e9
    floor = None
    if not args.no_read_floor:
        log("bench: read floor leg")
        floor = read_floor_leg(args, hip, torch, stream)
        floor["decode_frac"] = round(floor["us"] / (ms * 1e3), 4)
    shapes = None
    if not args.no_shapes:
        log("bench: decode shapes leg (configs 1, 2 and the Q6_K down projection)")
        shapes = shapes_leg(hip, torch, stream)
    pre = None
    if not args.no_prefill:
        log("bench: prefill leg")
        pre = prefill_leg(hip, torch, stream)
    moe = None
    if not args.no_moe:
        log("bench: moe leg")
        moe = moe_leg(hip, torch, stream, no_graph=args.no_graph)
    step = None
    if not args.no_step:
        log("bench: decode step leg")
        step = decode_step_leg(hip, torch, stream, w)
    epi = None
    if not args.no_epilogue:
        log("bench: epilogue leg")
        epi = epilogue_leg(hip, torch, stream)
    reg = None
    if not args.no_registry:
        log("bench: registry leg")
        reg = registry_leg(hip)
    hip.close()
    cpu = cpu_gemm = None
    if not args.no_cpu:
        log("bench: cpu baseline")
        cpu = cpu_leg(w)
        if not (args.no_prefill and args.no_moe):
            log("bench: cpu gemm baseline")
            cpu_gemm = cpu_gemm_leg()
    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Q4_K GEMV 14336x4096 M=1 (Llama-3-8B gate/up, F1 activation quant fused), "
                               f"{COPIES} rotating HBM-resident weight copies ({COPIES * M * 16 * 144 / 1e9:.2f} GB)",
                   "weights": "N(0,0.02) quantized to Q4_K", "activations": "N(0,1) f32",
                   "graph_launches": 0 if args.no_graph else args.steps, "wall_s": round(g["wall_s"], 4)},
        "host_pointer_call": {"us": round(g["host_us"], 2), "GBs": round(STEP_BYTES / (g["host_us"] * 1e-6) / 1e9, 1),
                              "note": "jamhip_mm with host A and C (16 KiB upload, 56 KiB of C stored by the kernel "
                                      "into pinned host memory, sync per call), pinned weights, wall clock; not the metric",
                              "unpinned_staged_us": round(g["staged_us"], 2), "unpinned_autopin_us": round(g["auto_us"], 2),
                              "autopin_note": "the same call on a weight nobody pinned: staged every call, then with "
                                              "jamhip_ctx_set_autopin(2) (pinned on its 2nd call, spot-checked each call)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles()},
        "read_floor": floor,
        "decode_shapes": shapes,
        "prefill": pre,
        "moe": moe,
        "decode_step": step,
        "epilogue": epi,
        "registry": reg,
        "cpu_baseline": cpu,
        "jam_vector": "not run: no JDK 25 (jdk.incubator.vector) on the GPU box or in the build image",
        "cpu_baseline_gemm": cpu_gemm,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
