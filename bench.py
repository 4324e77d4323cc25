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
  * ``prefill``: the metric's second half, M=512 prefill TOPS of Q4_K 14336x4096 and Q6_K 4096x14336
    (activations 99% N(0,1) + 1% outliers at +-20, F2-quantized in the timed calls) against MI355X's dense
    int8 and f16 MFMA peaks;
  * ``cpu_baseline``: the reference's own libjam (oracle/_ref, built from the reference C sources) on the
    same decode workload on this machine's host cores.

    python bench.py [--gpus 1] [--steps 2048] [--warmup 64] [--no-cpu] [--no-prefill]
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
    for cp in copies:
        hip.evict(Segment.of(cp))
    return {"event_ms": ev_ms, "wall_s": wall}


def prefill_leg(hip, torch, stream, reps: int = 10) -> dict:
    """M=512 prefill on the two BASELINE prefill shapes; each timed call quantizes its activations (F2)."""
    from qxotic_amd.jam import JAM, Segment

    out = {}
    n = 512
    for name, dt, m, k in (("Q4_K", JAM.Q4_K, 14336, 4096), ("Q6_K", JAM.Q6_K, 4096, 14336)):
        w = quantized(name, m, k, 0x5EED ^ dt)
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
        out[f"{name} {m}x{k} M=512"] = {"us": round(us, 2), "TOPS": round(tops, 2),
                                        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                        "frac_f16_peak": round(tops / F16_PEAK_TFLOPS, 4)}
        hip.evict(Segment.of(w))
        del a, c
    out["note"] = ("jam's F2 quantization + int8 products computed exactly on f16 MFMA (integer operands "
                   "<= 2048); peaks are MI355X dense int8 5.0 POP/s and f16 2.5 PFLOP/s")
    return out


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
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
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
    pre = None
    if not args.no_prefill:
        log("bench: prefill leg")
        pre = prefill_leg(hip, torch, stream)
    hip.close()
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline")
        cpu = cpu_leg(w)
    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Q4_K GEMV 14336x4096 M=1 (Llama-3-8B gate/up, F1 activation quant fused), "
                               f"{COPIES} rotating HBM-resident weight copies ({COPIES * M * 16 * 144 / 1e9:.2f} GB)",
                   "weights": "N(0,0.02) quantized to Q4_K", "activations": "N(0,1) f32",
                   "graph_launches": 0 if args.no_graph else args.steps, "wall_s": round(g["wall_s"], 4)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles()},
        "prefill": pre,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
