"""Benchmark of the MI355X jam backend on BASELINE.json's headline metric.

Step = one decode matmul of jam's hot path: Q4_K GEMV 14336x4096, M=1 (Llama-3-8B gate/up projection),
activation quantization (jam's F1) included, through the C-ABI device entry point. Weights are resident
in HBM before timing: 32 distinct copies (1.06 GB, > the 256 MB Infinity Cache) rotate so no step is
served from cache. The K timed steps are one captured HIP graph of K launches on the library's stream,
timed with HIP events on that stream between a synchronize on each side.

Also reported (same JSON line): the roofline of the dominant kernel and the reference's own CPU path
(libjam built from the reference sources, oracle/_ref) timed on this machine's host cores.

    python bench.py [--gpus 1] [--steps 2048] [--warmup 64]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

M, K, N = 14336, 4096, 1
COPIES = 32
HBM_PEAK_GBS = 8000.0
# Algorithmic bytes per step, each operand once (jam_bench.c:46-75): W + A (f32) + C (f32).
STEP_BYTES = M * (K // 256) * 144 + N * K * 4 + N * M * 4   # 33,103,872
METRIC = "GB/s (%HBM peak) Q4_K GEMV 14336x4096 M=1; TOPS (%MFMA) M=512 prefill"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weights(seed: int) -> np.ndarray:
    from qxotic_amd import ggml
    x = np.random.default_rng(seed).normal(0.0, 0.02, (M, K)).astype(np.float32)
    return ggml.quantize("Q4_K", x)


def gpu_leg(args, w: np.ndarray) -> dict:
    import torch
    from qxotic_amd.jam import JAM, HipJAM, Segment

    torch.cuda.set_device(0)
    hip = HipJAM(0)
    stream = torch.cuda.Stream()
    hip.set_stream(stream.cuda_stream)
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

    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(args.steps):
                step(i)
        graph.replay()   # warm replay
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1)
    # correctness spot check of the last output against a direct call
    ref = torch.empty((N, M), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(stream):
        st = hip.mm_device(Segment.of(copies[0]), JAM.Q4_K, K, a.data_ptr(), K, ref.data_ptr(), M, M, N, K)
    torch.cuda.synchronize()
    assert st == JAM.OK and torch.equal(ref, c[0]), "graph replay disagrees with a direct call"
    for cp in copies:
        hip.evict(Segment.of(cp))
    hip.close()
    return {"event_ms": ev_ms, "wall_s": wall}


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
    """HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE (profiles/)."""
    p = ROOT / "profiles" / "q4k_gemv_14336x4096_traffic.json"
    if p.exists():
        try:
            return int(json.loads(p.read_text())["bytes_per_launch"])
        except Exception:
            return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the matmul shards by weight rows; "
              "see DESIGN.md); run with --gpus 1", file=sys.stderr)
        return 2
    log("bench: quantizing weights")
    w = make_weights(0x5A11C0DE ^ 3)
    log("bench: gpu leg")
    g = gpu_leg(args, w)
    ms = g["event_ms"] / args.steps
    gbs = STEP_BYTES / (ms * 1e-3) / 1e9
    cpu = None if args.no_cpu else cpu_leg(w)
    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Q4_K GEMV 14336x4096 M=1 (Llama-3-8B gate/up, F1 activation quant fused), "
                               f"{COPIES} rotating HBM-resident weight copies ({COPIES * M * 16 * 144 / 1e9:.2f} GB)",
                   "weights": "N(0,0.02) quantized to Q4_K", "activations": "N(0,1) f32",
                   "graph_launches": args.steps, "wall_s": round(g["wall_s"], 4)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
