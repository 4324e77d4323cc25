"""GPU: the boundary's lifecycle and concurrency contract, through the C-ABI.

* ctx == NULL selects the process-global context, created on first use and released by
  jamhip_global_destroy (jam.h:128, 149-155; jam.c:420-437, 765-768; jam_test.c:445-457, 482-486);
* a context is a serial stream: a contended call returns EBUSY when the fair lock is off, and with the fair
  lock (the default) concurrent callers all succeed with bit-identical results (jam_test.c:475-480,
  JamTest.java:580-629);
* create / use / destroy cycles return every device byte (jam_test.c:522-567);
* a HIP graph captured around a call stays valid after a later, larger call grows the context's scratch;
* a process that exits with contexts and GGUF mappings still open tears down cleanly.
"""
import ctypes as C
import os
import subprocess
import sys
import threading
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def raw_mm(ctx, dt, w, a, c, m, n, k):
    from qxotic_amd._lib import lib
    return lib().jamhip_mm(ctx, w.ctypes.data, dt, k, a.ctypes.data, O.F32, k, c.ctypes.data, O.F32, m, m, n, k)


def test_null_context_is_the_global_one(hip, oracle):
    """jamhip_mm(NULL, ...) computes on the global context (same answer as an explicit context, bit for
    bit), the global context is a singleton, survives until jamhip_global_destroy, and is re-created by the
    next NULL call; a failed NULL call leaves its message in jamhip_last_error(NULL)."""
    from qxotic_amd._lib import lib
    L = lib()
    m, k = 96, 1024
    w = oracle.quantize(O.Q4_K, oracle.normal(41, (m, k), 0.0, 0.02))
    for n in (1, 9):
        say(f"global context n={n}")
        a = oracle.normal(42 + n, (n, k))
        want = np.zeros((n, m), np.float32)
        assert raw_mm(hip.ctx, O.Q4_K, w, a, want, m, n, k) == 0
        got = np.zeros((n, m), np.float32)
        assert raw_mm(None, O.Q4_K, w, a, got, m, n, k) == 0, L.jamhip_last_error(None)
        assert np.array_equal(bits(got), bits(want))
    assert L.jamhip_ctx_arch(None).decode().startswith("gfx950")
    s0 = L.jamhip_ctx_stream(None)
    assert s0 and L.jamhip_ctx_stream(None) == s0          # singleton
    # pins made through NULL live on the global context
    assert L.jamhip_weight_pin(None, w.ctypes.data, O.Q4_K, k, m) == 0
    assert L.jamhip_weight_bytes(None) > 0
    got = np.zeros((1, m), np.float32)
    assert raw_mm(None, O.Q4_K, w, oracle.normal(43, (1, k)), got, m, 1, k) == 0
    # a failure on the global context reports through jamhip_last_error(NULL)
    bad = np.zeros((1, m), np.float32)
    st = L.jamhip_mm(None, w.ctypes.data, O.Q4_K, k, a.ctypes.data, O.F16, k, bad.ctypes.data, O.F32, m, m, 1, k)
    assert st == 2 and b"F32" in L.jamhip_last_error(None)
    L.jamhip_global_destroy()
    assert L.jamhip_weight_bytes(None) == 0                  # pins went with it
    L.jamhip_global_destroy()                                # idempotent
    again = np.zeros((9, m), np.float32)
    a = oracle.normal(42 + 9, (9, k))
    assert raw_mm(None, O.Q4_K, w, a, again, m, 9, k) == 0   # lazily re-created
    assert np.array_equal(bits(again), bits(want))
    L.jamhip_global_destroy()


def _contend(jam, w, dt, m, k, threads, rounds, seed):
    """threads x rounds calls through jam.mm, all threads released together each round; returns the
    status counts and every thread's last output."""
    from qxotic_amd.jam import JAM, Segment
    barrier = threading.Barrier(threads)
    counts = {"ok": 0, "ebusy": 0, "other": 0}
    mu = threading.Lock()
    n = 8
    a = np.random.default_rng(seed).standard_normal((n, k)).astype(np.float32)
    outs = [np.zeros((n, m), np.float32) for _ in range(threads)]

    def work(t):
        for _ in range(rounds):
            barrier.wait()
            st = jam.mm(Segment.of(w), 0, dt, k, Segment.of(a), 0, JAM.F32, k, Segment.of(outs[t]), 0, JAM.F32, m,
                        m, n, k)
            with mu:
                counts["ok" if st == JAM.OK else "ebusy" if st == JAM.EBUSY else "other"] += 1

    ts = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
        assert not t.is_alive(), "a contended call never returned"
    return counts, outs, a


def test_fair_lock_serializes_concurrent_callers(oracle, monkeypatch):
    """JAM_HIP_SERIAL unset (jam.hip.serial=true): 4 threads x 20 simultaneous calls on one context all
    return OK, none EBUSY, and every output equals the single-threaded answer bit for bit."""
    from qxotic_amd.jam import JAM, HipJAM, Segment
    monkeypatch.delenv("JAM_HIP_SERIAL", raising=False)
    jam = HipJAM()
    try:
        m, k = 256, 2048
        w = oracle.quantize(O.Q4_K, oracle.normal(51, (m, k), 0.0, 0.02))
        say("fair lock: 4 threads x 20 rounds")
        counts, outs, a = _contend(jam, w, O.Q4_K, m, k, 4, 20, 52)
        assert counts == {"ok": 80, "ebusy": 0, "other": 0}, counts
        want = np.zeros((8, m), np.float32)
        assert jam.mm(Segment.of(w), 0, O.Q4_K, k, Segment.of(a), 0, JAM.F32, k, Segment.of(want), 0, JAM.F32, m, m,
                      8, k) == JAM.OK
        for o in outs:
            assert np.array_equal(bits(o), bits(want))
    finally:
        jam.close()


def test_ebusy_without_fair_lock(oracle, monkeypatch):
    """JAM_HIP_SERIAL=false (jam.hip.serial=false): the native serial-stream guard answers a call that
    arrives while another is in flight with EBUSY (jam.c:777-783), never anything else; the calls that ran
    are bit-identical to the single-threaded answer. Each round releases 4 threads onto a call that stages
    a 48 MB unpinned weight, so the calls overlap."""
    from qxotic_amd.jam import JAM, HipJAM, Segment
    monkeypatch.setenv("JAM_HIP_SERIAL", "false")
    jam = HipJAM()
    try:
        assert jam._lock is None
        m, k = 4096, 14336
        w = oracle.quantize(O.Q6_K, oracle.normal(61, (m, k), 0.0, 0.02))
        say("no fair lock: 4 threads x 6 rounds, staged 48 MB weight")
        counts, outs, a = _contend(jam, w, O.Q6_K, m, k, 4, 6, 62)
        assert counts["other"] == 0, counts
        assert counts["ebusy"] >= 1, counts
        assert counts["ok"] >= 6, counts
        want = np.zeros((8, m), np.float32)
        assert jam.mm(Segment.of(w), 0, O.Q6_K, k, Segment.of(a), 0, JAM.F32, k, Segment.of(want), 0, JAM.F32, m, m,
                      8, k) == JAM.OK
        for o in outs:
            if o.any():   # a thread whose every call met EBUSY left its output untouched
                assert np.array_equal(bits(o), bits(want))
        assert "busy" in jam.last_error() or counts["ebusy"] > 0
    finally:
        jam.close()


def test_create_use_destroy_returns_device_memory(oracle):
    """128 cycles of create -> use every lazily grown buffer (fused decode, split-K decode, F1 copy, F2
    tiles, matrix-core prep, pinned weight) -> destroy: device memory in use returns to where it started
    (the leak gate of jam_test.c:522-567, on device bytes)."""
    import torch
    from qxotic_amd.jam import JAM, HipJAM, Segment
    k1, k2, m = 1024, 9216, 64
    w1 = oracle.quantize(O.Q4_K, oracle.normal(71, (m, k1), 0.0, 0.02))
    w2 = oracle.quantize(O.Q8_0, oracle.normal(72, (m, k2), 0.0, 0.02))
    a1 = oracle.normal(73, (40, k1))
    a2 = oracle.normal(74, (4, k2))

    def use(h):
        c = np.zeros((40, m), np.float32)
        for n in (1, 9, 40):
            assert h.mm(Segment.of(w1), 0, JAM.Q4_K, k1, Segment.of(a1), 0, JAM.F32, k1, Segment.of(c), 0, JAM.F32, m,
                        m, n, k1) == JAM.OK
        assert h.pin(Segment.of(w2), JAM.Q8_0, k2, m) == JAM.OK
        assert h.mm(Segment.of(w2), 0, JAM.Q8_0, k2, Segment.of(a2), 0, JAM.F32, k2, Segment.of(c), 0, JAM.F32, m, m,
                    4, k2) == JAM.OK

    torch.cuda.synchronize()
    for _ in range(2):                      # settle one-time allocations (code objects, runtime pools)
        h = HipJAM()
        use(h)
        h.close()
    free0, _ = torch.cuda.mem_get_info()
    say("leak gate: 128 create/use/destroy cycles")
    for _ in range(128):
        h = HipJAM()
        use(h)
        h.close()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 - free1 < 32 << 20, f"device memory in use grew by {(free0 - free1) >> 20} MiB over 128 cycles"


def test_graph_replay_after_scratch_growth(hip, oracle):
    """A HIP graph captured around a split-K decode call (its partial sums live in the context's scratch)
    replays correctly after a later, larger call has grown that scratch: the captured address is retired,
    not freed. Each replay, with eager work between them, equals the eager result bit for bit."""
    import torch
    from qxotic_amd.jam import JAM, Segment
    m, k, n = 256, 9216, 4
    w = oracle.quantize(O.Q4_0, oracle.normal(81, (m, k), 0.0, 0.02))
    wbig = oracle.quantize(O.Q4_0, oracle.normal(82, (4096, 16384), 0.0, 0.02))
    assert hip.pin(Segment.of(w), JAM.Q4_0, k, m) == JAM.OK
    assert hip.pin(Segment.of(wbig), JAM.Q4_0, 16384, 4096) == JAM.OK
    s = torch.cuda.Stream()
    hip.set_stream(s.cuda_stream)
    try:
        a = torch.from_numpy(oracle.normal(83, (n, k))).cuda()
        c = torch.zeros((n, m), dtype=torch.float32, device="cuda")
        with torch.cuda.stream(s):
            assert hip.mm_device(Segment.of(w), JAM.Q4_0, k, a.data_ptr(), k, c.data_ptr(), m, m, n, k) == JAM.OK
        s.synchronize()
        eager = c.clone()
        g = torch.cuda.CUDAGraph()
        c.zero_()
        with torch.cuda.graph(g, stream=s):
            assert hip.mm_device(Segment.of(w), JAM.Q4_0, k, a.data_ptr(), k, c.data_ptr(), m, m, n, k) == JAM.OK
        # a larger split-K call grows the split scratch past the captured buffer
        abig = torch.from_numpy(oracle.normal(84, (7, 16384))).cuda()
        cbig = torch.zeros((7, 4096), dtype=torch.float32, device="cuda")
        for r in range(3):
            say(f"graph replay {r} after growth")
            with torch.cuda.stream(s):
                assert hip.mm_device(Segment.of(wbig), JAM.Q4_0, 16384, abig.data_ptr(), 16384, cbig.data_ptr(),
                                     4096, 4096, 7, 16384) == JAM.OK
            s.synchronize()
            c.fill_(-1.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(c, eager), r
        ref = oracle.mm_int8(O.Q4_0, w, a.cpu().numpy(), m, n, k)
        _, sa = oracle.mm_ref(O.Q4_0, w, a.cpu().numpy(), m, n, k)
        got = eager.cpu().numpy()
        assert (np.abs(got - ref) <= 1e-3 * np.abs(ref) + 1e-5 * sa).all()
    finally:
        hip.set_stream(None)
        hip.evict(Segment.of(w))
        hip.evict(Segment.of(wbig))


EXIT_SCRIPT = r"""
import sys, tempfile
from pathlib import Path
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
from oracle import oracle as O
from qxotic_amd import gguf as G
from qxotic_amd.jam import HipJAM, JAM, Segment
orc = O.Oracle()
hip = HipJAM(0)
glob = HipJAM.global_context()
w = orc.quantize(O.Q4_K, orc.normal(1, (64, 512), 0.0, 0.02))
path = Path(tempfile.mkdtemp()) / "m.gguf"
G.write(path, [("blk.0.ffn_up.weight", O.Q4_K, (512, 64), w)])
g = G.GGUF(path)
st, cnt, _ = g.pin(hip)
assert st == 0 and cnt == 1
st, cnt, _ = g.pin(glob)
assert st == 0 and cnt == 1
a = orc.normal(2, (3, 512))
c = np.zeros((3, 64), np.float32)
assert glob.mm(Segment.of(w), 0, JAM.Q4_K, 512, Segment.of(a), 0, JAM.F32, 512, Segment.of(c), 0, JAM.F32, 64, 64, 3, 512) == 0
print("left open", flush=True)
"""


def test_exit_with_open_contexts_and_mappings(tmp_path):
    """A process that exits with a context, the global context and a pinned GGUF mapping still open: the
    exit-time teardown releases them before the runtime finalizes, and the process ends with status 0."""
    script = tmp_path / "exit_open.py"
    script.write_text(EXIT_SCRIPT)
    say("exit with open contexts (subprocess)")
    r = subprocess.run([sys.executable, str(script), str(ROOT)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
    assert "left open" in r.stdout


def test_read_floor_entry_point(hip):
    """jamhip_read_floor (measurement aid) reads a device buffer and returns OK; unaligned sizes or addresses and
    null pointers are EINVAL, with the reason in the error text."""
    import torch
    from qxotic_amd.jam import JAM
    buf = torch.randint(0, 255, (1 << 20,), dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    assert hip.read_floor(buf.data_ptr(), buf.numel(), sink.data_ptr()) == JAM.OK, hip.last_error()
    assert hip.read_floor(buf.data_ptr(), 0, sink.data_ptr()) == JAM.OK
    assert hip.synchronize() == JAM.OK
    assert hip.read_floor(buf.data_ptr(), 1000, sink.data_ptr()) == JAM.EINVAL
    assert "aligned" in hip.last_error()
    assert hip.read_floor(buf.data_ptr() + 8, 1024, sink.data_ptr()) == JAM.EINVAL
    assert hip.read_floor(0, 1024, sink.data_ptr()) == JAM.EINVAL
    assert hip.read_floor(buf.data_ptr(), 1024, 0) == JAM.EINVAL
