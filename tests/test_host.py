"""CPU-only checks of the boundary: the C-ABI library loads and exports every entry point its header
declares; argument handling of the JAM mirror (NativeJAM.java:63-152, JAM.java:52-71); GGUF geometry
and the synthetic-weight quantizers."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "jamhip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jamhip_[a-z_]+)\s*\(", text)))


def test_library_exports_header():
    from qxotic_amd._lib import LIB_PATH, SIGNATURES, lib
    L = lib()
    names = header_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(L, name), name
    assert sorted(n for n, _, _ in SIGNATURES) == names
    assert LIB_PATH.exists()


def test_null_context_and_no_device_paths():
    from qxotic_amd._lib import lib
    L = lib()
    assert L.jamhip_mm(None, None, 8, 32, None, 0, 32, None, 0, 32, 1, 1, 32) == 1   # EINVAL
    assert L.jamhip_weight_pin(None, None, 8, 32, 1) == 1
    assert L.jamhip_ctx_synchronize(None) == 1
    assert isinstance(L.jamhip_last_error(None), bytes)


def test_device_disable_env(monkeypatch):
    from qxotic_amd._lib import lib
    monkeypatch.setenv("JAM_HIP_DISABLE", "1")
    assert lib().jamhip_device_available() == 0
    assert not lib().jamhip_ctx_create(0)


def _bare_backend():
    from qxotic_amd.jam import HipJAM
    h = object.__new__(HipJAM)   # argument checks run before any native call
    h._ctx = None
    h._global = False
    h._closed = False
    h._serial = True
    h._lock = None
    h.fallback = None
    return h


def test_mirror_rejects_heap_and_undersized_segments():
    from qxotic_amd.jam import JAM, IllegalArgumentError, IndexOutOfBoundsError, Segment
    h = _bare_backend()
    w = np.zeros((4, 34), np.uint8)
    a = np.zeros((2, 32), np.float32)
    r = np.zeros((2, 4), np.float32)
    with pytest.raises(IllegalArgumentError):
        h.mm(Segment.heap(w), 0, JAM.Q8_0, 32, Segment.of(a), 0, JAM.F32, 32, Segment.of(r), 0, JAM.F32, 4, 4, 2, 32)
    with pytest.raises(IndexOutOfBoundsError):   # 5 rows of Q8_0 need 170 B, segment has 136
        h.mm(Segment.of(w), 0, JAM.Q8_0, 32, Segment.of(a), 0, JAM.F32, 32, Segment.of(r), 0, JAM.F32, 5, 5, 2, 32)
    with pytest.raises(IndexOutOfBoundsError):   # offset pushes A past its end
        h.mm(Segment.of(w), 0, JAM.Q8_0, 32, Segment.of(a), 4, JAM.F32, 32, Segment.of(r), 0, JAM.F32, 4, 4, 2, 32)
    with pytest.raises(IndexOutOfBoundsError):   # R is n x ldr floats
        h.mm(Segment.of(w), 0, JAM.Q8_0, 32, Segment.of(a), 0, JAM.F32, 32, Segment.of(r), 0, JAM.F32, 5, 4, 2, 32)


def test_providers_disable_before_probe(monkeypatch):
    from qxotic_amd.jam import providers

    class Fake:
        probed = 0

        def __init__(self, pid, prio, ok=True):
            self.pid, self.prio, self.ok = pid, prio, ok

        def id(self):
            return self.pid

        def priority(self):
            return self.prio

        def is_available(self):
            Fake.probed += 1
            if self.ok == "raise":
                raise RuntimeError("probe failure")
            return self.ok

    ps = [Fake("a", 1), Fake("b", 5), Fake("c", 3, ok=False), Fake("d", 9, ok="raise")]
    assert [p.id() for p in providers(ps)] == ["b", "a"]
    Fake.probed = 0
    monkeypatch.setenv("JAM_B_DISABLED", "true")
    assert [p.id() for p in providers(ps)] == ["a"]
    assert Fake.probed == 3   # the disabled provider was never probed


def test_geometry_and_quantizers_match_oracle(oracle):
    from qxotic_amd import ggml
    assert ggml.by_code(12).span_bytes(3, 512, 256) == 2 * 288 + 144
    for dt in O.QUANT_TYPES:
        x = oracle.normal(123 + dt, (40, 512), 0.0, 0.02)
        assert np.array_equal(ggml.quantize(O.NAMES[dt], x), oracle.quantize(dt, x)), O.NAMES[dt]


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 (or a multi-rank launch) exits 2 with a message, before
    touching any device."""
    import os
    import subprocess
    import sys
    bench = ROOT / "bench.py"
    for argv, env in ((["--gpus", "2"], {}), (["--gpus", "1"], {"WORLD_SIZE": "2"})):
        r = subprocess.run([sys.executable, str(bench), *argv], capture_output=True, text=True, timeout=120,
                           env={**os.environ, **env})
        assert r.returncode == 2, (argv, env, r.stderr[-400:])
        assert "one GPU" in r.stderr and r.stdout == ""


def test_provider_delegates_unsupported_to_shadowed(monkeypatch):
    """Answering to id `native` hides jam-native from MatMul.load("native") (MatMul.java:1833-1844); the
    provider therefore hands every call the GPU answers with EUNSUPPORTED to the provider it shadows (the
    next available provider with the same id) and returns that provider's status. A provider of another id
    is never used as the fallback."""
    from qxotic_amd import jam as J

    calls = []

    class FakeNativeJAM:
        def mm(self, *args):
            calls.append(args[2])   # wt
            return J.JAM.OK

    class FakeProvider:
        def __init__(self, pid, prio):
            self.pid, self.prio = pid, prio

        def id(self):
            return self.pid

        def priority(self):
            return self.prio

        def is_available(self):
            return True

        def create(self):
            return FakeNativeJAM()

    monkeypatch.setattr(J, "_REGISTERED", [FakeProvider("vector", 500), FakeProvider("native", 1000)])
    monkeypatch.setattr(J, "_SHARED", None)
    statuses = iter([J.JAM.EUNSUPPORTED, J.JAM.OK, J.JAM.EINVAL])
    monkeypatch.setattr(J.HipJAM, "_native_mm", staticmethod(lambda args: next(statuses)))
    jam = J.Provider().create()
    assert isinstance(jam.fallback, FakeNativeJAM)
    w = np.zeros((4, 176), np.uint8)
    a = np.zeros((1, 256), np.float32)
    r = np.zeros((1, 4), np.float32)
    args = (J.Segment.of(w), 0, J.JAM.Q5_K, 256, J.Segment.of(a), 0, J.JAM.F32, 256, J.Segment.of(r), 0, J.JAM.F32,
            4, 4, 1, 256)
    assert jam.mm(*args) == J.JAM.OK and calls == [J.JAM.Q5_K]     # EUNSUPPORTED -> jam-native ran it
    assert jam.mm(*args) == J.JAM.OK and calls == [J.JAM.Q5_K]     # the GPU ran it
    assert jam.mm(*args) == J.JAM.EINVAL and len(calls) == 1       # only EUNSUPPORTED is delegated
    monkeypatch.setenv("JAM_HIP_ID", "hip")                          # own id: nothing to shadow
    assert J.Provider().shadowed() is None


def test_exit_teardown_runs_without_a_device(tmp_path):
    """The exit-time teardown (qxotic_amd._lib.on_exit) closes open GGUF mappings and the backend objects and
    calls jamhip_global_destroy; a process that leaves them open exits with status 0."""
    import subprocess
    import sys
    from qxotic_amd import gguf as G
    path = tmp_path / "m.gguf"
    G.write(path, [("w", 8, (32, 2), np.zeros(68, np.uint8))])
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from qxotic_amd import gguf as G, _lib\n"
            "from qxotic_amd.jam import HipJAM\n"
            "import atexit\n"
            "atexit.register(lambda: print('closed', g._h is None, h._closed, flush=True))  # runs after on_exit\n"
            "g = G.GGUF(%r); h = HipJAM.global_context()\n") % (str(ROOT), str(path))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-1000:]
    assert "closed True True" in r.stdout
