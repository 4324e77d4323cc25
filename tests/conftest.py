import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402  (test infrastructure)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


def _ensure_oracle():
    if not O.ORACLE_SO.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "oracle"], check=True, capture_output=True)


@pytest.fixture(scope="session")
def oracle():
    _ensure_oracle()
    return O.Oracle()


@pytest.fixture(scope="session")
def refjam():
    if not O.ref_available():
        pytest.skip("oracle/_ref/libjam.so not built (reference sources absent when built)")
    r = O.RefJam(nthreads=4)
    yield r
    r.close()


@pytest.fixture(scope="session")
def refjam_generic():
    """libjam capped to its portable float floor (JAM_ISA_GENERIC): exact float dots of the dequantized
    weights (jam_kernels_generic.c:42-321)."""
    if not O.ref_available():
        pytest.skip("oracle/_ref/libjam.so not built")
    r = O.RefJam(nthreads=2, max_isa=1)
    yield r
    r.close()


@pytest.fixture(scope="session")
def hip():
    from qxotic_amd.jam import HipJAM
    h = HipJAM()
    yield h
    h.close()


def adversarial_activations(k: int = 256) -> np.ndarray:
    """Rows that stress the per-32 quantizers (jam_test.c:392-420, 355-390): zero block, all-equal,
    tiny scale, exact .5 ties at d=1, saturation, mixed signs, huge range."""
    rows = []
    z = np.zeros(k, np.float32)
    rows.append(z.copy())                                        # all zero -> d=0, q=0
    rows.append(np.full(k, 0.75, np.float32))                    # all equal -> +127
    rows.append(np.full(k, -3.0, np.float32))                    # all equal negative -> -127
    rows.append((np.arange(k) % 7 - 3).astype(np.float32) * 1e-6)   # tiny scale
    t = np.tile(np.array([127.0, 2.5, -2.5, 3.5, -0.5, 0.5, 1.5, -126.5] * 4, np.float32), k // 32)
    rows.append(t)                                               # amax 127 -> d = 1: exact .5 ties
    rows.append(np.tile(np.array([1e30, -1e30] + [1.0] * 30, np.float32), k // 32))   # huge dynamic range
    s = np.where(np.arange(k) % 2 == 0, 1.0, -1.0).astype(np.float32) * 1e4
    rows.append(s)                                               # saturation-scale magnitudes
    rng = np.random.default_rng(1234)
    rows.append(rng.standard_normal(k).astype(np.float32))
    return np.stack(rows)


def random_blocks(dt: int, rows: int, k: int, seed: int) -> np.ndarray:
    """[rows, row_bytes] uint8 of random but valid GGUF blocks (the reference's random-valid-block builders,
    jam/jam-native/tests/jam_ref.h:160-293): random quant bytes, block scales drawn so the decoded weights
    are of the N(0, 0.02) order. Much faster than quantizing f32 draws at 100M+ elements."""
    rng = np.random.default_rng(seed)
    be, bb = O.BLOCK[dt]
    nb = k // be
    blk = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)

    def f16(lo, hi, shape):
        return rng.uniform(lo, hi, shape).astype(np.float16).view(np.uint8).reshape(*shape, 2)

    if dt == O.Q8_0:
        blk[:, :, 0:2] = f16(1e-4, 3e-4, (rows, nb))
    elif dt == O.Q4_0:
        blk[:, :, 0:2] = f16(2e-3, 6e-3, (rows, nb))
    elif dt == O.MXFP4:
        blk[:, :, 0] = rng.integers(118, 123, (rows, nb), dtype=np.uint8)
    elif dt == O.Q4_K:
        blk[:, :, 0:2] = f16(5e-5, 2e-4, (rows, nb))      # d
        blk[:, :, 2:4] = f16(1e-4, 5e-4, (rows, nb))      # dmin
    elif dt == O.Q6_K:
        blk[:, :, 192:208] = rng.integers(-40, 41, (rows, nb, 16), dtype=np.int8).view(np.uint8)
        blk[:, :, 208:210] = f16(1e-5, 4e-5, (rows, nb))
    else:
        raise ValueError(dt)
    return np.ascontiguousarray(blk.reshape(rows, nb * bb))


def parity_report(label: str, got: np.ndarray, ref: np.ndarray, sa: np.ndarray) -> dict:
    """The largest relative error (over outputs with |ref| above 1e-3 of the largest) and the largest error
    in units of sum|w*a|, printed with the case's label; returns both."""
    err = np.abs(got.astype(np.float64) - ref)
    big = np.abs(ref) > 1e-3 * np.abs(ref).max()
    rel = float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    per_sa = float((err / np.maximum(sa, 1e-30)).max())
    print(f"parity {label}: max_rel {rel:.3e}  max_err/sumAbs {per_sa:.3e}  outputs {got.size}", file=sys.stderr,
          flush=True)
    out = {"max_rel": rel, "max_err_per_sumabs": per_sa}
    log = os.environ.get("JAM_PARITY_LOG")   # a JSON line per case, for the committed per-config summary
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"case": label, "outputs": int(got.size), **out}) + "\n")
    return out
