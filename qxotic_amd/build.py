"""Build libjamhip.so (gfx950) in-tree with hipcc: ``python -m qxotic_amd.build``.

Every translation unit is compiled for gfx950 only, with packed-FP32 instructions disabled; the
activation quantizers, the MoE routing (top-k weights) and the gated activations additionally compile with
-ffp-contract=off so their f32 products round exactly where jam's and jinfer's do (a product is never fused
into a following add unless the reference writes an fma).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libjamhip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
UNITS = {   # source -> extra flags
    "prep.hip": ["-ffp-contract=off"],
    "gemv.hip": [],
    "gemv_q4k.hip": [],
    "gemv_q6k.hip": [],
    "gemv_q80.hip": [],
    "gemv_q40.hip": [],
    "gemv_mxfp4.hip": [],
    "gemv_q5k.hip": [],
    "gemv_nvfp4.hip": [],
    "gemv_q10.hip": [],
    "dense.hip": [],
    "gemm.hip": [],
    "mma.hip": [],
    "mxn.hip": [],
    "moe.hip": ["-ffp-contract=off"],
    "epilogue.hip": ["-ffp-contract=off"],
    "readfloor.hip": [],
    "jamhip.cpp": ["-x", "hip"],
    "gguf.cpp": [],
}


def _compile(src: str, extra: list[str]) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return out


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(os.cpu_count() or 8, len(UNITS), 16)) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), UNITS.items()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
