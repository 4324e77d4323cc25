"""Write tests/golden/jam_golden.npz from the reference's own libjam (oracle/_ref/libjam.so, compiled
from jam/jam-native/src by oracle/Makefile). Run in the build container:

    make -C oracle && python tests/golden/gen_golden.py

Contents (all inputs are stored next to the outputs, so the fixture is self-contained):
  act                 seeded + adversarial f32 activation rows, k = 256
  f1_q/f1_d/f1_s      jam_q8_0_requant on every row      (jam_kernels_generic.c:71-94)
  f2_q/f2_d/f2_s      jam_q4k_quant on every row          (jam_kernels_q4k_avx512.c:25-47)
  mm_<DT>_w           weight bytes [m, row_bytes], m = 32, k = 512
  mm_a                f32 activations [16, 512]
  mm_<DT>_n<N>        jam_mm output [N, 32] on the avx512_vnni context for N in {1, 3, 7, 8, 13, 16}
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from conftest import adversarial_activations  # noqa: E402
from oracle import oracle as O  # noqa: E402

NS = (1, 3, 7, 8, 13, 16)


def main() -> None:
    ref = O.RefJam(nthreads=4)
    if ref.active_isa() != O.JAM_ISA_AVX512_VNNI:
        raise SystemExit("golden vectors are taken on an avx512_vnni context")
    orc = O.Oracle()
    rng = np.random.default_rng(0x5A11C0DE)
    act = np.concatenate([adversarial_activations(256), rng.standard_normal((8, 256)).astype(np.float32) * 3])
    out = {"act": act}
    out["f1_q"], out["f1_d"], out["f1_s"] = ref.quant_f1(act)
    out["f2_q"], out["f2_d"], out["f2_s"] = ref.quant_f2(act)
    m, k = 32, 512
    a = orc.normal(0x5A11C0DE ^ 7, (16, k))
    out["mm_a"] = a
    for dt in O.QUANT_TYPES:
        w = orc.quantize(dt, orc.normal(0x5A11C0DE ^ dt, (m, k), 0.0, 0.02))
        out[f"mm_{O.NAMES[dt]}_w"] = w
        for n in NS:
            out[f"mm_{O.NAMES[dt]}_n{n}"] = ref.mm(dt, w, a[:n], m, n, k).copy()
    ref.close()
    path = Path(__file__).resolve().parent / "jam_golden.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
