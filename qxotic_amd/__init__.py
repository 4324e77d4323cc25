"""MI355X (gfx950) backend for jam's quantized matmul R = W @ A^T.

``qxotic_amd.jam`` mirrors jam's backend SPI over the C-ABI in ``include/jamhip.h``; the kernels are
hand-written HIP in ``qxotic_amd/csrc``. Build with ``python -m qxotic_amd.build``.
"""
from .ggml import BY_CODE, BY_NAME, GGMLType, by_code  # noqa: F401

__all__ = ["BY_CODE", "BY_NAME", "GGMLType", "by_code"]
