"""baracuda_amd -- MI355X (gfx950) quantized-inference contraction path.

Drop-in for baracuda's int8 / FP8 RCR GEMMs, the m=1 decode GEMVs,
gather_rows and a grouped int8 MoE GEMM, behind the reference's flat C ABI
(include/baracuda_kernels.h) and a mirror of its Plan surface (plans.py).
"""
from .ffi import LIB_PATH, SYMBOLS, lib  # noqa: F401

__all__ = ["LIB_PATH", "SYMBOLS", "lib"]
