"""strixite_amd: the quantized MoE FFN path of strixite, rebuilt for MI355X (gfx950, CDNA4, wave64).

The product is the C-ABI shared library libstrixite_moe.so (include/strixite_moe.h, include/strixite_moe.hpp);
``strixite_amd.moe`` mirrors the reference's launch interface over it on torch device tensors.
"""
from ._lib import GpuError, StrixError, lib  # noqa: F401
from . import moe  # noqa: F401

__all__ = ["lib", "moe", "StrixError", "GpuError"]
