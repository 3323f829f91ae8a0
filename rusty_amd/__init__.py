"""rusty_amd: Rusty's int8 quantized-linear hot path, MI355X-native (gfx950).

The compute lives in ``librusty_hip.so`` (hand-written HIP kernels behind the C
ABI of ``include/rusty_hip.h``); this package is its host-side mirror of the
reference's ``ComputeEngine`` surface.
"""
from ._lib import RqError, header_symbols, lib  # noqa: F401
from .engine import ComputeEngine, Context, DType, QuantizedTensor, UnifiedTensor, WgpuContext  # noqa: F401

__all__ = ["ComputeEngine", "Context", "DType", "QuantizedTensor", "RqError", "UnifiedTensor", "WgpuContext",
           "header_symbols", "lib"]
