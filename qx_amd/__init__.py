"""qx_amd -- MI355X (gfx950) grouped-query-attention path of blasrodri/qx.

The product is libqx_hip.so (hand-written HIP kernels behind the C ABI in
include/qx_hip.h).  This package holds its sources (csrc/), its build recipe
(build.py), ctypes bindings (abi.py), a Python mirror of the reference
interface (runtime.py, api.py).  There is no CPU fallback: using the package
without the built library raises.
"""
from .abi import BF16, F16, F32, SHAPE_GRANITE, SHAPE_QWEN3, QxhError, lib  # noqa: F401

__all__ = ["lib", "QxhError", "F32", "F16", "BF16", "SHAPE_GRANITE", "SHAPE_QWEN3"]
