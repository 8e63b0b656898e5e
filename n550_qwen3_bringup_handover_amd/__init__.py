"""MI355X-native GEMM/GEMV hot path for the Qwen3-0.6B bare-metal C runtime.

The product is libqwen3_hip.so (C ABI: include/qwen3_hip.h), a drop-in for
the runtime's GEMM plug-in.  This package only builds and loads it:
`runtime` (build + ctypes loader) and `abi` (numpy-friendly mirror of the C
entry points).
"""
from . import runtime  # noqa: F401

__all__ = ["runtime"]
