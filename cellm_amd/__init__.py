"""cellm_amd: MI355X-native (gfx950) quantized-weight matmul path for cellm.

The product is libcellm_hip.so (HIP kernels + the C ABI in include/cellm_hip.h);
this package binds it with ctypes (`HipOps`, the MetalOps mirror) and builds it
(`cellm_amd.build`).
"""
from ._lib import CellmHipError, LIB_PATH, load  # noqa: F401
from .hipops import HipOps, device_count, smoke_test  # noqa: F401

__all__ = ["HipOps", "CellmHipError", "device_count", "smoke_test", "load", "LIB_PATH"]
