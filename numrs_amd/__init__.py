"""numrs_amd -- MI355X (gfx950) backend for numrs's reverse-mode autograd hot path.

Layers:
  include/numrs_hip.h     the C ABI (device pointers, int status codes)
  numrs_amd/csrc/*.hip    hand-written HIP kernels behind it
  numrs_amd.device        Context / DeviceArray over the C ABI (ctypes)
"""
from ._lib import LIB_PATH, LibraryMissing, header_functions, load  # noqa: F401
from .device import Context, DeviceArray, HipError  # noqa: F401

__all__ = ["Context", "DeviceArray", "HipError", "LibraryMissing", "load", "header_functions",
           "LIB_PATH"]
