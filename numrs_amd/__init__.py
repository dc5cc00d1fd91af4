"""numrs_amd -- MI355X (gfx950) backend for numrs's reverse-mode autograd hot path.

Layers:
  include/numrs_hip.h     the C ABI (device pointers, int status codes)
  numrs_amd/csrc/*.hip    hand-written HIP kernels behind it
  numrs_amd.device        Context / DeviceArray over the C ABI (ctypes)
  numrs_amd.autograd      numrs's Tensor / backward on the device (tensor engine)
  numrs_amd.nn, .optim    Linear/ReLU/Sequential/..., SGD/Adam
  numrs_amd.graph         StepGraph: one training step recorded once, replayed per step
"""
from ._lib import LIB_PATH, LibraryMissing, header_functions, load  # noqa: F401
from .autograd import (Tensor, default_context, is_grad_enabled, no_grad,  # noqa: F401
                       set_default_context, set_grad_enabled, set_unbroadcast_mode)
from .device import Context, DeviceArray, HipError  # noqa: F401
from . import checkpoint, nn, optim  # noqa: F401,E402
from .graph import StepGraph  # noqa: F401,E402

__all__ = ["Context", "DeviceArray", "HipError", "LibraryMissing", "load", "header_functions",
           "LIB_PATH", "Tensor", "no_grad", "is_grad_enabled", "set_grad_enabled",
           "set_unbroadcast_mode", "default_context", "set_default_context", "nn", "optim",
           "StepGraph"]
