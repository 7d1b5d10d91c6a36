"""zigneuron_amd -- MI355X (gfx950) fp32 GEMM backend for ZigNeuron.

The product is the C-ABI library ``lib/libzn_hip.so`` (include/zn_hip.h) and
its offline-built gfx950 code objects; this package is the host-side mirror
of the reference ``Backend``/``Dense`` interfaces over that ABI.
"""
from ._lib import (ZnError, NoDeviceError, CodeObjectError, SymbolError, InvalidArgumentError,  # noqa: F401
                   OutOfMemoryError, LaunchError, HipError)
from .backend import Backend, Context, DeviceBuffer, available  # noqa: F401
from .layer import Dense, DenseDevice, pair_backward, pair_forward  # noqa: F401

__all__ = ["Backend", "Context", "DeviceBuffer", "Dense", "DenseDevice", "pair_forward", "pair_backward", "available", "ZnError",
           "NoDeviceError", "CodeObjectError", "SymbolError", "InvalidArgumentError", "OutOfMemoryError",
           "LaunchError", "HipError"]
