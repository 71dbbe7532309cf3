"""onnx_amd -- MI355X (gfx950) device path for the Lokad.Onnx elementwise,
broadcast and reduction operators.

The compute lives in liblonnx_hip.so (hand-written HIP kernels behind the C ABI
of include/lonnx.h); this package is its Python binding and the
HipExecutionProvider twin of the reference's CPUExecutionProvider.
"""
from ._lib import LIB_PATH, lib, plan_broadcast  # noqa: F401
from .provider import (DeviceTensor, HipExecutionProvider, OpResult, OpStatus, init,  # noqa: F401
                       set_stream, synchronize)

__all__ = ["DeviceTensor", "HipExecutionProvider", "OpResult", "OpStatus", "init", "set_stream", "synchronize",
           "plan_broadcast", "lib", "LIB_PATH"]
