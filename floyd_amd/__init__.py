"""floyd_amd -- MI355X-native quantized Moonlight hot path (HIP / gfx950).

The product is the C-ABI shared library floyd_amd/lib/libfloyd_amd.so
(declared in include/moonlight_hip.h, include/fm_backend.h and
include/moonlight_kernels.h).  This package only loads it and wraps the
kernel-level entry points for Python callers (tests, bench).  There is no
CPU fallback: loading fails loudly when the library is missing.
"""
from . import native  # noqa: F401
from .native import (  # noqa: F401
    LIBRARY_PATH, DeviceBuffer, MLK_F32, MLK_Q4, MLK_Q8, NativeError, load)

__all__ = ["native", "load", "DeviceBuffer", "NativeError", "LIBRARY_PATH",
           "MLK_F32", "MLK_Q8", "MLK_Q4"]
