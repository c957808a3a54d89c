"""mnemocuda_amd -- MI355X (gfx950) quantized-matmul hot path of MnemoCUDA.

The product is the C-ABI shared library ``libmnemo_hip.so`` (include/mnemo_kernels.h,
include/mnemo_host.h).  This package loads it with ctypes and exposes thin wrappers that
take torch tensors (torch is only the device-memory and stream plumbing).  There is no
fallback: if the library is missing or the device is not a GPU, calls raise.
"""
from __future__ import annotations

from .lib import LIB_PATH, load_library, MnemoError  # noqa: F401
from . import ops  # noqa: F401

__all__ = ["LIB_PATH", "load_library", "MnemoError", "ops"]
