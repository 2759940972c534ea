"""acfun_amd -- Acfun's convolution/GEMM path on one AMD Instinct MI355X (gfx950).

The product is the C-ABI library libacfun_amd.so (include/acfun/acfun.h),
host C++ over hand-written HIP kernels.  This package holds its sources
(csrc/), the ctypes binding (capi.py) and the ACFUN0 model writer (acfun0.py).
"""
from .capi import LIB_PATH, SIGNATURES, bind, last_error, lib  # noqa: F401

__all__ = ["LIB_PATH", "SIGNATURES", "bind", "last_error", "lib"]
