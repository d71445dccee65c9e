"""qengine_amd - MI355X-native (gfx950) weight-only quantized matmul path of QEngine.

The product is libqe_kernels.so (C-ABI in include/qe_kernels.h, HIP kernels in qengine_amd/csrc). This package
is the host-side mirror of the reference's ctypes test binding (reference tests/qe.py) plus typed torch
wrappers; torch provides device memory and streams only.
"""
from .qe import LIB_PATH, call, lib, sync  # noqa: F401
from . import ops  # noqa: F401
