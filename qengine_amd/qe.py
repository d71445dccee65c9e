"""ctypes binding of libqe_kernels.so, the counterpart of the reference's tests/qe.py (pass torch tensors).

`call(name, *args)` converts tensors to their data pointers, ints to c_int (c_longlong beyond 32 bits) and
floats to c_float, exactly as the reference binding does (reference tests/qe.py:14-25). The library is loaded
after torch so that both share one HIP runtime (same SONAME). A missing library is an error: there is no
fallback path.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime first)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QE_LIB") or os.path.join(HERE, "libqe_kernels.so")

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m qengine_amd.build` "
                               "(there is no fallback path)")
        _LIB = ctypes.CDLL(LIB_PATH)
        _LIB.qe_skinny_w4.restype = ctypes.c_int
        _LIB.qe_gemv_w4hxx.restype = ctypes.c_int
        _LIB.qe_abi_version.restype = ctypes.c_int
        _LIB.qe_clock_probe_mhz.restype = ctypes.c_float
    return _LIB


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _conv(a):
    if isinstance(a, torch.Tensor):
        return _p(a)
    if isinstance(a, bool):
        return ctypes.c_int(int(a))
    if isinstance(a, float):
        return ctypes.c_float(a)
    if isinstance(a, int):
        return ctypes.c_longlong(a) if abs(a) > 2**31 - 1 else ctypes.c_int(a)
    if a is None:
        return ctypes.c_void_p(0)
    return a


def call(name, *args):
    return getattr(lib(), name)(*[_conv(a) for a in args])


def sync():
    torch.cuda.synchronize()
