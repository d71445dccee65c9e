"""The C-ABI library loads without a GPU, exports every entry point include/qe_kernels.h declares, and a
violated precondition aborts with the reference's "check failed" message before any GPU call. CPU only."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qe_kernels.h")
LIB = os.path.join(ROOT, "qengine_amd", "libqe_kernels.so")


def declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(qe_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_entry_points():
    names = declared()
    for must in ["qe_repack_w4", "qe_gemv_w4", "qe_gemv_w4g", "qe_skinny_w4", "qe_gemm_w4", "qe_gemm_w4_t",
                 "qe_gemm_w4_s", "qe_gemv_w4_s", "qe_gemm_set_out_bf16", "qe_quantize_w8", "qe_gemv_w8",
                 "qe_gemv_workspace_init"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build first: python -m qengine_amd.build"
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    lib.qe_abi_version.restype = ctypes.c_int
    assert lib.qe_abi_version() == 1


@pytest.mark.parametrize("call,msg", [
    ("lib.qe_repack_w4(None, None, 15, 128, None, None)", "repack_w4 15 128"),
    ("lib.qe_tile_w8(None, None, 16, 100, 1, None, None, None)", "tile_w8 16 100"),
    ("lib.qe_dequant_w4(None, None, 16, 64, 0, None, None)", "dequant_w4 16 64"),
    ("lib.qe_set_config(ctypes.byref((ctypes.c_int * 8)(2, 0, 5, 0, 0, 0, 0, 0)))", "batch_invariant 5"),
    ("lib.qe_set_config(ctypes.byref((ctypes.c_int * 8)(2, 0, 0, 0, 3, 0, 0, 0)))", "gemm_h16 3"),
    ("lib.qe_set_config(ctypes.byref((ctypes.c_int * 8)(2, 0, 0, 0, 0, 0, 7, 0)))", "reserved fields must be 0"),
    # the reduced-precision prefill paths check their shapes and the activation group on the host
    ("lib.qe_gemm_w4_i8_ex(None, None, 256, 512, None, 512, None, 256, 8, 48, 0, None)", "activation group G = 48"),
    ("lib.qe_gemm_w4h_ex(None, None, 250, 512, None, 512, None, 256, 8, 0, None)", "gemm_w4h: n = 250"),
    # the allocation-free MoE layer rejects a workspace above its scratch array before touching the GPU
    ("lib.qe_moe_w4_noalloc(None, None, None, 100000, 512, 10, 2048, 512, None, 0, None)",
     "qe_moe_w4_noalloc: T 100000"),
    # the H16 paths need the caller's XH workspace (reference tests/test_q8.py:62-67 passes it)
    ("lib.qe_gemv_q8(None, None, 64, 256, None, None, 1, 0, 1, None, None)", "h16 needs the XH workspace"),
    ("lib.qe_gemv_q8(None, None, 64, 256, None, None, 1, 0, 0, None, ctypes.c_void_p(64))", "output of the h16 path"),
    ("lib.qe_gemv_w4h(None, None, 64, 256, None, None, 1, 0, None, None)", "qe_gemv_w4h: needs the XH workspace"),
])
def test_precondition_aborts_with_check_message(call, msg):
    code = f"import ctypes; lib = ctypes.CDLL({LIB!r}); {call}"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "check failed" in r.stderr and msg in r.stderr, r.stderr


def test_skinny_declines_unsupported_rows():
    lib = ctypes.CDLL(LIB)
    lib.qe_skinny_w4.restype = ctypes.c_int
    assert lib.qe_skinny_w4(None, None, 16, 128, None, None, 17, 0) == 0
    assert lib.qe_skinny_w4(None, None, 16, 128, None, None, 0, 0) == 0
