"""On-disk weights (qengine_amd/csrc/loader.cpp) on the CPU: the .safetensors reader against files written by the
safetensors package (the format's own writer) and against hand-built headers, and the matrix dimensions of the
quantized-matrix loader (the reference's Worker::load_w4 rules, src/model.cpp:994-1009: bits from the packed width,
row ranges concatenated, column slices on 128-k groups). The device side (copy, GLU interleave, repack) is
tests/test_loader_gpu.py."""
import ctypes
import json
import struct
import subprocess
import sys

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from qengine_amd import ops
from qengine_amd.qe import LIB_PATH


def ct_tensors(prefix, n, k, bits, seed, scale_dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.integers(-2**31, 2**31, size=(n, k * bits // 32), dtype=np.int64).astype(np.int32))
    s = (torch.from_numpy(rng.random((n, k // 128)).astype(np.float32)) * 0.01 + 0.001).to(scale_dtype)
    return {prefix + ".weight_packed": q, prefix + ".weight_scale": s}


@pytest.fixture
def st_file(tmp_path):
    t = {}
    t.update(ct_tensors("model.layers.0.mlp.gate_proj", 64, 512, 4, 1))
    t.update(ct_tensors("model.layers.0.mlp.up_proj", 64, 512, 4, 2))
    t.update(ct_tensors("model.layers.0.mlp.down_proj", 48, 1024, 8, 3))
    t.update(ct_tensors("experts.0.gate_up", 32, 256, 4, 4, torch.float16))
    t["norm.weight"] = torch.arange(96, dtype=torch.float32).reshape(2, 48)
    t["bias"] = torch.arange(5, dtype=torch.int64)
    path = tmp_path / "model.safetensors"
    save_file(t, str(path), metadata={"format": "pt", "note": "quote \" and \\u00e9 in metadata"})
    return path, t


def test_reader_matches_writer(st_file):
    path, t = st_file
    with ops.SafeTensorsFile(path) as f:
        assert f.names() == sorted(t)
        for name, ten in t.items():
            dt, shape, nb, addr = f.info(name)
            assert shape == tuple(ten.shape) and nb == ten.numel() * ten.element_size()
            want = {torch.int32: "I32", torch.bfloat16: "BF16", torch.float16: "F16", torch.float32: "F32",
                    torch.int64: "I64"}[ten.dtype]
            assert dt == want
            got = np.ctypeslib.as_array((ctypes.c_uint8 * nb).from_address(addr))
            assert np.array_equal(got, ten.contiguous().view(torch.uint8).numpy().reshape(-1))
        assert f.info("no.such.tensor") is None


def handmade(tmp_path, header, data, name="h.safetensors", pad=True):
    hb = header.encode() if isinstance(header, str) else header
    if pad:
        hb += b" " * ((8 - len(hb) % 8) % 8)
    p = tmp_path / name
    p.write_bytes(struct.pack("<Q", len(hb)) + hb + data)
    return p


def test_header_parser_on_handmade_json(tmp_path):
    """whitespace, escapes (\\u0041 = 'A', \\" and \\\\ in names), nested metadata, an empty shape (a scalar)"""
    hdr = ('{\n "\\u0041.w" : {"dtype":"U8","shape":[ 2 , 3 ],"data_offsets":[0,6]},\t"q\\"x\\\\y": {"dtype": "F32", '
           '"shape": [], "data_offsets": [6, 10]}, "__metadata__": {"a": "b", "n": {"x": [1, 2, true, null]}}}')
    p = handmade(tmp_path, hdr, bytes(range(6)) + struct.pack("<f", 2.5))
    assert json.loads(hdr)  # the header is valid JSON
    with ops.SafeTensorsFile(p) as f:
        assert f.names() == ["A.w", 'q"x\\y']
        dt, shape, nb, addr = f.info("A.w")
        assert (dt, shape, nb) == ("U8", (2, 3), 6)
        assert bytes((ctypes.c_uint8 * 6).from_address(addr)) == bytes(range(6))
        dt, shape, nb, addr = f.info('q"x\\y')
        assert (dt, shape, nb) == ("F32", (), 4) and ctypes.c_float.from_address(addr).value == 2.5


@pytest.mark.parametrize("header,data,msg", [
    ('{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}', bytes(16), "data_offsets"),
    ('{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}', bytes(8), "data_offsets"),
    ('{"a": {"dtype": "Q7", "shape": [4], "data_offsets": [0, 4]}}', bytes(4), "unknown dtype"),
    ('{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}', bytes(4), "JSON header"),
    ('{"a": {"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}}', bytes(4), "non-integer"),
    ('{"a": {"dtype": "F32", "shape": [1]}}', bytes(4), "malformed entry"),
    # dims whose product wraps past 64 bits (2^36 * 2^32) to 0 elements, with empty data_offsets
    ('{"q": {"dtype": "I32", "shape": [68719476736, 4294967296], "data_offsets": [0, 0]}}', bytes(8), "overflows"),
    # no wrap of the count, but of the byte size (2^39 * 2^24 elements of 4 bytes = 2^65)
    ('{"q": {"dtype": "F32", "shape": [549755813888, 16777216], "data_offsets": [0, 8]}}', bytes(8), "byte size"),
    # no wrap, more bytes than the file holds (2^39 * 2^20 fp32)
    ('{"q": {"dtype": "F32", "shape": [549755813888, 1048576], "data_offsets": [0, 8]}}', bytes(8), "data_offsets"),
])
def test_malformed_files_abort_with_message(tmp_path, header, data, msg):
    p = handmade(tmp_path, header, data)
    code = f"import ctypes; lib = ctypes.CDLL({LIB_PATH!r}); lib.qe_st_open({str(p)!r}.encode())"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "check failed" in r.stderr and msg in r.stderr, r.stderr


def test_header_length_beyond_file_aborts(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 20) + b"{}")
    code = f"import ctypes; lib = ctypes.CDLL({LIB_PATH!r}); lib.qe_st_open({str(p)!r}.encode())"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "header length" in r.stderr


def test_load_w4_dims(st_file):
    path, _ = st_file
    g, u, d = "model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj", "model.layers.0.mlp.down_proj"
    with ops.SafeTensorsFile(path) as f:
        assert f.w4_dims([(g, 0, 64)]) == (64, 512, 4, 0)
        assert f.w4_dims([(g, 16, 48), (u, 0, 32)], 128, 384) == (64, 256, 4, 0)  # row ranges + a column slice
        assert f.w4_dims([(d, 0, 48)]) == (48, 1024, 8, 0)                         # 8-bit: Q8
        assert f.w4_dims([("experts.0.gate_up", 0, 32)]) == (32, 256, 4, 1)       # fp16 scales


@pytest.mark.parametrize("rows,c0,c1,msg", [
    ([("model.layers.0.mlp.gate_proj", 0, 40)], -1, -1, "multiple of 16"),
    ([("model.layers.0.mlp.gate_proj", 0, 70)], -1, -1, "rows [0, 70)"),
    ([("model.layers.0.mlp.gate_proj", 0, 64)], 64, 256, "columns"),
    ([("model.layers.0.mlp.gate_proj", 0, 32), ("model.layers.0.mlp.down_proj", 0, 32)], -1, -1, "differ"),
    ([("model.layers.0.mlp.nothing", 0, 32)], -1, -1, "has no tensor"),
    ([("norm", 0, 2)], -1, -1, "has no tensor"),
])
def test_load_w4_dims_rejects(st_file, rows, c0, c1, msg):
    path, _ = st_file
    names = ", ".join(f"({r[0]!r}, {r[1]}, {r[2]})" for r in rows)
    code = (f"import sys; sys.path.insert(0, {str(__import__('os').path.dirname(__import__('os').path.dirname(__file__)))!r})\n"
            f"from qengine_amd import ops\nf = ops.SafeTensorsFile({str(path)!r})\nf.w4_dims([{names}], {c0}, {c1})\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "check failed" in r.stderr and msg in r.stderr, r.stderr
