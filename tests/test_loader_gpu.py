"""Quantized-matrix loader (qe_load_w4, the reference's Worker::load_w4, src/model.cpp:994-1059) on the GPU: the
device matrix equals, bit for bit, the oracle's repack of the same rows and columns taken from the source tensors
on the host (numpy slicing), for 4-bit (W4 layout, bf16 and fp16 scales) and 8-bit (Q8 layout) tensors, row ranges
of several tensors, a column slice, and the GLU interleave; and the loaded matrix multiplies like the repacked one."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from qengine_amd import ops, synth

pytestmark = pytest.mark.gpu


def source(n, k, bits, seed, scale_dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    q = rng.integers(-2**31, 2**31, size=(n, k * bits // 32), dtype=np.int64).astype(np.int32)
    s = torch.from_numpy(rng.random((n, k // 128)).astype(np.float32) * 0.01 + 0.001).to(scale_dtype)
    return q, s


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    d = {}
    src = {}
    for seed, (name, n, k, bits, sdt) in enumerate([("a", 64, 1024, 4, torch.bfloat16), ("b", 48, 1024, 4, torch.bfloat16),
                                  ("gate", 64, 512, 4, torch.float16), ("up", 64, 512, 4, torch.float16),
                                  ("q8", 32, 1024, 8, torch.bfloat16), ("q8g", 32, 512, 8, torch.bfloat16),
                                  ("q8u", 32, 512, 8, torch.bfloat16)]):
        q, s = source(n, k, bits, seed, sdt)
        d[name + ".weight_packed"] = torch.from_numpy(q)
        d[name + ".weight_scale"] = s
        src[name] = (q, s.view(torch.int16).numpy().view(np.uint16))
    path = tmp_path_factory.mktemp("st") / "model.safetensors"
    save_file(d, str(path))
    with ops.SafeTensorsFile(path) as f:
        yield f, src


def host_matrix(src, rows, c0, c1, bits):
    """the loader's input on the host: row ranges concatenated, columns [c0, c1)"""
    qs, ss = [], []  # columns c0..c1 are the int32 words c0 * bits / 32 .. c1 * bits / 32
    for name, r0, r1 in rows:
        q, s = src[name]
        qs.append(q[r0:r1, c0 * bits // 32:c1 * bits // 32])
        ss.append(s[r0:r1, c0 // 128:c1 // 128])
    return np.ascontiguousarray(np.concatenate(qs)), np.ascontiguousarray(np.concatenate(ss))


@pytest.mark.parametrize("rows,c0,c1", [
    ([("a", 0, 64)], -1, -1),
    ([("a", 16, 48), ("b", 0, 32)], 256, 768),
    ([("b", 16, 48)], 0, 128),
])
def test_load_w4_bit_exact(dev, model, rows, c0, c1):
    f, src = model
    w = f.load_w4(rows, c0, c1)
    torch.cuda.synchronize()
    K = src[rows[0][0]][1].shape[1] * 128
    lo, hi = (0, K) if c0 < 0 else (c0, c1)
    q, s = host_matrix(src, rows, lo, hi, 4)
    n, k = q.shape[0], hi - lo
    assert (w.n, w.k) == (n, k) and isinstance(w, ops.W4) and w.s.dtype == torch.bfloat16
    dq, ds = oracle.repack_w4(q, s, n, k)
    assert np.array_equal(w.q.cpu().numpy().view(np.uint32).reshape(-1), dq.reshape(-1))
    assert np.array_equal(synth.bits(w.s).reshape(-1), ds.reshape(-1))


def test_load_w4_glu_fp16_scales(dev, model):
    """gate rows then up rows, GLU-interleaved before the repack; fp16 scales stay fp16"""
    f, src = model
    w = f.load_w4([("gate", 0, 64), ("up", 0, 64)], glu=True)
    torch.cuda.synchronize()
    q, s = host_matrix(src, [("gate", 0, 64), ("up", 0, 64)], 0, 512, 4)
    gq, gs = oracle.glu_rows(q, s, 128, 512)
    dq, ds = oracle.repack_w4(gq, gs, 128, 512)
    assert w.glu and w.s.dtype == torch.float16
    assert np.array_equal(w.q.cpu().numpy().view(np.uint32).reshape(-1), dq.reshape(-1))
    assert np.array_equal(synth.bits(w.s).reshape(-1), ds.reshape(-1))
    # and it runs: the GLU decode GEMV of the loaded matrix equals that of the matrix repacked from the host arrays
    ref = ops.repack_w4(synth.to_dev(gq), synth.to_dev(gs, torch.float16), glu=True)
    x = synth.to_dev(synth.x_host(3, 512, seed=1))
    assert torch.equal(ops.gemv_w4(w, x).view(torch.int16), ops.gemv_w4(ref, x).view(torch.int16))


def test_load_q8_and_glu(dev, model):
    f, src = model
    w = f.load_w4([("q8", 0, 32)], 128, 896)
    torch.cuda.synchronize()
    q, s = host_matrix(src, [("q8", 0, 32)], 128, 896, 8)
    dq, ds = oracle.repack_q8(q, s, 32, 768)
    assert isinstance(w, ops.Q8) and (w.n, w.k) == (32, 768)
    assert np.array_equal(w.q.cpu().numpy().reshape(-1), dq.reshape(-1))
    assert np.array_equal(synth.bits(w.s).reshape(-1), ds.reshape(-1))
    g = f.load_w4([("q8g", 0, 32), ("q8u", 0, 32)], glu=True)
    torch.cuda.synchronize()
    q, s = host_matrix(src, [("q8g", 0, 32), ("q8u", 0, 32)], 0, 512, 8)
    gq, gs = oracle.glu_rows(q, s, 64, 512, bits=8)
    dq, ds = oracle.repack_q8(gq, gs, 64, 512)
    assert np.array_equal(g.q.cpu().numpy().reshape(-1), dq.reshape(-1))
    assert np.array_equal(synth.bits(g.s).reshape(-1), ds.reshape(-1))
