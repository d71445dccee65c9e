"""Q8 layer weights (reference src/kernels/q8_layout.h, hooks src/capi.cpp:19-45) through the reference-named C-ABI
vs the CPU oracle: repack bit-exact, GEMV / GEMM within the BASELINE gate, plus the kernels' own arithmetic: the
GEMV multiplies the exact int8 weights (scales applied per group in fp32) -> 1e-4 * rms of the exact product; the
GEMM multiplies bf16_rn(w * s) tiles -> 1e-4 * rms of the matmul on the oracle's bf16 dequantization."""
import numpy as np
import pytest
import torch

import oracle
from qengine_amd import ops, synth
from test_gemv_gpu import assert_bf16_close, assert_glu_close, err_ratio, glu_act, matmul_f64

pytestmark = pytest.mark.gpu


def q8_host(n, k, seed):
    """compressed-tensors 8-bit source: int32 [n][k/4] with bytes u = w + 128, w uniform in [-127, 127]; bf16 scales
    |N(0,1)| * 0.005 per (row, 128-k group)"""
    rng = np.random.default_rng(seed)
    w = rng.integers(-127, 128, size=(n, k)).astype(np.int64)
    u = (w + 128).astype(np.uint32).reshape(n, k // 4, 4)
    q = (u[..., 0] | (u[..., 1] << 8) | (u[..., 2] << 16) | (u[..., 3] << 24)).view(np.int32)
    s = synth.np_bf16((np.abs(rng.standard_normal((n, k // 128))) * 0.005).astype(np.float32))
    return q, s, w


def exact_q8(w, s):
    return w.astype(np.float64) * np.repeat(oracle.bf16_to_f32(s).astype(np.float64), 128, axis=1)


def test_repack_q8_bit_exact(dev):
    n, k = 96, 512
    q, s, _ = q8_host(n, k, 1)
    w = ops.repack_q8(synth.to_dev(q), synth.to_dev(s))
    torch.cuda.synchronize()
    dq, ds = oracle.repack_q8(q, s, n, k)
    assert np.array_equal(w.q.cpu().numpy(), dq)
    assert np.array_equal(synth.bits(w.s), ds)


def test_glu_rows8_bit_exact(dev):
    n, k = 64, 256
    q, s, _ = q8_host(n, k, 2)
    dq, ds = ops.glu_rows(synth.to_dev(q), synth.to_dev(s), bits=8)
    torch.cuda.synchronize()
    rq, rs = oracle.glu_rows(q, s, n, k, bits=8)
    assert np.array_equal(dq.cpu().numpy(), rq) and np.array_equal(synth.bits(ds), rs)


@pytest.mark.parametrize("n,k", [(64, 256), (1024, 2048), (2048, 5120)])
def test_gemv_q8_parity(dev, n, k):
    q, s, w = q8_host(n, k, n + k)
    wq = ops.repack_q8(synth.to_dev(q), synth.to_dev(s))
    xh = synth.x_host(20, k, seed=k)
    ref_ex = matmul_f64(xh, exact_q8(w, s))
    ref = matmul_f64(xh, oracle.bf16_to_f32(oracle.dequant_q8(q, s, n, k)))
    for m in (1, 3, 16, 20):
        y = ops.gemv_q8(wq, synth.to_dev(xh[:m]))
        torch.cuda.synchronize()
        yv = y.cpu().numpy()
        assert_bf16_close(yv, ref[:m])
        assert err_ratio(yv, ref_ex[:m]) <= 1e-4, m


def test_gemv_q8_glu(dev):
    n, k = 256, 1024
    q, s, w = q8_host(n, k, 5)
    wq = ops.repack_q8(synth.to_dev(q), synth.to_dev(s), glu=True)
    xh = synth.x_host(4, k, seed=6)
    y = ops.gemv_q8(wq, synth.to_dev(xh))
    torch.cuda.synchronize()
    gq, gs = oracle.glu_rows(q, s, n, k, bits=8)
    # the GLU rows of the exact weights: rows follow the interleave applied to the source
    wg = np.empty_like(w)
    for dr in range(n):
        t, j = dr // 16, dr % 16
        wg[dr] = w[8 * t + j if j < 8 else n // 2 + 8 * t + (j - 8)]
    act = glu_act(matmul_f64(xh, exact_q8(wg, gs)))
    assert_glu_close(oracle.bf16_to_f32(synth.bits(y)), act, 1e-4)


@pytest.mark.parametrize("n,k,t", [(256, 512, 33), (1024, 2048, 300)])
def test_gemm_q8_parity(dev, n, k, t):
    q, s, _ = q8_host(n, k, 7 + t)
    wq = ops.repack_q8(synth.to_dev(q), synth.to_dev(s))
    xh = synth.x_host(t, k, seed=8)
    y = ops.gemm_q8(wq, synth.to_dev(xh))
    torch.cuda.synchronize()
    ref = matmul_f64(xh, oracle.bf16_to_f32(oracle.dequant_q8(q, s, n, k)))
    yv = y.cpu().numpy()
    assert_bf16_close(yv, ref)
    assert err_ratio(yv, ref) <= 1e-4


def test_gemm_q8_glu(dev):
    n, k, t = 256, 512, 64
    q, s, _ = q8_host(n, k, 11)
    wq = ops.repack_q8(synth.to_dev(q), synth.to_dev(s), glu=True)
    xh = synth.x_host(t, k, seed=12)
    y = ops.gemm_q8(wq, synth.to_dev(xh))
    torch.cuda.synchronize()
    gq, gs = oracle.glu_rows(q, s, n, k, bits=8)
    act = glu_act(matmul_f64(xh, oracle.bf16_to_f32(oracle.dequant_q8(gq, gs, n, k))))
    assert_glu_close(oracle.bf16_to_f32(synth.bits(y)), act, 1e-3)
