"""W8A8 row GEMM of a W8 matrix (qe_gemm_w8a8_ex, qe_rows8): the reference's k_x_to_r8 + k_rows_qt
(src/flash/flash_pfq.cuh:473-651), dispatched by Worker::rows8 (src/flash/flash.cu:369-411), through the C-ABI vs the
CPU oracle.

The reference's arithmetic fixes every output bit (per (row, 128-k group): the exact integer sum, rn(sum * sx), one
fma at sw, groups in k order), so the tests are bit-exact against oracle.rows_w8a8 over oracle.x_to_i8(x, 128):
* channel-outlier activations (the reference test's make_x), group-128 and per-channel, fp16 and bf16 scales,
  ragged m and n, and the bf16 output as the RNE of the fp32 output;
* activation rows that are not 16-byte aligned (the scalar pre-pass);
* the rows8 dispatch: m >= 64 with k <= 4096 and an 8-element stride takes W8A8, anything else the W8A16 GEMM;
* BASELINE config 3 at m = 4096 (K = 2048, N = 8192, per-channel fp16 scales), sampled rows.
Against the float64 product of the unquantized activations the error is the 8-bit activation quantization itself:
a sanity bound only."""
import numpy as np
import pytest
import torch

import oracle
from qengine_amd import ops, synth
from test_gemm_i8_gpu import outlier_x, relrms

pytestmark = pytest.mark.gpu


def setup(n, k, per_channel, sdt, seed):
    q, s = synth.w8_host(n, k, seed=seed, per_channel=per_channel)
    if not sdt:  # the same magnitudes as bf16 scales
        s = synth.np_bf16(oracle.f16_to_f32(s))
    if not per_channel:
        s = s.reshape(n, k // 128)
    w = ops.tile_w8(synth.to_dev(q), synth.to_dev(s, torch.float16 if sdt else torch.bfloat16), per_channel)
    return w, q, oracle.scale_to_f32(s, sdt).astype(np.float32)


def want(xb, q, sw, per_channel):
    xq, sx = oracle.x_to_i8(xb, 128)
    return oracle.rows_w8a8(xq, sx, q, sw, per_channel)


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("n,k,t,sdt", [(256, 128, 1, 1), (272, 640, 37, 0), (1040, 1024, 200, 1), (512, 4096, 130, 0)])
def test_w8a8_bit_exact(dev, per_channel, n, k, t, sdt):
    w, q, sw = setup(n, k, per_channel, sdt, seed=n + k + t)
    xb = outlier_x(t, k, seed=t + k)
    ref = want(xb, q, sw, per_channel)
    y = ops.gemm_w8a8(w, synth.to_dev(xb))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.array_equal(y, ref), f"{np.count_nonzero(y != ref)} of {y.size} differ"
    yb = ops.gemm_w8a8(w, synth.to_dev(xb), out_bf16=True)
    assert np.array_equal(synth.bits(yb.cpu()), oracle.f32_to_bf16(ref))
    wd = q.astype(np.float64) * (sw[:, None] if per_channel else np.repeat(sw, 128, axis=1))
    exact = oracle.bf16_to_f32(xb).astype(np.float64) @ wd.T
    assert relrms(y, exact) < 5e-2


def test_w8a8_unaligned_rows(dev):
    """rows at an odd element offset with an odd stride: the scalar pre-pass, the same bits"""
    n, k, t = 384, 1024, 75
    w, q, sw = setup(n, k, False, 1, seed=9)
    xb = outlier_x(t, k, seed=10)
    big = torch.zeros(t, k + 3, dtype=torch.bfloat16, device=dev)
    big[:, 1:k + 1] = synth.to_dev(xb, torch.bfloat16)
    y = ops.gemm_w8a8(w, big[:, 1:k + 1])
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), want(xb, q, sw, False))


@pytest.mark.parametrize("m,k,stride_pad,w8a8", [(64, 1024, 0, True), (63, 1024, 0, False), (100, 4224, 0, False),
                                                 (100, 1024, 2, False), (300, 4096, 8, True)])
def test_rows8_dispatch(dev, m, k, stride_pad, w8a8):
    """Worker::rows8: W8A8 only for m >= 64, k <= 4096 and ldx % 8 == 0; otherwise the W8A16 GEMM's bits (aligned
    rows) or the W8A16 GEMV's over 16-row blocks (its gemv_w8_rows)"""
    n = 512
    w, q, sw = setup(n, k, False, 0, seed=m + k)
    xb = outlier_x(m, k, seed=m)
    big = torch.zeros(m, k + stride_pad, dtype=torch.bfloat16, device=dev)
    big[:, :k] = synth.to_dev(xb, torch.bfloat16)
    x = big[:, :k]
    y = ops.rows8(w, x)
    if w8a8:
        other = ops.gemm_w8a8(w, x)
    elif x.stride(0) % 8 == 0:
        other = ops.gemm_w8(w, x)
    else:
        other = torch.cat([ops.gemv_w8(w, x[r:r + 16]) for r in range(0, m, 16)])
    torch.cuda.synchronize()
    assert torch.equal(y, other)
    if w8a8:
        assert np.array_equal(y.cpu().numpy(), want(xb, q, sw, False))


def test_w8a8_baseline_shape_sampled(dev):
    """BASELINE config 3 at M = 4096 (K = 2048, N = 8192, per-channel fp16 scales): 64 sampled rows bit-exact"""
    n, k, t = 8192, 2048, 4096
    w, q, sw = setup(n, k, True, 1, seed=77)
    x = synth.x_dev(t, k, seed=78)
    y = ops.gemm_w8a8(w, x)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(6).choice(t, 64, replace=False))
    xb = synth.bits(x[torch.from_numpy(rows).to(dev)].contiguous().cpu())
    got = y[torch.from_numpy(rows).to(dev)].cpu().numpy()
    assert np.array_equal(got, want(xb, q, sw, True))
