"""One-pass decode GEMM for 1..64 rows (qe_matmul_w4_onepass_ex, wdec.hip) through the C-ABI vs the CPU oracle.

The kernel has the decode kernels' arithmetic: the exact products (u - 8) x summed in fp32 (as (128 + u) x and
-136 x on the matrix cores) and scaled once per 128-k group, i.e. the unrounded weights (u - 8) s: its fp32 output
is within 1e-4 * rms of the float64 product on those weights (the skinny kernel's gate), and inside the BASELINE
gate (2e-2 * rms) of the oracle's reference on the bf16 operand bf16_rn((u - 8) s). bf16 outputs are the RN of the
fp32 ones, GLU outputs silu(gate) up of the same sums. Rows of one call do not depend on each other (rows past m are
never stored), and the result does not depend on timing.
"""
import numpy as np
import pytest
import torch

import oracle
from qengine_amd import ops, synth
from test_gemv_gpu import (assert_gate, assert_glu_close, assert_rn_of, err_ratio, exact_w4, glu_act, matmul_f64,
                           oracle_ref, out_f32, setup_w4)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k", [(17408, 5120), (5120, 5120), (2048, 2048)])
@pytest.mark.parametrize("m", [1, 5, 32, 33, 64])
def test_onepass_vs_oracle(dev, n, k, m):
    """fp32 output within 1e-4 * rms of the float64 product on the unrounded weights and inside the BASELINE gate of
    the oracle's reference; the bf16 output is its RN bit for bit"""
    w, q, s = setup_w4(n, k, 1, seed=60 + m)
    xh = synth.x_host(m, k, seed=61 + m)
    x = synth.to_dev(xh)
    y = ops.matmul_w4_onepass(w, x)
    yb = ops.matmul_w4_onepass(w, x, out_bf16=True)
    torch.cuda.synchronize()
    assert y is not None and yb is not None
    r = err_ratio(y.cpu().numpy(), matmul_f64(xh, exact_w4(q, s, n, k, 1)))
    print(f"onepass n={n} k={k} m={m}: max|y - exact| / rms = {r:.2e}", flush=True)
    assert r <= 1e-4
    assert_gate(y.cpu().numpy(), oracle_ref(xh, q, s, n, k, 1), f"onepass n={n} k={k} m={m}")
    assert_rn_of(yb, y.cpu().numpy(), f"onepass m={m}")


@pytest.mark.parametrize("m", [7, 40])
def test_onepass_glu_and_bf16_scales(dev, m):
    """GLU matrices (the bf16 activation silu(gate) up, n / 2 columns) with fp16 scales, and plain bf16 scales"""
    n, k = 4096, 2048
    wg, qg, sg = setup_w4(n, k, 1, seed=70 + m, glu=True)
    xh = synth.x_host(m, k, seed=71 + m)
    x = synth.to_dev(xh)
    a = ops.matmul_w4_onepass(wg, x)
    wb, qb, sb = setup_w4(n, k, 0, seed=72 + m)
    yb = ops.matmul_w4_onepass(wb, x)
    torch.cuda.synchronize()
    act = glu_act(matmul_f64(xh, exact_w4(qg, sg, n, k, 1)))
    assert_glu_close(out_f32(a), act, 1e-4)
    assert err_ratio(yb.cpu().numpy(), matmul_f64(xh, exact_w4(qb, sb, n, k, 0))) <= 1e-4


def test_onepass_rows_independent_and_deterministic(dev):
    """a row's bits do not depend on the other rows of the call within a token-block count (m <= 32: one block of
    32; 33..64: two), and repeated calls are bit-identical"""
    n, k = 5120, 5120
    w, q, s = setup_w4(n, k, 1, seed=80)
    x = synth.to_dev(synth.x_host(64, k, seed=81))
    y64 = ops.matmul_w4_onepass(w, x).cpu().numpy().view(np.uint32)
    y40 = ops.matmul_w4_onepass(w, x[:40].contiguous()).cpu().numpy().view(np.uint32)
    y32 = ops.matmul_w4_onepass(w, x[:32].contiguous()).cpu().numpy().view(np.uint32)
    y3 = ops.matmul_w4_onepass(w, x[:3].contiguous()).cpu().numpy().view(np.uint32)
    y64b = ops.matmul_w4_onepass(w, x).cpu().numpy().view(np.uint32)
    assert np.array_equal(y64, y64b)
    assert np.array_equal(y40, y64[:40])
    assert np.array_equal(y3, y32[:3])


def test_onepass_shape_checks(dev):
    """shapes the kernel does not take are declined (returns None, nothing written): n % 64, an odd number of
    64-k steps per wave, x not 16-byte aligned"""
    w, _, _ = setup_w4(4096 + 16, 2048, 1, seed=90)
    x = synth.to_dev(synth.x_host(4, 2048, seed=91))
    assert ops.matmul_w4_onepass(w, x) is None
    w2, _, _ = setup_w4(1024, 1280, 1, seed=92)  # 20 steps: 5 per wave at m <= 32
    assert ops.matmul_w4_onepass(w2, synth.to_dev(synth.x_host(4, 1280, seed=93))) is None
    xb = torch.zeros(4 * 2048 + 1, dtype=torch.bfloat16, device=dev)[1:].view(4, 2048)
    w3, _, _ = setup_w4(1024, 2048, 1, seed=94)
    assert ops.matmul_w4_onepass(w3, xb) is None


def test_onepass_tail_parts_deterministic_and_graph(dev):
    """N = 17408 has 272 slabs of 64 rows: the 16 past the last whole round of 256 CUs run as K parts added by the
    last part to finish (a device-side count per tail slab, zero again after every call). Repeated calls, calls of
    other shapes in between, and a HIP graph captured on a stream that ran the kernel eagerly all give the same bits;
    a capture on a stream without its workspace runs the tail slabs whole (another summation order), within the same
    1e-4 * rms of the exact product"""
    n, k = 17408, 5120
    w, q, s = setup_w4(n, k, 1, seed=95)
    xh = synth.x_host(40, k, seed=96)
    x = synth.to_dev(xh)
    exact = matmul_f64(xh, exact_w4(q, s, n, k, 1))
    iv = torch.int32
    for m in (40, 8):
        xm = x[:m].contiguous()
        y1 = ops.matmul_w4_onepass(w, xm)
        w2, _, _ = setup_w4(4096, 2048, 1, seed=97)
        ops.matmul_w4_onepass(w2, synth.to_dev(synth.x_host(3, 2048, seed=98)))  # another shape in between
        y2 = ops.matmul_w4_onepass(w, xm)
        torch.cuda.synchronize()
        assert torch.equal(y1.view(iv), y2.view(iv)), m
        assert err_ratio(y1.cpu().numpy(), exact[:m]) <= 1e-4
        for warm in (True, False):
            cs = torch.cuda.Stream()
            cs.wait_stream(torch.cuda.current_stream())
            x_in = xm.clone()
            out = torch.empty(m, n, dtype=torch.float32, device=dev)
            if warm:
                with torch.cuda.stream(cs):
                    ops.matmul_w4_onepass(w, x_in, y=out)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cs):
                ops.matmul_w4_onepass(w, x_in, y=out)
            for r in range(3):
                xr = synth.to_dev(synth.x_host(m, k, seed=100 + r))
                want = ops.matmul_w4_onepass(w, xr)
                torch.cuda.synchronize()
                x_in.copy_(xr)
                g.replay()
                torch.cuda.synchronize()
                if warm:
                    assert torch.equal(out.view(iv), want.view(iv)), (m, r)
                else:
                    rr = err_ratio(out.cpu().numpy(), want.cpu().numpy())
                    assert rr <= 1e-5, (m, r, rr)
