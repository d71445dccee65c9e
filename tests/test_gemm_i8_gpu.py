"""W4A8 prefill GEMM (qe_gemm_w4_i8*, the reference's gemm_w4_i8 = x_to_i8_kernel + gemm_i8*_kernel,
src/kernels/gemm.cu:463-594) through the C-ABI vs the CPU oracle.

* Integer-valued inputs (every activation group holds one +-127 * 2^e, so sx = 2^e and q = x / 2^e exactly; power-
  of-two weight scales): the int32 group sums and every fp32 flush are exact, so the fp32 outputs equal the float64
  product bit for bit. This pins the activation permutation, the int8 operand layouts, the flush indexing and the
  epilogue.
* Random inputs (the reference test's channel-outlier activations, tests/test_gemm_i8.py:42-49): relative rms below
  1e-5 against the float64 emulation of the same quantization (the reference's own gate, test_gemm_i8.py:125-135),
  for G = 32, 64, 128, fp16 / bf16 scales, ragged T and N; GLU and bf16 outputs; the reference-named hooks."""
import numpy as np
import pytest
import torch

import oracle
from qengine_amd import call, ops, synth
from test_gemv_gpu import exact_w4, glu_act, out_f32

pytestmark = pytest.mark.gpu


def setup(n, k, sdt, seed, glu=False, q=None, s=None):
    if q is None:
        q, s = synth.w4_host(n, k, seed=seed, sdt=sdt)
    if glu:
        q, s = oracle.glu_rows(q, s, n, k)
    w = ops.repack_w4(synth.to_dev(q), synth.to_dev(s, torch.float16 if sdt else torch.bfloat16), glu=glu)
    return w, q, s


def outlier_x(t, k, seed):
    """bf16 activations with channel outliers (amax / rms per row ~ 15-60), as the reference's make_x"""
    rng = np.random.default_rng(seed)
    ch = np.exp(rng.standard_normal(k) * 0.6)
    ch[rng.permutation(k)[:max(1, k // 200)]] *= 12.0
    x = rng.standard_normal((t, k)) * ch * np.exp(rng.standard_normal((t, 1)) * 0.3)
    return synth.np_bf16(x.astype(np.float32))


def i8_ref(xb, q, s, n, k, sdt, G):
    xq, sx = oracle.x_to_i8(xb, G)
    return oracle.gemm_i8(xq, sx, oracle.unpack_w4(q, n, k), oracle.scale_to_f32(s, sdt).reshape(n, k // 128), G)


def relrms(y, ref):
    return float(np.sqrt(np.mean((np.asarray(y, np.float64) - ref) ** 2) / np.mean(ref ** 2)))


@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("n,k,t,sdt", [(256, 640, 37, 1), (304, 1024, 130, 0)])
def test_gemm_i8_exact_on_integer_inputs(dev, G, n, k, t, sdt):
    rng = np.random.default_rng(n + t + G)
    e = rng.integers(-1, 1, (t, k // G)).astype(np.float32)  # sums stay within fp32's 24 bits (exact flushes)
    xf = rng.integers(-20, 21, (t, k)).astype(np.float32).reshape(t, k // G, G)
    pos = rng.integers(0, G, (t, k // G))
    np.put_along_axis(xf, pos[:, :, None], np.where(rng.random((t, k // G, 1)) < 0.5, 127.0, -127.0), axis=2)
    xf = (xf * (2.0 ** e)[:, :, None]).reshape(t, k).astype(np.float32)
    xb = synth.np_bf16(xf)
    assert np.array_equal(oracle.bf16_to_f32(xb), xf)
    q, _ = synth.w4_host(n, k, seed=n)
    sf = (2.0 ** rng.integers(-8, -6, (n, k // 128))).astype(np.float32)
    s = sf.astype(np.float16).view(np.uint16) if sdt else synth.np_bf16(sf)
    w, q, s = setup(n, k, sdt, 0, q=q, s=s)
    y = ops.gemm_w4_i8(w, synth.to_dev(xb), G=G)
    torch.cuda.synchronize()
    want = xf.astype(np.float64) @ (oracle.unpack_w4(q, n, k).astype(np.float64) * np.repeat(sf, 128, axis=1)).T
    assert np.array_equal(y.cpu().numpy().astype(np.float64), want)


@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("n,k,t,sdt", [(128, 128, 1, 1), (512, 1024, 300, 1), (384, 2048, 129, 0), (1040, 5120, 200, 1)])
def test_gemm_i8_parity(dev, G, n, k, t, sdt):
    w, q, s = setup(n, k, sdt, seed=n + k + t)
    xb = outlier_x(t, k, seed=t + G)
    ref = i8_ref(xb, q, s, n, k, sdt, G)
    y = ops.gemm_w4_i8(w, synth.to_dev(xb), G=G)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert relrms(y, ref) < 1e-5  # the reference's gate against its int8 emulation
    exact = oracle.bf16_to_f32(xb).astype(np.float64) @ exact_w4(q, s, n, k, sdt).astype(np.float64).T
    # the quantization error of the 8-bit activations themselves (channel outliers: ~1e-2 at G = 32, ~2e-2 at 128);
    # a sanity bound, not a parity gate
    assert relrms(y, exact) < 5e-2
    yb = out_f32(ops.gemm_w4_i8(w, synth.to_dev(xb), G=G, out_bf16=True))
    assert np.all(np.abs(yb - y) <= 2.0 ** -8 * np.abs(y))  # bf16 output = RNE of the fp32 output


def test_gemm_i8_glu(dev):
    n, k, t, G = 512, 1024, 77, 64
    w, q, s = setup(n, k, 1, seed=5, glu=True)
    xb = outlier_x(t, k, seed=6)
    act = glu_act(i8_ref(xb, q, s, n, k, 1, G))
    y = out_f32(ops.gemm_w4_i8(w, synth.to_dev(xb), G=G))
    bound = 1e-4 * np.sqrt(np.mean(act ** 2)) + 2.0 ** -8 * np.abs(act)
    assert np.all(np.abs(y - act) <= bound), float((np.abs(y - act) / bound).max())


def test_gemm_i8_reference_hooks(dev):
    """qe_gemm_w4_i8 / qe_gemm_w4_i8_glu (the reference's signatures: bf16 scales, fp32 y or the bf16 act) equal
    the _ex entry point bit for bit; ci / ks are accepted"""
    n, k, t, G = 512, 1024, 40, 64
    w, q, s = setup(n, k, 0, seed=7)
    x = synth.to_dev(outlier_x(t, k, seed=8))
    want = ops.gemm_w4_i8(w, x, G=G)
    y = torch.zeros(t, n, device=dev)
    call("qe_gemm_w4_i8", w.q, w.s, n, k, x, y, t, G, 2, 100)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    wg, _, _ = setup(n, k, 0, seed=9, glu=True)
    want = ops.gemm_w4_i8(wg, x, G=G)
    act = torch.zeros(t, n // 2, dtype=torch.bfloat16, device=dev)
    call("qe_gemm_w4_i8_glu", wg.q, wg.s, n, k, x, act, t, G, 0, 0)
    torch.cuda.synchronize()
    assert torch.equal(act.view(torch.int16), want.view(torch.int16))


def test_gemm_i8_baseline_shape_sampled(dev):
    """C2's shape (M = 8192, K = 5120, N = 17408, fp16 scales, G = 64): 24 sampled rows vs the oracle"""
    n, k, t, G = 17408, 5120, 8192, 64
    qd, sd = synth.w4_dev(n, k, seed=21)
    w = ops.repack_w4(qd, sd)
    x = synth.x_dev(t, k, seed=22)
    y = ops.gemm_w4_i8(w, x, G=G)
    torch.cuda.synchronize()
    rows = np.random.default_rng(3).choice(t, 24, replace=False)
    ref = i8_ref(synth.bits(x[rows]), qd.cpu().numpy(), synth.bits(sd), n, k, 1, G)
    assert relrms(y[rows].cpu().numpy(), ref) < 1e-5


def test_gemm_i8_unaligned_activations(dev):
    """activation rows that are not 16-byte aligned (offset 1, row stride k + 9) take the pre-pass's scalar-load
    path; the results equal those of the aligned copy bit for bit"""
    n, k, t = 512, 1024, 45
    w, _, _ = setup(n, k, 1, seed=31)
    xa = synth.to_dev(synth.x_host(t, k, seed=32))
    big = torch.zeros(t, k + 9, dtype=torch.bfloat16, device=dev)
    big[:, 1:1 + k] = xa
    xu = big[:, 1:1 + k]
    want = ops.gemm_w4_i8(w, xa, G=64)
    got = ops.gemm_w4_i8(w, xu, G=64)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("glu", [False, True])
def test_gemm_q8_w8a8(dev, G, glu):
    """qe_gemm_q8 with G > 0 (the reference's W8A8 on a Q8 matrix, src/capi.cpp:41-44): the Q8 bytes are the int8
    weights; within 1e-5 relative rms of the float64 emulation (int8 activations x int8 weights x both scales)"""
    n, k, t = 512, 1024, 70
    rng = np.random.default_rng(G + glu)
    u = rng.integers(0, 256, (n, k))  # stored u = w + 128 (compressed-tensors 8-bit)
    q = (u[:, 0::4] | (u[:, 1::4] << 8) | (u[:, 2::4] << 16) | (u[:, 3::4] << 24)).astype(np.uint32).view(np.int32)
    s = synth.np_bf16((np.abs(rng.standard_normal((n, k // 128))) * 0.003).astype(np.float32))
    if glu:
        q, s = oracle.glu_rows(q, s, n, k, bits=8)
    dq, ds = oracle.repack_q8(q, s, n, k)
    xb = outlier_x(t, k, seed=G)
    xq, sx = oracle.x_to_i8(xb, G)
    wi = (np.stack([(q.view(np.uint32) >> (8 * b)) & 0xFF for b in range(4)], axis=2).reshape(n, k).astype(np.int64) - 128)
    ref = oracle.gemm_i8(xq, sx, wi, oracle.bf16_to_f32(s).reshape(n, k // 128), G)
    cols = n // 2 if glu else n
    y = torch.zeros(t, cols, dtype=torch.bfloat16 if glu else torch.float32, device=dev)
    call("qe_gemm_q8", synth.to_dev(dq.view(np.int8)), synth.to_dev(ds), n, k, synth.to_dev(xb), y, t, int(glu), G, 0)
    torch.cuda.synchronize()
    if glu:
        act = glu_act(ref)
        yb = out_f32(y)
        bound = 1e-4 * np.sqrt(np.mean(act ** 2)) + 2.0 ** -8 * np.abs(act)
        assert np.all(np.abs(yb - act) <= bound), float((np.abs(yb - act) / bound).max())
    else:
        assert relrms(y.cpu().numpy(), ref) < 1e-5
