"""Decode GEMV / skinny GEMM (m = 1..16) through the C-ABI vs the CPU oracle.

Gates:
  * BASELINE: max|y - ref| <= 2e-2 * rms(ref), ref = the oracle's dequantize-then-matmul: weights dequantized to
    bf16 exactly as the reference does (bf16_rn((u - 8) * s), bf16_rn(w * s)), product in fp32/float64.
  * the reference's own test gate (tests/test_gemv.py:36,84): max|y - ref| / max|ref| < 1e-2, same ref.
  * the kernel's own arithmetic: this GEMV multiplies the unrounded weights (u - 8) * s (exact in fp32), so its
    fp32 outputs are within 1e-4 * rms of that exact product (float64).
  * bit-identity: every row count from 2 to 16 (the matrix-core skinny kernel) gives the same bits per row (the
    reference's skinny == GEMV contract, tests/test_skinny.py:1-2), and repeated calls are identical (deterministic
    split-K). The m = 1 matrix-core GEMV (gemv1.hip, another summation order) agrees with them to 1e-5 * rms; with
    the batch_invariant config m = 1 takes the skinny kernel and every m in 1..64 has the row's own bits.
"""
import numpy as np
import pytest
import torch

import oracle
from qengine_amd import call, ops, synth

pytestmark = pytest.mark.gpu
TOL = 2e-2


def err_ratio(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / np.sqrt(np.mean(ref ** 2)))


def assert_bf16_close(y, ref, tol=TOL):
    """BASELINE gate for bf16 outputs: max|y - ref| <= tol * rms(ref), plus the output's own rounding (half an ulp
    of each value, doubled: 2^-8 |ref|). With heavy-tailed outputs (per-row scales |N(0,1)|) the correctly rounded
    exact result alone exceeds tol * rms on the largest values, so the rounding allowance is part of the gate."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    bound = tol * np.sqrt(np.mean(ref ** 2)) + 2.0 ** -8 * np.abs(ref)
    assert np.all(np.abs(y - ref) <= bound), float((np.abs(y - ref) / bound).max())


def assert_gate(y, ref, what, tol=TOL):
    """the BASELINE gate as stated, with no allowance: max|y - ref| <= tol * rms(ref), ref = the fp32 dequantize-then-
    matmul reference on the weight operand the kernel multiplies; prints the ratio"""
    r = err_ratio(y, ref)
    print(f"gate {what}: max|y - ref| / rms(ref) = {r:.3e}", flush=True)
    assert r <= tol, (what, r)
    return r


def assert_rn_of(y_bf16, y_f32, what):
    """a bf16 output equals the round-to-nearest-even of the same call's fp32 output, bit for bit (so the gate on the
    fp32 output covers the bf16 output up to its own rounding, <= 2^-9 |y|)"""
    want = synth.np_bf16(np.asarray(y_f32, np.float32))
    got = synth.bits(y_bf16) if isinstance(y_bf16, torch.Tensor) else np.asarray(y_bf16)
    assert np.array_equal(got, want), (what, int(np.sum(got != want)))


def ref_gate(y, ref):
    """reference tests/test_gemv.py:84 gate"""
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / np.abs(ref).max())


def exact_w4(q, s, n, k, sdt):
    """(u - 8) * s as float32 (exact)"""
    return oracle.unpack_w4(q, n, k).astype(np.float32) * np.repeat(oracle.scale_to_f32(s, sdt), 128, axis=1)


def exact_w8(q, s, n, k, per_channel):
    sf = oracle.f16_to_f32(s)
    sf = sf.reshape(n, 1) if per_channel else np.repeat(sf.reshape(n, k // 128), 128, axis=1)
    return q.astype(np.float32) * sf


def oracle_ref(xh, q, s, n, k, sdt):
    """the BASELINE reference: bf16 dequantization as the reference does it, then the matmul (float64)"""
    return matmul_f64(xh, oracle.bf16_to_f32(oracle.dequant_w4(q, s, n, k, sdt)))


def oracle_ref_w8(xh, q, s, n, k, per_channel):
    return matmul_f64(xh, oracle.bf16_to_f32(oracle.dequant_w8(q, s, n, k, per_channel, 1)))


def matmul_f64(xh, w):
    return oracle.bf16_to_f32(xh).astype(np.float64) @ w.astype(np.float64).T


def out_f32(y):
    return oracle.bf16_to_f32(synth.bits(y)) if y.dtype == torch.bfloat16 else y.cpu().numpy()


def glu_act(y):
    """product [m][n] of a GLU-interleaved matrix -> act [m][n/2] = silu(gate) * up (float64)"""
    y = np.asarray(y, np.float64)
    m, n = y.shape
    yt = y.reshape(m, n // 16, 2, 8)
    gate, up = yt[:, :, 0, :], yt[:, :, 1, :]
    return (gate / (1 + np.exp(-gate)) * up).reshape(m, n // 2)


def assert_glu_close(y_bf16, act_ref, rel_rms):
    """GLU outputs are heavy-tailed (a product of two sums): besides a tolerance relative to rms(act), each
    bf16 output carries its own rounding (<= 2^-9 relative, doubled): |y - act| <= rel_rms * rms + 2^-8 |act|"""
    y = np.asarray(y_bf16, np.float64)
    bound = rel_rms * np.sqrt(np.mean(act_ref ** 2)) + 2.0 ** -8 * np.abs(act_ref)
    assert np.all(np.abs(y - act_ref) <= bound), float((np.abs(y - act_ref) / bound).max())


def setup_w4(n, k, sdt, seed, glu=False):
    q, s = synth.w4_host(n, k, seed=seed, sdt=sdt)
    if glu:
        q, s = oracle.glu_rows(q, s, n, k)
    w = ops.repack_w4(synth.to_dev(q), synth.to_dev(s, torch.float16 if sdt else torch.bfloat16), glu=glu)
    return w, q, s


# (8192, 1280), (16384, 5120): two to four 16-row tiles per CU, as in the BASELINE shapes
@pytest.mark.parametrize("n,k", [(64, 256), (256, 1280), (1024, 5120), (8192, 1280), (16384, 5120)])
@pytest.mark.parametrize("sdt", [0, 1])
def test_gemv_w4_parity(dev, n, k, sdt):
    w, q, s = setup_w4(n, k, sdt, seed=n + k + sdt)
    xh = synth.x_host(16, k, seed=k)
    x = synth.to_dev(xh)
    ref_ex = matmul_f64(xh, exact_w4(q, s, n, k, sdt))
    ref = oracle_ref(xh, q, s, n, k, sdt)
    for m in (1, 2, 3, 4, 5, 8, 9, 16):
        for out_bf16 in (False, True):
            y = out_f32(ops.gemv_w4(w, x[:m], out_bf16=out_bf16))
            assert_bf16_close(y, ref[:m])
            assert ref_gate(y, ref[:m]) < 1e-2
            if not out_bf16:
                ex = err_ratio(y, ref_ex[:m])
                assert ex <= 1e-4, (m, ex)


@pytest.mark.parametrize("n,k", [(256, 1280), (5120, 5120), (16384, 2048), (5120, 13824), (2048, 13824)])
def test_gemv_w4_batch_equals_alone(dev, n, k):
    w, _, _ = setup_w4(n, k, 1, seed=7)
    x = synth.to_dev(synth.x_host(16, k, seed=8))
    full = ops.gemv_w4(w, x)
    torch.cuda.synchronize()
    fb = full.cpu().numpy().view(np.uint32)
    for m in range(2, 17):
        y = ops.gemv_w4(w, x[:m])
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), fb[:m]), m
    for r in (0, 5, 14):
        y = ops.gemv_w4(w, x[r:r + 2])
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), fb[r:r + 2]), r
    for r in (0, 9):
        y = ops.gemv_w4(w, x[r:r + 1])
        torch.cuda.synchronize()
        assert err_ratio(y.cpu().numpy()[0], full.cpu().numpy()[r]) <= 1e-5, r
    again = ops.gemv_w4(w, x)
    torch.cuda.synchronize()
    assert np.array_equal(again.cpu().numpy().view(np.uint32), fb)


@pytest.mark.parametrize("n,k", [(64, 256), (1024, 2048), (8192, 1280)])
def test_gemv_w4_glu(dev, n, k):
    w, q, s = setup_w4(n, k, 1, seed=31, glu=True)
    xh = synth.x_host(16, k, seed=32)
    x = synth.to_dev(xh)
    act = glu_act(matmul_f64(xh, exact_w4(q, s, n, k, 1)))
    full = ops.gemv_w4(w, x)
    torch.cuda.synchronize()
    yv = out_f32(full)
    assert_glu_close(yv, act, 1e-4)
    # the reference's bf16-rounded weights: their rounding shows up in act
    act_bw = glu_act(oracle.matmul_bf16(xh, oracle.dequant_w4(q, s, n, k, 1)))
    assert_glu_close(yv, act_bw, 2 * TOL)
    fb = synth.bits(full)
    for m in (2, 3, 8):
        y = ops.gemv_w4(w, x[:m])
        torch.cuda.synchronize()
        assert np.array_equal(synth.bits(y), fb[:m])
    y1 = out_f32(ops.gemv_w4(w, x[:1]))
    assert_glu_close(y1, act[:1], 1e-4)


def test_reference_named_hooks(dev):
    """qe_gemv_w4 / qe_gemv_w4g / qe_skinny_w4 (bf16 scales, fp32 out, stride k / n) == the _ex entry"""
    n, k = 512, 2048
    w, q, s = setup_w4(n, k, 0, seed=41)
    x = synth.to_dev(synth.x_host(16, k, seed=42))
    for m in (1, 7, 16):
        ref = ops.gemv_w4(w, x[:m])
        y = torch.full((m, n), float("nan"), device=dev)
        call("qe_gemv_w4", w.q, w.s, n, k, x, y, m)
        y2 = torch.full((m, n), float("nan"), device=dev)
        r = call("qe_skinny_w4", w.q, w.s, n, k, x, y2, m, 0)
        y3 = torch.full((m, n), float("nan"), device=dev)
        call("qe_gemv_w4g", w.q, w.s, n, k, x, y3, m, 0)
        torch.cuda.synchronize()
        assert r == 1
        for yy in (y, y2, y3):
            assert torch.equal(yy.view(torch.int32), ref[:m].view(torch.int32))
    # 17..32 rows: the GEMV in row blocks of 16
    xh32 = synth.x_host(32, k, seed=43)
    y = torch.empty(32, n, device=dev)
    call("qe_gemv_w4", w.q, w.s, n, k, synth.to_dev(xh32), y, 32)
    torch.cuda.synchronize()
    assert err_ratio(y.cpu().numpy(), matmul_f64(xh32, exact_w4(q, s, n, k, 0))) <= 1e-4


# the reference's row counts for its skinny == GEMV test (reference tests/test_skinny.py:13)
MS_SKINNY = [1, 2, 5, 8, 9, 12, 15, 16, 17, 20, 24, 25, 31, 32]


# 17..32 rows: (5120, 5120) and (2048, 1280) take the skinny kernel's 32-row launch, (16384, 2048) (one round of
# 64-row slabs) the one-pass kernel
@pytest.mark.parametrize("n,k", [(5120, 5120), (2048, 1280), (16384, 2048)])
def test_skinny_hook_bit_identical_to_gemv_w4g(dev, n, k):
    """the reference's skinny test (tests/test_skinny.py:16-41) bound to this library: qe_skinny_w4 returns 1 for
    every m in its MS list (1..32, the reference's skinny_w4 range, skinny.cu:572) and its outputs equal qe_gemv_w4g's
    bit for bit, plain (fp32) and GLU (bf16 act); plain outputs within 1e-4 rms of the exact product"""
    for glu in (0, 1):
        w, q, s = setup_w4(n, k, 0, seed=71 + glu, glu=bool(glu))
        xh = synth.x_host(32, k, seed=72 + glu)
        ref_ex = matmul_f64(xh, exact_w4(q, s, n, k, 0))
        for m in MS_SKINNY:
            x = synth.to_dev(xh[:m])
            cols, dt = (n // 2, torch.bfloat16) if glu else (n, torch.float32)
            y0 = torch.full((m, cols), float("nan"), dtype=dt, device=dev)
            y1 = y0.clone()
            call("qe_gemv_w4g", w.q, w.s, n, k, x, y0, m, glu)
            r = call("qe_skinny_w4", w.q, w.s, n, k, x, y1, m, glu)
            torch.cuda.synchronize()
            assert r == 1, (glu, m)
            iv = torch.int16 if glu else torch.int32
            assert torch.equal(y0.view(iv), y1.view(iv)), (glu, m)
            if not glu:
                assert err_ratio(y1.cpu().numpy(), ref_ex[:m]) <= 1e-4, m


def test_skinny_hook_unsupported_returns_0(dev):
    """17..32 rows need an even K slicing for the one-launch wide kernel: K / 128 = 63 has none, so qe_skinny_w4
    returns 0 there (the reference's "unsupported", its callers fall back to gemv_w4) and writes nothing; 1..16 rows
    run"""
    n, k = 1024, 8064
    w, q, s = setup_w4(n, k, 0, seed=73)
    x = synth.to_dev(synth.x_host(20, k, seed=74))
    for m, want in ((16, 1), (17, 0), (20, 0)):
        y = torch.full((m, n), float("nan"), device=dev)
        r = call("qe_skinny_w4", w.q, w.s, n, k, x[:m], y, m, 0)
        torch.cuda.synchronize()
        assert r == want, m
        assert bool(torch.isnan(y).all()) == (want == 0), m


@pytest.mark.parametrize("n,k", [(5120, 5120), (17408, 5120)])
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_gemv_w4_baseline_shapes(dev, n, k, m):
    """BASELINE configs 0 (m = 1, n = 17408) and 1 (m in {2,4,8,16}, n in {5120, 17408}), full size, bf16 out"""
    if m == 1 and n == 5120:
        pytest.skip("not a BASELINE shape")
    w, q, s = setup_w4(n, k, 1, seed=1000 + n)
    xh = synth.x_host(m, k, seed=2000 + m)
    x = synth.to_dev(xh)
    y16 = ops.gemv_w4(w, x, out_bf16=True)
    y32 = ops.gemv_w4(w, x)
    torch.cuda.synchronize()
    # the decode kernels multiply the unrounded weights (u - 8) * s: ref = that exact fp32 dequantization, product in
    # float64; the gate holds on the fp32 and on the bf16 output, and the bf16 output is the RN of the fp32 one
    ref_ex = matmul_f64(xh, exact_w4(q, s, n, k, 1))
    assert_gate(y32.cpu().numpy(), ref_ex, f"C0/C1 m={m} n={n} fp32 out")
    assert_gate(out_f32(y16), ref_ex, f"C0/C1 m={m} n={n} bf16 out")
    assert_rn_of(y16, y32.cpu().numpy(), "C0/C1")
    assert err_ratio(y32.cpu().numpy(), ref_ex) <= 1e-4
    # against the reference's bf16-rounded weight operand: the weight rounding (~2^-9 relative per weight) plus the
    # output's own rounding
    assert_bf16_close(out_f32(y16), oracle.matmul_bf16(xh, oracle.dequant_w4(q, s, n, k, 1)))


@pytest.mark.parametrize("n,k", [(16, 128), (48, 384), (80, 640)])
def test_gemv_small_odd_shapes(dev, n, k):
    """one and an odd number of 16-row tiles (the skinny kernel's one-tile-per-wave fallback), one group, slices that
    no even slicing divides (K / 128 = 3, 5), W4 and W8, every m"""
    w, q, s = setup_w4(n, k, 1, seed=n * k)
    xh = synth.x_host(16, k, seed=n + k)
    x = synth.to_dev(xh)
    ref = oracle_ref(xh, q, s, n, k, 1)
    ref_ex = matmul_f64(xh, exact_w4(q, s, n, k, 1))
    full = ops.gemv_w4(w, x)
    torch.cuda.synchronize()
    for m in range(1, 17):
        y = ops.gemv_w4(w, x[:m])
        torch.cuda.synchronize()
        assert_bf16_close(out_f32(y), ref[:m])
        assert err_ratio(y.cpu().numpy(), ref_ex[:m]) <= 1e-4, m
        if m >= 2:
            assert np.array_equal(y.cpu().numpy().view(np.uint32), full.cpu().numpy().view(np.uint32)[:m]), m
    q8, s8 = synth.w8_host(n, k, seed=n, per_channel=True)
    w8 = ops.tile_w8(synth.to_dev(q8), synth.to_dev(s8, torch.float16), True)
    ref8 = oracle_ref_w8(xh, q8, s8, n, k, True)
    for m in (1, 2, 7, 16):
        assert_bf16_close(out_f32(ops.gemv_w8(w8, x[:m], out_bf16=True)), ref8[:m])


@pytest.mark.parametrize("n,k", [(20480, 5120), (20480, 8064)])
def test_gemv_long_slices(dev, n, k):
    """K slices of more than 8 groups, whose scale dwords (and up-front activation pieces) outnumber a wave's 64
    lanes: (20480, 5120) takes 10-group slices in the m = 1 and skinny matrix-core kernels; (20480, 8064) has no even
    slicing (K / 128 = 63) and takes 4 uneven slices of 15-16 groups in the VALU GEMV (m = 1, W4 and W8) and the
    skinny kernel (m >= 2)"""
    w, q, s = setup_w4(n, k, 1, seed=n + k)
    xh = synth.x_host(16, k, seed=k + 1)
    x = synth.to_dev(xh)
    ref = oracle_ref(xh, q, s, n, k, 1)
    for m in (1, 2, 4, 16):
        y = out_f32(ops.gemv_w4(w, x[:m], out_bf16=True))
        assert_bf16_close(y, ref[:m])
    del w, ref
    q8, s8 = synth.w8_host(n, k, seed=53, per_channel=False)
    s8 = s8.reshape(n, k // 128)
    w8 = ops.tile_w8(synth.to_dev(q8), synth.to_dev(s8, torch.float16), False)
    ref8 = oracle_ref_w8(xh[:2], q8, s8, n, k, False)
    for m in (1, 2):
        assert_bf16_close(out_f32(ops.gemv_w8(w8, x[:m], out_bf16=True)), ref8[:m])


# m = 1 grids whose tiles past the last whole round of the 256 CUs run as quarter blocks (4 rows each): slices of
# 20 groups (5 wave-loads of 8 steps), 5 (the last wave-load 2 steps short), 8 with two quarters on half the CUs, 10
# (the last wave-load half full) and 16
@pytest.mark.parametrize("n,k,sdt", [(17408, 5120, 1), (5120, 5120, 0), (14336, 4096, 1), (16640, 2560, 0),
                                     (17408, 4096, 0)])
def test_gemv_m1_quarter_tiles(dev, n, k, sdt):
    """every row (quarter rows included) within 1e-4 * rms of the exact product, the bf16 output its RN, GLU outputs
    silu(gate) up of the same sums, repeated calls bit-identical"""
    w, q, s = setup_w4(n, k, sdt, seed=n + 3 * k + sdt)
    xh = synth.x_host(1, k, seed=k + 5)
    x = synth.to_dev(xh)
    y = ops.gemv_w4(w, x)
    y2 = ops.gemv_w4(w, x)
    yb = ops.gemv_w4(w, x, out_bf16=True)
    torch.cuda.synchronize()
    ex = matmul_f64(xh, exact_w4(q, s, n, k, sdt))
    r = err_ratio(y.cpu().numpy(), ex)
    tail = err_ratio(y.cpu().numpy()[:, n - 1024:], ex[:, n - 1024:])
    print(f"m1 quarter n={n} k={k}: max|y - exact| / rms = {r:.2e} (last 1024 rows {tail:.2e})", flush=True)
    assert r <= 1e-4 and tail <= 1e-4
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    assert_rn_of(yb, y.cpu().numpy(), f"quarter n={n}")
    del w, ex
    wg, qg, sg = setup_w4(n, k, sdt, seed=n + 3 * k + sdt + 1, glu=True)
    a = ops.gemv_w4(wg, x)
    torch.cuda.synchronize()
    assert_glu_close(out_f32(a), glu_act(matmul_f64(xh, exact_w4(qg, sg, n, k, sdt))), 1e-4)


# m = 1 where K / 128 has no even slicing of the streaming kernel: 8 slices of floor / ceil (K / 1024) groups.
# K = 17408 (136 groups, 17 per slice) on 320 tiles (quarter blocks for the 64 past one round) and on 128 tiles;
# K = 13824 (108 groups: slices of 13 and 14); K = 28672 (224 groups: 28 per slice, the 32-group instance)
@pytest.mark.parametrize("n,k,sdt", [(5120, 17408, 1), (2048, 17408, 0), (4096, 13824, 1), (1024, 28672, 0), (5120, 13824, 0), (1024, 8192, 1), (1536, 6144, 0)])
def test_gemv_m1_uneven_slices(dev, n, k, sdt):
    """every row within 1e-4 * rms of the exact product, the bf16 output its RN, GLU outputs silu(gate) up of the same
    sums, repeated calls bit-identical"""
    w, q, s = setup_w4(n, k, sdt, seed=n + k + sdt + 7)
    xh = synth.x_host(1, k, seed=k + 9)
    x = synth.to_dev(xh)
    y = ops.gemv_w4(w, x)
    y2 = ops.gemv_w4(w, x)
    yb = ops.gemv_w4(w, x, out_bf16=True)
    torch.cuda.synchronize()
    ex = matmul_f64(xh, exact_w4(q, s, n, k, sdt))
    r = err_ratio(y.cpu().numpy(), ex)
    print(f"m1 uneven n={n} k={k}: max|y - exact| / rms = {r:.2e}", flush=True)
    assert r <= 1e-4
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    assert_rn_of(yb, y.cpu().numpy(), f"uneven n={n}")
    del w, ex
    wg, qg, sg = setup_w4(n, k, sdt, seed=n + k + sdt + 8, glu=True)
    a = ops.gemv_w4(wg, x)
    torch.cuda.synchronize()
    assert_glu_close(out_f32(a), glu_act(matmul_f64(xh, exact_w4(qg, sg, n, k, sdt))), 1e-4)


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("n,k", [(64, 256), (8192, 2048), (4096, 5120)])
def test_gemv_w8_parity(dev, per_channel, n, k):
    q, s = synth.w8_host(n, k, seed=51, per_channel=per_channel)
    if not per_channel:
        s = s.reshape(n, k // 128)
    w = ops.tile_w8(synth.to_dev(q), synth.to_dev(s, torch.float16), per_channel)
    xh = synth.x_host(16, k, seed=52)
    x = synth.to_dev(xh)
    ref_ex = matmul_f64(xh, exact_w8(q, s, n, k, per_channel))
    ref = oracle_ref_w8(xh, q, s, n, k, per_channel)
    full = ops.gemv_w8(w, x)
    torch.cuda.synchronize()
    assert err_ratio(full.cpu().numpy(), ref_ex) <= 1e-4
    # against the reference's bf16-rounded weights (K = 5120: their rounding alone reaches ~2e-2 * rms on the rows
    # with the largest scales), the BASELINE gate with the rounding allowance of the other tests
    assert_bf16_close(full.cpu().numpy(), ref)
    for m in (1, 2, 4, 9):
        y = ops.gemv_w8(w, x[:m], out_bf16=True)
        assert_bf16_close(out_f32(y), ref[:m])
        y32 = ops.gemv_w8(w, x[:m])
        torch.cuda.synchronize()
        # the unrelaxed gate on the fp32 output (per-channel scales make the outputs heavy-tailed: max|y| ~ 20 rms,
        # so a bf16 output's own rounding, up to 2^-9 |y|, alone can exceed 2e-2 rms); the bf16 output is its RN
        assert_gate(y32.cpu().numpy(), ref_ex[:m], f"W8 m={m} n={n} k={k} pc={per_channel} fp32 out")
        assert_rn_of(y, y32.cpu().numpy(), "W8 GEMV")
        if m == 1:  # m = 1 kernels (per-channel: the streaming W8 kernel; m >= 2: the skinny kernel, same rows for every m)
            assert err_ratio(y32.cpu().numpy(), full.cpu().numpy()[:1]) <= 1e-5
        else:
            assert np.array_equal(y32.cpu().numpy().view(np.uint32), full.cpu().numpy().view(np.uint32)[:m]), m


# the streaming m = 1 kernel on per-channel W8 records (8 K slices of 4, 10 and 8 wave-loads of 64 k: C3, N = 12288 and
# 16384), and grids it does not take (fewer than 16 waves per CU: the VALU GEMV at K = 2048, the skinny kernel at 5120)
@pytest.mark.parametrize("n,k,sdt", [(8192, 2048, 1), (12288, 5120, 0), (16384, 4096, 0), (2048, 2048, 1),
                                     (4096, 5120, 1)])
def test_gemv_w8c_m1(dev, n, k, sdt):
    """fp32 output within 1e-4 * rms of the exact product and inside the BASELINE gate, the bf16 output its RN,
    repeated calls bit-identical, within 1e-5 * rms of the batched rows' kernel (batch_invariant: m = 1 on it)"""
    q, s16 = synth.w8_host(n, k, seed=n + k + sdt, per_channel=True)
    s = s16 if sdt else synth.np_bf16(oracle.f16_to_f32(s16))  # fp16 or bf16 scales
    sf = oracle.f16_to_f32(s) if sdt else oracle.bf16_to_f32(s)
    w = ops.tile_w8(synth.to_dev(q), synth.to_dev(s, torch.float16 if sdt else torch.bfloat16), True)
    xh = synth.x_host(1, k, seed=k + 3)
    x = synth.to_dev(xh)
    ex = matmul_f64(xh, q.astype(np.float32) * sf.reshape(n, 1))
    y = ops.gemv_w8(w, x)
    y2 = ops.gemv_w8(w, x)
    yb = ops.gemv_w8(w, x, out_bf16=True)
    torch.cuda.synchronize()
    r = err_ratio(y.cpu().numpy(), ex)
    print(f"w8c m1 n={n} k={k}: max|y - exact| / rms = {r:.2e}", flush=True)
    assert r <= 1e-4
    assert_gate(y.cpu().numpy(), ex, f"W8C m=1 n={n} k={k}")
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    assert_rn_of(yb, y.cpu().numpy(), "W8C m=1")
    ops.set_config(batch_invariant=1)
    try:
        yi = ops.gemv_w8(w, x)
        torch.cuda.synchronize()
    finally:
        ops.set_config(batch_invariant=0)
    assert err_ratio(y.cpu().numpy(), yi.cpu().numpy()) <= 1e-5


def test_gemv_w8_reference_hook(dev):
    """qe_quantize_w8 + qe_gemv_w8 vs the reference's torch check (tests/test_w8.py), m = 1, 4, 8"""
    n, k = 256, 5120
    rng = np.random.default_rng(60)
    wb = synth.np_bf16(rng.standard_normal((n, k)) * 0.02)
    wd = ops.quantize_w8(synth.to_dev(wb))
    qr, sr = oracle.quantize_w8(wb, n, k)
    wref = qr.astype(np.float64) * np.repeat(oracle.bf16_to_f32(sr), 128, axis=1)
    for m in (1, 4, 8):
        xh = synth.x_host(m, k, seed=61 + m)
        y = torch.empty(m, n, device=dev)
        call("qe_gemv_w8", wd.q, wd.s, n, k, synth.to_dev(xh), y, m)
        torch.cuda.synchronize()
        ref = oracle.bf16_to_f32(xh).astype(np.float64) @ wref.T
        assert ref_gate(y.cpu().numpy(), ref) < 1e-2


def _unaligned_rows(xh, mode):
    """x rows whose start is not 16-byte aligned: 'offset' = the block starts 2 elements into its allocation (row
    stride k), 'stride' = rows k + 2 elements apart (aligned start)"""
    m, k = xh.shape
    xd = synth.to_dev(xh)
    if mode == "offset":
        buf = torch.empty(m * k + 2, dtype=torch.bfloat16, device=xd.device)
        x = buf[2:].view(m, k)
    else:
        buf = torch.empty(m, k + 2, dtype=torch.bfloat16, device=xd.device)
        x = buf[:, :k]
    x.copy_(xd)
    assert x.data_ptr() % 16 != 0 or x.stride(0) % 8 != 0
    return x


@pytest.mark.parametrize("mode", ["offset", "stride"])
@pytest.mark.parametrize("n,k", [(1024, 5120), (256, 1280), (5120, 13824)])
def test_gemv_unaligned_activations(dev, mode, n, k):
    """activation rows that are only 4-byte aligned: m = 1 takes the VALU GEMV, m >= 2 the matrix-core kernel with
    4-dword activation loads, whose rows equal those of the aligned copy bit for bit; W4 and W8 against the oracle"""
    w, q, s = setup_w4(n, k, 1, seed=n + 3 * k)
    xh = synth.x_host(16, k, seed=k + 7)
    x = _unaligned_rows(xh, mode)
    xa = synth.to_dev(xh)
    ref_ex = matmul_f64(xh, exact_w4(q, s, n, k, 1))
    for m in (1, 2, 8, 16):
        y = ops.gemv_w4(w, x[:m])
        torch.cuda.synchronize()
        assert err_ratio(y.cpu().numpy(), ref_ex[:m]) <= 1e-4, (mode, m)
        if m >= 2:
            assert torch.equal(y, ops.gemv_w4(w, xa[:m])), (mode, m)
    q8, s8 = synth.w8_host(n, k, seed=n + k, per_channel=True)
    w8 = ops.tile_w8(synth.to_dev(q8), synth.to_dev(s8, torch.float16), True)
    ref8 = matmul_f64(xh, exact_w8(q8, s8, n, k, True))
    for m in (1, 2, 16):
        y = ops.gemv_w8(w8, x[:m])
        torch.cuda.synchronize()
        assert err_ratio(y.cpu().numpy(), ref8[:m]) <= 1e-4, (mode, m)
        if m >= 2:
            assert torch.equal(y, ops.gemv_w8(w8, xa[:m])), (mode, m)


# the reference's row counts for its skinny == GEMV test (reference tests/test_skinny.py:13), with the 33..64 rows of
# its decode batch test (tests/test_q8.py:28)
MS_REF = [1, 2, 5, 8, 9, 12, 15, 16, 17, 20, 24, 25, 31, 32, 33, 40, 48, 63, 64]


@pytest.fixture
def batch_invariant(dev):
    old = ops.set_config(batch_invariant=1)
    yield
    ops.set_config(**old)


@pytest.mark.parametrize("glu", [False, True])
@pytest.mark.parametrize("n,k", [(5120, 5120), (2048, 1280)])
def test_batch_invariant_rows(dev, batch_invariant, n, k, glu):
    """with batch_invariant set, every row of a decode call of m = 1..64 rows (qe_matmul_w4_ex: 16-row launches of the
    skinny kernel) has the same bits as that row decoded alone, plain and GLU (the reference's contract,
    skinny.cu:1-14; its test takes m up to 64, tests/test_q8.py:28)"""
    w, q, s = setup_w4(n, k, 1, seed=11 + n, glu=glu)
    xh = synth.x_host(64, k, seed=12)
    x = synth.to_dev(xh)
    alone = []
    for r in range(64):
        alone.append(synth.bits(ops.matmul_w4(w, x[r:r + 1], out_bf16=True)) if glu else
                     ops.matmul_w4(w, x[r:r + 1]).cpu().numpy().view(np.uint32))
    alone = np.concatenate(alone)
    for m in MS_REF:
        y = ops.matmul_w4(w, x[:m], out_bf16=glu)
        torch.cuda.synchronize()
        yb = synth.bits(y) if glu else y.cpu().numpy().view(np.uint32)
        assert np.array_equal(yb, alone[:m]), m
    if not glu:
        assert err_ratio(ops.matmul_w4(w, x).cpu().numpy(), matmul_f64(xh, exact_w4(q, s, n, k, 1))) <= 1e-4


def test_batch_invariant_w8(dev, batch_invariant):
    """the same for INT8 (per-channel W8): m = 1 runs the matrix-core kernel too"""
    n, k = 4096, 2048
    q8, s8 = synth.w8_host(n, k, seed=13, per_channel=True)
    w8 = ops.tile_w8(synth.to_dev(q8), synth.to_dev(s8, torch.float16), True)
    x = synth.to_dev(synth.x_host(16, k, seed=14))
    full = ops.gemv_w8(w8, x).cpu().numpy().view(np.uint32)
    for r in (0, 7, 15):
        y = ops.gemv_w8(w8, x[r:r + 1]).cpu().numpy().view(np.uint32)
        assert np.array_equal(y, full[r:r + 1]), r


def test_config_defaults_and_checks(dev):
    c = ops.get_config()
    assert c == {"skinny_min_m": 2, "w8_mfma_min_m": 0, "batch_invariant": 0, "gemm_tune": 0, "gemm_h16": 0}


def test_measurement_probes(dev):
    """the bench's measurement helpers: the shader clock is within gfx950's range, and the read probe runs on the
    m = 1 GEMV's launch shape without writing its sink (a 2^-32 chance per block)"""
    from qengine_amd.qe import lib
    mhz = float(lib().qe_clock_probe_mhz(ops._stream()))
    print(f"shader clock {mhz:.0f} MHz")
    assert 300.0 <= mhz <= 3500.0, mhz
    n, k = 1024, 5120
    q, s = synth.w4_dev(n, k, seed=3)
    w = ops.repack_w4(q, s)
    sink = torch.zeros(n // 16, dtype=torch.int32, device="cuda")
    call("qe_read_probe", w.q, n, k, sink, ops._stream())
    torch.cuda.synchronize()
    assert int((sink != 0).sum()) <= 1
