"""Prefill GEMM (bf16 MFMA on LDS-staged dequantized tiles) through the C-ABI vs the CPU oracle.

Gate (BASELINE): max|y - ref| <= 2e-2 * rms(ref), ref = the oracle's dequantize-then-matmul (weights dequantized
to bf16 as the reference does, bf16_rn((u - 8) * s), product in float64). That bf16 weight is exactly the operand
this kernel multiplies, so fp32 outputs are also held to 1e-4 * rms (fp32 sums only), far inside the reference's own
gate (tests/test_gemm.py:26-27, max|err| / max|ref| < 1e-2). Full BASELINE shapes are checked on sampled rows."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from qengine_amd import call, ops, synth
from test_gemv_gpu import (TOL, assert_bf16_close, assert_gate, assert_glu_close, assert_rn_of, err_ratio, exact_w4,
                           glu_act, matmul_f64, oracle_ref, oracle_ref_w8, out_f32)

pytestmark = pytest.mark.gpu


def setup(n, k, sdt, seed, glu=False):
    q, s = synth.w4_host(n, k, seed=seed, sdt=sdt)
    if glu:
        q, s = oracle.glu_rows(q, s, n, k)
    w = ops.repack_w4(synth.to_dev(q), synth.to_dev(s, torch.float16 if sdt else torch.bfloat16), glu=glu)
    return w, q, s


@pytest.mark.parametrize("n,k,t", [(128, 128, 1), (256, 512, 37), (512, 1024, 300), (384, 2048, 129),
                                   (1024, 5120, 256)])
@pytest.mark.parametrize("sdt", [0, 1])
def test_gemm_w4_parity(dev, n, k, t, sdt):
    w, q, s = setup(n, k, sdt, seed=n + k + t)
    xh = synth.x_host(t, k, seed=t)
    ref = oracle_ref(xh, q, s, n, k, sdt)
    x = synth.to_dev(xh)
    y32 = out_f32(ops.gemm_w4(w, x))
    assert err_ratio(y32, ref) <= 1e-4
    y16 = out_f32(ops.gemm_w4(w, x, out_bf16=True))
    assert_bf16_close(y16, ref)


def test_gemm_w4_glu(dev):
    n, k, t = 512, 1024, 77
    w, q, s = setup(n, k, 1, seed=5, glu=True)
    xh = synth.x_host(t, k, seed=6)
    act = glu_act(oracle.bf16_to_f32(xh).astype(np.float64)
                  @ oracle.bf16_to_f32(oracle.dequant_w4(q, s, n, k, 1)).astype(np.float64).T)
    y = out_f32(ops.gemm_w4(w, synth.to_dev(xh)))
    assert_glu_close(y, act, 1e-4)


@pytest.mark.parametrize("glu", [False, True])
def test_gemm_w4_strided_output(dev, glu):
    """outputs written into a wider matrix at an odd offset and row stride (the epilogue's scalar stores) equal the
    contiguous outputs (8- / 16-byte stores) bit for bit, for bf16, fp32 and GLU outputs"""
    n, k, t = 512, 1024, 70
    w, _, _ = setup(n, k, 1, seed=12, glu=glu)
    x = synth.to_dev(synth.x_host(t, k, seed=13))
    cols = n // 2 if glu else n
    for out_bf16 in ((True,) if glu else (False, True)):
        dt = torch.bfloat16 if (out_bf16 or glu) else torch.float32
        want = ops.gemm_w4(w, x, out_bf16=out_bf16)
        big = torch.full((t, cols + 7), float("nan"), dtype=dt, device=dev)
        got = ops.gemm_w4(w, x, out_bf16=out_bf16, y=big[:, 1:1 + cols])
        torch.cuda.synchronize()
        iv = torch.int16 if dt == torch.bfloat16 else torch.int32
        assert torch.equal(got.contiguous().view(iv), want.view(iv)), (glu, out_bf16)
        assert torch.isnan(big[:, 0]).all() and torch.isnan(big[:, 1 + cols:]).all()


def test_gemm_matches_gemv_rows(dev):
    """matmul dispatch: m <= 64 runs the decode kernels (here the one-pass kernel for 64 rows), from 65 rows the GEMM;
    both meet the gate on the same rows. The decode kernels multiply the exact weights (u - 8) * s, the GEMM their bf16 rounding (the reference's
    operand), so a row's result at m = 64 and m = 65 differs by at most the weight rounding:
    |dy| <= 2^-9 * sum_k |x_k (u_k - 8) s_k| (plus fp32 summation noise), checked element by element"""
    n, k = 1024, 2048
    w, q, s = setup(n, k, 1, seed=9)
    xh = synth.x_host(96, k, seed=10)
    x = synth.to_dev(xh)
    ref = oracle_ref(xh, q, s, n, k, 1)
    yg = out_f32(ops.matmul_w4(w, x))                       # GEMM (96 rows)
    y65 = out_f32(ops.matmul_w4(w, x[:65].contiguous()))    # GEMM (65 rows)
    y64 = out_f32(ops.matmul_w4(w, x[:64].contiguous()))    # decode (64 rows, one pass)
    assert err_ratio(yg, ref) <= 1e-4 and err_ratio(y64, ref[:64]) <= TOL
    assert err_ratio(y64, matmul_f64(xh[:64], exact_w4(q, s, n, k, 1))) <= 1e-4
    wabs = np.abs(exact_w4(q, s, n, k, 1)).astype(np.float64)
    bound = 2.0 ** -9 * (np.abs(oracle.bf16_to_f32(xh[:64]).astype(np.float64)) @ wabs.T)
    rms = np.sqrt(np.mean(ref ** 2))
    assert np.all(np.abs(y65[:64].astype(np.float64) - y64) <= bound + 1e-5 * rms)


def test_reference_named_gemm_hooks(dev):
    """qe_gemm_w4 / _t / _s (bf16 scales, fp32 out) and qe_gemm_set_out_bf16 (bf16 RN of the same sums)"""
    n, k, t = 256, 1024, 100
    w, q, s = setup(n, k, 0, seed=11)
    x = synth.to_dev(synth.x_host(t, k, seed=12))
    ref = ops.gemm_w4(w, x)
    y = torch.full((t, n), float("nan"), device=dev)
    call("qe_gemm_w4", w.q, w.s, n, k, x, y, t)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    # the tuned hook may choose another tile configuration: the same products, another fp32 summation order
    yt = torch.full((t, n), float("nan"), device=dev)
    call("qe_gemm_w4_t", w.q, w.s, n, k, x, yt, t)
    torch.cuda.synchronize()
    assert err_ratio(yt.cpu().numpy(), ref.cpu().numpy()) <= 1e-5
    call("qe_gemm_tune_clear")
    call("qe_gemm_set_out_bf16", 1)
    try:
        yb = torch.full((t, n), float("nan"), device=dev, dtype=torch.bfloat16)
        call("qe_gemm_w4", w.q, w.s, n, k, x, yb, t)
        torch.cuda.synchronize()
    finally:
        call("qe_gemm_set_out_bf16", 0)
    assert torch.equal(yb.view(torch.int16), ref.bfloat16().view(torch.int16))  # RN of the fp32 result, bit for bit


@pytest.mark.parametrize("n,k", [(17408, 5120), (5120, 17408)])
def test_gemm_w4_baseline_shapes_sampled(dev, n, k):
    """BASELINE config 2 (M = 8192) at full size; 48 sampled token rows checked against the oracle"""
    t = 8192
    w, q, s = setup(n, k, 1, seed=n)
    x = synth.x_dev(t, k, seed=3)
    y = ops.gemm_w4(w, x, out_bf16=True)
    rows = np.random.default_rng(4).choice(t, 48, replace=False)
    rows.sort()
    sel = torch.from_numpy(rows).to(dev)
    y = y[sel].contiguous()
    y32 = ops.gemm_w4(w, x)[sel].contiguous()
    torch.cuda.synchronize()
    xh = synth.bits(x[sel].contiguous())
    # the GEMM multiplies the reference's operand bf16_rn((u - 8) s): ref = that dequantization, product in float64
    ref = oracle_ref(xh, q, s, n, k, 1)
    assert_gate(y32.cpu().numpy(), ref, f"C2 n={n} k={k} fp32 out")
    assert_gate(out_f32(y), ref, f"C2 n={n} k={k} bf16 out")
    assert_rn_of(y, y32.cpu().numpy(), "C2")
    assert err_ratio(y32.cpu().numpy(), ref) <= 1e-4


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("n,k,t", [(256, 512, 33), (1024, 2048, 300)])
def test_gemm_w8_parity(dev, per_channel, n, k, t):
    q, s = synth.w8_host(n, k, seed=n + t, per_channel=per_channel)
    if not per_channel:
        s = s.reshape(n, k // 128)
    w = ops.tile_w8(synth.to_dev(q), synth.to_dev(s, torch.float16), per_channel)
    xh = synth.x_host(t, k, seed=t + 1)
    ref = oracle_ref_w8(xh, q, s, n, k, per_channel)
    y = out_f32(ops.gemm_w8(w, synth.to_dev(xh)))
    assert err_ratio(y, ref) <= 1e-4
    yb = out_f32(ops.gemm_w8(w, synth.to_dev(xh), out_bf16=True))
    assert_bf16_close(yb, ref)


def test_gemm_w8_baseline_shape_sampled(dev):
    """BASELINE config 3 at M = 4096 (K = 2048, N = 8192, per-channel fp16 scales), sampled rows"""
    n, k, t = 8192, 2048, 4096
    q, s = synth.w8_host(n, k, seed=77, per_channel=True)
    w = ops.tile_w8(synth.to_dev(q), synth.to_dev(s, torch.float16), True)
    x = synth.x_dev(t, k, seed=78)
    y = ops.gemm_w8(w, x, out_bf16=True)
    rows = np.sort(np.random.default_rng(5).choice(t, 48, replace=False))
    sel = torch.from_numpy(rows).to(dev)
    y = y[sel].contiguous()
    y32 = ops.gemm_w8(w, x)[sel].contiguous()
    torch.cuda.synchronize()
    ref = oracle_ref_w8(synth.bits(x[sel].contiguous()), q, s, n, k, True)
    # per-channel scales: max|y| ~ 20 rms, so the unrelaxed gate is on the fp32 output and the bf16 output is its RN
    assert_gate(y32.cpu().numpy(), ref, "C3 M=4096 W8A16 fp32 out")
    assert_rn_of(y, y32.cpu().numpy(), "C3 M=4096")
    assert_bf16_close(out_f32(y), ref)


# n = 40960, t = 512: 2 x 160 tiles of 256 x 256 on 256 CUs leave a last round of 64 tiles, which the split runs as
# 2 or 4 K ranges (stream-K of the tail); 256 x 128 tiles: 640, a tail of 128
SPLIT_SHAPE = (40960, 1024, 512)


@pytest.mark.parametrize("cfg,ks", [(0, 2), (0, 4), (1, 2)])
def test_gemm_split_tail(dev, cfg, ks):
    """the split of the last partial round: every output (split tiles and direct tiles) equals the unsplit GEMM to
    fp32 summation order (1e-5 * rms), fp32, bf16 and GLU outputs; sampled rows vs the oracle"""
    n, k, t = SPLIT_SHAPE
    w, q, s = setup(n, k, 1, seed=5)
    xh = synth.x_host(t, k, seed=6)
    x = synth.to_dev(xh)
    base, applied0 = ops.gemm_w4_choice(w, x, cfg, 1)
    y, applied = ops.gemm_w4_choice(w, x, cfg, ks)
    torch.cuda.synchronize()
    assert applied and not applied0
    b, yv = base.cpu().numpy(), y.cpu().numpy()
    assert err_ratio(yv, b) <= 1e-5
    rows = [0, 255, 256, 300, 511]  # the split tiles hold tokens 256..511
    ref = oracle_ref(xh[rows], q, s, n, k, 1)
    assert err_ratio(yv[rows], ref) <= 1e-4
    yb, _ = ops.gemm_w4_choice(w, x, cfg, ks, out_bf16=True)
    assert_bf16_close(out_f32(yb)[rows], ref)
    wg, qg, sg = setup(n, k, 1, seed=7, glu=True)
    ag, _ = ops.gemm_w4_choice(wg, x, cfg, ks)
    a1, _ = ops.gemm_w4_choice(wg, x, cfg, 1)
    torch.cuda.synchronize()
    act = glu_act(matmul_f64(xh[rows], oracle.bf16_to_f32(oracle.dequant_w4(qg, sg, n, k, 1))))
    assert_glu_close(out_f32(ag)[rows], act, 1e-4)
    # two bf16 roundings of fp32 sums that differ in summation order: at most one bf16 step (2^-7 relative) apart
    a1v, agv = out_f32(a1).astype(np.float64), out_f32(ag).astype(np.float64)
    assert np.all(np.abs(agv - a1v) <= 1e-5 * np.sqrt(np.mean(a1v ** 2)) + 2.0 ** -7 * np.abs(a1v))


def test_gemm_sk_maxparts(dev):
    """qe_gemm_set_sk_maxparts caps the split of the last partial round: on SPLIT_SHAPE the cost model splits it in 2
    (bits of the (0, 2) choice); with the cap at 1 the same call is the unsplit (0, 1) GEMM bit for bit, and the
    reference-named hook is honoured by qe_gemm_w4 too; cap 0 restores the split"""
    n, k, t = SPLIT_SHAPE
    w, q, s = setup(n, k, 0, seed=8)  # bf16 scales: the reference-named qe_gemm_w4 takes them
    x = synth.to_dev(synth.x_host(t, k, seed=9))
    call("qe_gemm_tune_clear")
    split, applied = ops.gemm_w4_choice(w, x, 0, 2)
    whole, _ = ops.gemm_w4_choice(w, x, 0, 1)
    assert applied
    try:
        y0 = ops.gemm_w4(w, x)
        call("qe_gemm_set_sk_maxparts", 1)
        y1 = ops.gemm_w4(w, x)
        yr = torch.empty(t, n, dtype=torch.float32, device=dev)
        call("qe_gemm_w4", w.q, w.s, n, k, x, yr, t)
        call("qe_gemm_set_sk_maxparts", 3)  # 2 or 3: a split in 2 stays allowed
        y3 = ops.gemm_w4(w, x)
    finally:
        call("qe_gemm_set_sk_maxparts", 0)
    y00 = ops.gemm_w4(w, x)
    torch.cuda.synchronize()
    iv = torch.int32
    assert torch.equal(y0.view(iv), split.view(iv)) and torch.equal(y00.view(iv), split.view(iv))
    assert torch.equal(y1.view(iv), whole.view(iv)) and torch.equal(yr.view(iv), whole.view(iv))
    assert torch.equal(y3.view(iv), split.view(iv))


def test_gemm_tuner_table_and_file(dev, tmp_path):
    """qe_gemm_w4_t times the candidates once per (shape, token bucket) and keeps the choice; with a tuning file the
    choice survives a cleared table (reloaded from the file) and the output is bit-identical"""
    from qengine_amd import lib
    lib().qe_gemm_tune_entries.restype = ctypes.c_int
    n, k, t = 2048, 1024, 300
    w, q, s = setup(n, k, 0, seed=9)
    xh = synth.x_host(t, k, seed=10)
    x = synth.to_dev(xh)
    path = str(tmp_path / "tune.txt")
    call("qe_gemm_tune_file", ctypes.c_char_p(path.encode()))
    call("qe_gemm_tune_clear")
    y = torch.empty(t, n, device=dev)
    call("qe_gemm_w4_t", w.q, w.s, n, k, x, y, t)
    torch.cuda.synchronize()
    assert lib().qe_gemm_tune_entries() == 1
    assert err_ratio(y.cpu().numpy(), oracle_ref(xh, q, s, n, k, 0)) <= 1e-4
    txt = open(path).read().splitlines()
    assert txt[0].startswith("qengine_amd gemm tune v1") and txt[1].startswith("device ") and len(txt) == 3
    call("qe_gemm_tune_clear")
    assert lib().qe_gemm_tune_entries() == 0
    call("qe_gemm_tune_file", ctypes.c_char_p(path.encode()))
    assert lib().qe_gemm_tune_entries() == 1
    y2 = torch.empty(t, n, device=dev)
    call("qe_gemm_w4_t", w.q, w.s, n, k, x, y2, t)
    torch.cuda.synchronize()
    assert lib().qe_gemm_tune_entries() == 1 and torch.equal(y.view(torch.int32), y2.view(torch.int32))
    call("qe_gemm_tune_file", ctypes.c_char_p(b""))
    call("qe_gemm_tune_clear")
