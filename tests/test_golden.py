"""Committed golden vectors (tests/golden/golden.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every frozen vector exactly, and the Q8 positions frozen from the reference's own header
(q8_layout.h, compiled in oracle/_ref) match the oracle's restatement, so the Q8 layout stays pinned where the
reference is absent. GPU: the HIP path, through the C-ABI, reproduces the frozen repack, dequantization, GLU
interleave, INT8 quantize / tile, routing and segmentation bit for bit, and the frozen float64 product of the INT4
matrix within the BASELINE gate (2e-2 * rms) and its own arithmetic bound (1e-4 * rms against the product on the
unrounded weights, which the decode GEMV multiplies).
"""
import os

import numpy as np
import pytest

import oracle
from qengine_amd import synth

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))
N4, K4 = 32, 256
N8, K8 = 16, 256


def test_fixture_q8_positions_match_oracle():
    for K in (64, 128):
        tab = G[f"q8_pos_K{K}"]
        mine = np.array([[oracle.q8_pos(r, k, K) for k in range(K)] for r in range(16)], dtype=np.uint32)
        assert np.array_equal(tab, mine), K
        assert np.array_equal(np.sort(tab.ravel()), np.arange(16 * K))  # a permutation of the tile's bytes


def test_fixture_w4_oracle():
    q, s = G["w4_q"].view(np.int32), G["w4_s"]
    dq, ds = oracle.repack_w4(q, s, N4, K4)
    assert np.array_equal(dq, G["w4_dq"]) and np.array_equal(ds, G["w4_ds"])
    assert np.array_equal(oracle.dequant_w4(q, s, N4, K4, 1), G["w4_deq"])
    gq, gs = oracle.glu_rows(q, s, N4, K4)
    assert np.array_equal(np.asarray(gq).view(np.uint32), G["w4_glu_q"]) and np.array_equal(gs, G["w4_glu_s"])
    y = oracle.matmul_bf16(G["w4_x"], G["w4_deq"])
    ref = G["w4_y"].astype(np.float64)
    assert np.abs(y - ref).max() <= 1e-5 * np.sqrt(np.mean(ref ** 2))


def test_fixture_w8_oracle():
    q, s = oracle.quantize_w8(G["w8_w"], N8, K8)
    assert np.array_equal(q.view(np.uint8), G["w8_q"]) and np.array_equal(s, G["w8_s"])
    tq, ts = oracle.tile_w8(q, s, N8, K8, False)
    assert np.array_equal(np.asarray(tq), G["w8_tq"]) and np.array_equal(np.asarray(ts), G["w8_ts"])


def test_fixture_moe_oracle():
    sel, w = oracle.moe_route(G["moe_logits"], 3)
    assert np.array_equal(sel, G["moe_sel"]) and np.array_equal(w, G["moe_w"])
    assert list(sel[1]) == [3, 7, 11] and list(sel[4]) == [0, 1, 2]  # the planted ties: lower index first
    for i, a in enumerate(oracle.moe_segment(sel, 16)):
        assert np.array_equal(a, G[f"moe_seg{i}"]), i


@pytest.mark.gpu
def test_fixture_hip_path(dev):
    import torch
    from qengine_amd import ops
    q, s = G["w4_q"].view(np.int32), G["w4_s"]
    w = ops.repack_w4(synth.to_dev(q), synth.to_dev(s, torch.float16))
    torch.cuda.synchronize()
    assert np.array_equal(w.q.cpu().numpy().view(np.uint32), G["w4_dq"])
    assert np.array_equal(synth.bits(w.s), G["w4_ds"])
    assert np.array_equal(synth.bits(ops.dequant_w4(w)), G["w4_deq"])
    gq, gs = ops.glu_rows(synth.to_dev(q), synth.to_dev(s, torch.float16))
    torch.cuda.synchronize()
    assert np.array_equal(gq.cpu().numpy().view(np.uint32), G["w4_glu_q"]) and np.array_equal(synth.bits(gs), G["w4_glu_s"])
    # the product: decode GEMV per row count and the prefill GEMM
    ref = G["w4_y"].astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    exact = oracle.bf16_to_f32(G["w4_x"]).astype(np.float64) @ (
        oracle.unpack_w4(q, N4, K4).astype(np.float64) * np.repeat(oracle.f16_to_f32(s), 128, axis=1)).T
    x = synth.to_dev(G["w4_x"])
    for m in (1, 2, 3):
        y = ops.gemv_w4(w, x[:m]).cpu().numpy()
        assert np.abs(y - ref[:m]).max() <= 2e-2 * rms, m
        assert np.abs(y - exact[:m]).max() <= 1e-4 * rms, m
    c = ops.gemm_w4(w, x).cpu().numpy()
    assert np.abs(c - ref).max() <= 1e-4 * rms  # the GEMM multiplies the bf16-dequantized weights, as the fixture
    # INT8
    w8 = ops.quantize_w8(synth.to_dev(G["w8_w"]))
    torch.cuda.synchronize()
    assert np.array_equal(w8.q.cpu().numpy(), G["w8_tq"]) and np.array_equal(synth.bits(w8.s), G["w8_ts"])
    # routing and segmentation
    sel, wt = ops.moe_route(torch.from_numpy(G["moe_logits"]).to(dev), 3)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), G["moe_sel"])
    assert np.allclose(wt.cpu().numpy(), G["moe_w"], rtol=2e-6, atol=1e-7)
    seg = ops.moe_segment(sel, wt, 16, 64)
    torch.cuda.synchronize()
    assert np.array_equal(seg["off"].cpu().numpy(), G["moe_seg1"])
    assert np.array_equal(seg["slot_pair"].cpu().numpy(), G["moe_seg2"])
    assert np.array_equal(seg["inv"].cpu().numpy(), G["moe_seg3"])
