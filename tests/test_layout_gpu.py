"""Load-time layout kernels on the GPU vs the CPU oracle: bit-exact (integer permutations, exact dequant)."""
import numpy as np
import pytest
import torch

import oracle
from qengine_amd import call, ops, synth

pytestmark = pytest.mark.gpu


def _w4_dev(q, s, sdt):
    return synth.to_dev(q), synth.to_dev(s, torch.float16 if sdt else torch.bfloat16)


@pytest.mark.parametrize("n,k", [(16, 128), (64, 512), (96, 1280), (2048, 5120)])
@pytest.mark.parametrize("sdt", [0, 1])
def test_repack_w4_bit_exact(dev, n, k, sdt):
    q, s = synth.w4_host(n, k, seed=n * 7 + k, sdt=sdt)
    dq_ref, ds_ref = oracle.repack_w4(q, s, n, k)
    qd, sd = _w4_dev(q, s, sdt)
    w = ops.repack_w4(qd, sd)
    torch.cuda.synchronize()
    assert np.array_equal(w.q.cpu().numpy().view(np.uint32), dq_ref)
    assert np.array_equal(synth.bits(w.s), ds_ref)


@pytest.mark.parametrize("n,k", [(16, 128), (96, 1280), (1024, 2048)])
@pytest.mark.parametrize("sdt", [0, 1])
def test_dequant_w4_bit_exact(dev, n, k, sdt):
    q, s = synth.w4_host(n, k, seed=n + 3 * k, sdt=sdt)
    qd, sd = _w4_dev(q, s, sdt)
    w = ops.repack_w4(qd, sd)
    out = ops.dequant_w4(w)
    torch.cuda.synchronize()
    assert np.array_equal(synth.bits(out), oracle.dequant_w4(q, s, n, k, sdt))


def test_dequant_w4_special_scales(dev):
    """fp16 subnormal / large scales and every nibble value: still bf16_rn((u - 8) * s) exactly"""
    n, k = 16, 128
    u = (np.arange(n)[:, None] * 3 + np.arange(k)[None, :]) % 16
    q = np.zeros((n, k // 8), np.uint32)
    for j in range(8):
        q |= u[:, j::8].astype(np.uint32) << np.uint32(4 * j)
    q = q.view(np.int32)
    s = np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x3555, 0x2E66, 0x8001, 0x0000, 0x1234, 0x4567,
                  0x0200, 0x3800, 0x5000, 0x6000, 0x7000], np.uint16).reshape(n, 1)
    qd, sd = _w4_dev(q, s, 1)
    out = ops.dequant_w4(ops.repack_w4(qd, sd))
    torch.cuda.synchronize()
    assert np.array_equal(synth.bits(out), oracle.dequant_w4(q, s, n, k, 1))


@pytest.mark.parametrize("bits", [4, 8])
def test_glu_rows_bit_exact(dev, bits):
    n, k = 64, 256
    rng = np.random.default_rng(bits)
    q = rng.integers(-2**31, 2**31 - 1, size=(n, k * bits // 32), dtype=np.int64).astype(np.int32)
    s = rng.integers(0, 65535, size=(n, k // 128), dtype=np.int64).astype(np.uint16)
    dq_ref, ds_ref = oracle.glu_rows(q, s, n, k, bits)
    dq, ds = ops.glu_rows(synth.to_dev(q), synth.to_dev(s), bits)
    torch.cuda.synchronize()
    assert np.array_equal(dq.cpu().numpy(), dq_ref)
    assert np.array_equal(synth.bits(ds), ds_ref)


@pytest.mark.parametrize("n,k", [(32, 256), (256, 2048)])
def test_quantize_w8_bit_exact(dev, n, k):
    rng = np.random.default_rng(n)
    wb = synth.np_bf16(rng.standard_normal((n, k)) * 0.02)
    wb[1, 128:256] = 0
    q_ref, s_ref = oracle.quantize_w8(wb, n, k)
    dq_ref, ds_ref = oracle.tile_w8(q_ref, s_ref, n, k, False)
    w = ops.quantize_w8(synth.to_dev(wb))
    torch.cuda.synchronize()
    assert np.array_equal(w.q.cpu().numpy(), dq_ref)
    assert np.array_equal(synth.bits(w.s), ds_ref)


@pytest.mark.parametrize("per_channel", [True, False])
def test_tile_and_dequant_w8_bit_exact(dev, per_channel):
    n, k = 64, 512
    q, s = synth.w8_host(n, k, seed=21, per_channel=per_channel)
    if not per_channel:
        s = s.reshape(n, k // 128)
    dq_ref, ds_ref = oracle.tile_w8(q, s, n, k, per_channel)
    w = ops.tile_w8(synth.to_dev(q), synth.to_dev(s, torch.float16), per_channel)
    deq = ops.dequant_w8(w)
    torch.cuda.synchronize()
    assert np.array_equal(w.q.cpu().numpy(), dq_ref)
    assert np.array_equal(synth.bits(w.s), ds_ref)
    assert np.array_equal(synth.bits(deq), oracle.dequant_w8(q, s, n, k, per_channel, 1))


def test_reference_named_repack_hook(dev):
    n, k = 32, 256
    q, s = synth.w4_host(n, k, seed=1, sdt=0)
    qd, sd = _w4_dev(q, s, 0)
    dq = torch.empty(n * k // 2, dtype=torch.uint8, device=dev)
    ds = torch.empty(n * k // 128, dtype=torch.bfloat16, device=dev)
    call("qe_repack_w4", qd, sd, n, k, dq, ds)
    torch.cuda.synchronize()
    dq_ref, ds_ref = oracle.repack_w4(q, s, n, k)
    assert np.array_equal(dq.cpu().numpy().view(np.uint32), dq_ref)
