"""qe_moe_w4_noalloc (the allocation-free MoE layer, workspace = the library's per-device scratch array) against
qe_moe_w4 (caller workspace) through the C-ABI: bit-identical outputs on two calls in a row, the second with fewer
tokens, on the prefill path (T > 32) and the decode path (T <= 32)."""
import ctypes

import numpy as np
import pytest
import torch

from qengine_amd import call, lib, ops

pytestmark = pytest.mark.gpu


def _layer(dev, E, topk, H, I, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    gq = torch.randint(-2**31, 2**31 - 1, (E, 2 * I, H // 8), dtype=torch.int32, device=dev, generator=g)
    gs = (torch.randn(E, 2 * I, H // 128, device=dev, generator=g).abs() * 0.02).half()
    dq = torch.randint(-2**31, 2**31 - 1, (E, H, I // 8), dtype=torch.int32, device=dev, generator=g)
    ds = (torch.randn(E, H, I // 128, device=dev, generator=g).abs() * 0.02).half()
    return ops.MoE.pack(gq, gs, dq, ds, topk), g


def _run_noalloc(moe, lg, x, out_bf16):
    T = x.shape[0]
    out = torch.empty(T, moe.H, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=x.device)
    call("qe_moe_w4_noalloc", lg, x, moe.records, T, moe.E, moe.topk, moe.H, moe.I, out,
         ops.OUT_BF16 if out_bf16 else 0, ops._stream())
    return out


@pytest.mark.parametrize("out_bf16", [True, False])
def test_noalloc_equals_workspace_entry(dev, out_bf16):
    E, topk, H, I = 128, 10, 2048, 512
    moe, g = _layer(dev, E, topk, H, I, seed=71)
    lib().qe_moe_workspace_bytes.restype = ctypes.c_size_t
    for T in (40, 7):  # prefill path, then a smaller call on the decode path: the scratch keeps the first call's bytes
        assert lib().qe_moe_workspace_bytes(T, E, topk, H, I) <= 8 << 20
        lg = torch.randn(T, E, device=dev, generator=g)
        x = torch.randn(T, H, device=dev, generator=g).bfloat16()
        y_na = _run_noalloc(moe, lg, x, out_bf16)
        y_ws = moe(lg, x, out_bf16=out_bf16)
        torch.cuda.synchronize()
        a = y_na.view(torch.int16 if out_bf16 else torch.int32).cpu().numpy()
        b = y_ws.view(torch.int16 if out_bf16 else torch.int32).cpu().numpy()
        assert np.array_equal(a, b), T
        assert np.isfinite(y_na.float().cpu().numpy()).all()
