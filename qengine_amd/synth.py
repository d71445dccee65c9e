"""Seeded synthetic inputs in the BASELINE distributions (numpy on the host, torch on the device).

W4: int32 words of 8 uniform nibbles u in [0, 15] (zero point 8), fp16 scales |N(0,1)| * 0.02 per (row, 128-k
group). INT8: w uniform in [-127, 127], fp16 per-row scales |N(0,1)| * 0.005. x: bf16 N(0,1). Router logits:
fp32 N(0,1). The reference's own tests draw the same packed words (tests/test_gemm.py:10).
"""
import numpy as np
import torch


def np_bf16(a):
    """float32 -> bf16 bit patterns (round to nearest even) as uint16"""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def w4_host(n, k, seed, sdt=1, scale=0.02):
    """-> (q int32 [n][k/8], s uint16 [n][k/128]); sdt 1: fp16 scales, 0: bf16"""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    sf = (np.abs(rng.standard_normal((n, k // 128))) * scale).astype(np.float32)
    s = sf.astype(np.float16).view(np.uint16) if sdt else np_bf16(sf)
    return q, s


def x_host(m, k, seed):
    rng = np.random.default_rng(seed)
    return np_bf16(rng.standard_normal((m, k)).astype(np.float32)).reshape(m, k)


def w8_host(n, k, seed, per_channel=True, scale=0.005):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int32).astype(np.int8)
    shape = (n,) if per_channel else (n, k // 128)
    s = (np.abs(rng.standard_normal(shape)) * scale).astype(np.float16).view(np.uint16)
    return q, s


def logits_host(t, e, seed):
    return np.random.default_rng(seed).standard_normal((t, e)).astype(np.float32)


def to_dev(a, dtype=None, device="cuda"):
    """numpy array -> torch device tensor; uint16 bit patterns become `dtype` (torch.bfloat16 / float16)"""
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16).copy())
        t = t.view(dtype if dtype is not None else torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(device)


def bits(t):
    """torch 16-bit tensor -> numpy uint16 bit patterns"""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ---- device-side generation for full-size benchmarks (torch generator, seeded)
def w4_dev(n, k, seed, device="cuda", sdt_f16=True):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    q = torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32, device=device, generator=g)
    s = (torch.randn(n, k // 128, device=device, generator=g).abs() * 0.02)
    s = s.half() if sdt_f16 else s.bfloat16()
    return q, s


def x_dev(m, k, seed, device="cuda"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(m, k, device=device, generator=g).bfloat16()


def moe_host(E, H, I, seed):
    """experts in compressed-tensors form: gate_up int32 [E][2I][H/8] + fp16 scales [E][2I][H/128], down int32
    [E][H][I/8] + fp16 [E][H][I/128] (BASELINE: uniform nibbles, scales |N(0,1)| * 0.02)"""
    rng = np.random.default_rng(seed)
    gq = rng.integers(0, 2**32, size=(E, 2 * I, H // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    gs = (np.abs(rng.standard_normal((E, 2 * I, H // 128))) * 0.02).astype(np.float16).view(np.uint16)
    dq = rng.integers(0, 2**32, size=(E, H, I // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    ds = (np.abs(rng.standard_normal((E, H, I // 128))) * 0.02).astype(np.float16).view(np.uint16)
    return gq, gs, dq, ds
