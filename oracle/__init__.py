"""CPU oracle of the weight-only quantized matmul path: numpy wrappers over liboracle.so (qe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker and the CPU baseline. The product (qengine_amd, include/) never imports, links or calls it.

Parity pins (each function is checked against something other than itself in tests/test_oracle.py):
  f32_to_bf16 / bf16_to_f32 / f16_to_f32  torch's dtype conversions (independent RNE / IEEE implementations)
  unpack_w4         the reference's torch unpack expression (tests/test_gemv.py:13-15) restated in numpy
  repack_w4         round trip through an independent decoder written from the PTX ISA m16n8k16 A-fragment
                    layout + the reference's nibble pairing (gemv.cu:25-36), bijection, known answers
  dequant_w4        closed form bf16_rn((u - 8) * s) in numpy/torch (tests/test_gemv.py:36)
  dequant_w4_f16    closed form fp16_rn((u - 8) * s) through torch's float -> half conversion
  matmul_bf16       numpy float64 matmul (|err| bound), brute force on tiny shapes
  glu_rows / glu    the reference's interleave closed form (tests/test_q8.py:75-79 interleave_ref) + torch silu
  quantize_w8       the reference's torch closed form (tests/test_w8.py:6-9)
  w8_pos / tile_w8  bijection + inverse map of src/tools/qe_w8q.cu:34-45 + A-fragment decoder
  moe_route         brute force sort with the tie rule (numpy lexsort) + softmax renormalisation
  moe_segment       invariants (counts, contiguity, every pair once, stable order) + numpy argsort(stable)
  q8_pos / repack_q8 the reference's own q8_layout.h (compiled into oracle/_ref when /root/reference is present)
                    for every position, the reference's unit test (tests/q8_layout_unit.cpp, built and run there),
                    bijection, known answers written from the layout comment (q8_layout.h:5-12)
  dequant_q8        closed form bf16_rn((u - 128) * s) in numpy
  moe_pack          records decoded back to the source rows with the independent fragment decoder
  moe_ref           an independent float64 torch composition of the layer (routing by lexsort, the reference test's
                    unpack, torch's silu), with planted mistakes (gate / up swapped, the routing weight inside the
                    silu, no renormalisation, ties to the higher index, a dropped expert) that it must reject
  xh_pos / xh_pack  the lane / k-step statement of the XH layout (gemv_h16.cuh:8-10) for every position, bijection
                    per 64-k chunk, torch's clamp + fp16 conversion for the values
  gemv_h16          exact on integer-valued inputs (equal to the float64 product), and elsewhere within the
                    closed-form bound of one fp16 rounding per 64-k chunk (step = 64) or per 16-k step (step = 16,
                    the reference's MMA accumulation) of the float64 product
  x_to_h            torch's float32 amax / division / product and fp16 conversion (an independent RNE
                    implementation), known answers (zero row, amax = 16)
  gemm_h            exact on integer-valued inputs (equal to the float64 product), and elsewhere within the
                    closed-form bound of one fp16 rounding per 64-k chunk (step = 64) of the float64 product;
                    step = 16 (the reference's per-MMA-step rounding) is the same code path as gemv_h16's, pinned there
  x_to_i8           the reference test's own torch emulation (tests/test_gemm_i8.py:52-61 quant_emul) restated in
                    torch, known answers (zero group, amax = 127 * 2^e)
  gemm_i8           float64 product of the dequantized int8 operands: brute force on tiny shapes
  rows_w8a8         brute force on tiny shapes in exact rational arithmetic (integer sums, one float32 rounding
                    of the product, one of the fused multiply-add, ties to even, written independently of libm's
                    fmaf), and the float64 product exactly on integer-valued inputs
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIBPATH = os.path.join(HERE, "liboracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIBPATH):
            build()
        _lib = ctypes.CDLL(_LIBPATH)
        f = _lib
        f.or_f32_to_bf16.restype = ctypes.c_uint16
        f.or_f32_to_bf16.argtypes = [ctypes.c_float]
        f.or_bf16_to_f32.restype = ctypes.c_float
        f.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        f.or_f16_to_f32.restype = ctypes.c_float
        f.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        f.or_w8_pos.restype = ctypes.c_size_t
        f.or_w8_pos.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        f.or_q8_pos.restype = ctypes.c_size_t
        f.or_q8_pos.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        f.or_silu_mul.restype = ctypes.c_float
        f.or_silu_mul.argtypes = [ctypes.c_float, ctypes.c_float]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


# ---------------------------------------------------------------- 16-bit floats
def f32_to_bf16(a):
    """float32 array -> bf16 bit patterns (uint16), round to nearest even."""
    a = _c(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def scale_to_f32(s, sdt):
    return f16_to_f32(s) if sdt else bf16_to_f32(s)


# ---------------------------------------------------------------- W4
def unpack_w4(q, n, k):
    """int32 [n][k/8] -> int8 w = u - 8, [n][k]"""
    q = _c(q, np.int32).reshape(n, k // 8)
    w = np.empty((n, k), np.int8)
    lib().or_unpack_w4(_p(q), n, k, _p(w))
    return w


def repack_w4(q, s, n, k):
    """compressed-tensors (q int32 [n][k/8], s uint16 [n][k/128]) -> W4 layout (uint32 [n*k/8], uint16 [n*k/128])"""
    q = _c(q, np.int32)
    s = _c(s, np.uint16)
    dq = np.empty(n * k // 8, np.uint32)
    ds = np.empty(n * (k // 128), np.uint16)
    lib().or_repack_w4(_p(q), _p(s), n, k, _p(dq), _p(ds))
    return dq, ds


def dequant_w4(q, s, n, k, sdt):
    """-> bf16 bits [n][k] of bf16_rn((u - 8) * s)"""
    q = _c(q, np.int32)
    s = _c(s, np.uint16)
    out = np.empty((n, k), np.uint16)
    lib().or_dequant_w4(_p(q), _p(s), n, k, int(sdt), _p(out))
    return out


def dequant_w4_f16(q, s, n, k):
    """-> float32 [n][k] of fp16_rn((u - 8) * s) (fp16 scales): the exact product in float32, rounded to fp16 (numpy's
    float32 -> float16 conversion rounds to nearest even)"""
    e = unpack_w4(q, n, k).astype(np.float32) * np.repeat(f16_to_f32(s), 128, axis=1)
    return e.astype(np.float16).astype(np.float32)


def glu_rows(q, s, n, k, bits=4):
    q = _c(q, np.int32)
    s = _c(s, np.uint16)
    wpr = k * bits // 32
    dq = np.empty((n, wpr), np.int32)
    ds = np.empty((n, k // 128), np.uint16)
    lib().or_glu_rows(_p(q), _p(s), n, k, wpr, _p(dq), _p(ds))
    return dq, ds


# ---------------------------------------------------------------- matmul
def matmul_bf16(x, w, nthreads=0):
    """x bf16 bits [m][k], w bf16 bits [n][k] -> fp32 [m][n] (fp32 accumulation)"""
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    lib().or_matmul_bf16(_p(x), _p(w), m, n, k, _p(y), int(nthreads))
    return y


def rows_w8a8(xq, sx, w, sw, per_channel, nthreads=0):
    """the reference's W8A8 row GEMM (k_rows_qt, src/flash/flash_pfq.cuh:520-651): xq int8 [m][k] in natural k
    order and sx float32 [m][k/128] from x_to_i8(x, 128) (k_x_to_r8's arithmetic), w int8 [n][k], sw float32
    [n][k/128] (per_channel: [n]) -> fp32 [m][n], per 128-k group in k order y = fma(rn(float(sum) sx), sw, y)"""
    xq = _c(xq, np.int8)
    sx = _c(sx, np.float32)
    w = _c(w, np.int8)
    sw = _c(sw, np.float32)
    m, k = xq.shape
    n = w.shape[0]
    assert k % 128 == 0 and w.shape[1] == k and sx.shape == (m, k // 128)
    assert sw.shape == ((n,) if per_channel else (n, k // 128))
    y = np.empty((m, n), np.float32)
    lib().or_rows_w8a8(_p(xq), _p(sx), _p(w), _p(sw), int(bool(per_channel)), m, n, k, _p(y), int(nthreads))
    return y


def glu_epilogue(y):
    """fp32 [m][n] product of a GLU-interleaved matrix -> bf16 bits [m][n/2]"""
    y = _c(y, np.float32)
    m, n = y.shape
    act = np.empty((m, n // 2), np.uint16)
    lib().or_glu_epilogue(_p(y), m, n, _p(act))
    return act


# ---------------------------------------------------------------- W8
def quantize_w8(w, n, k):
    """bf16 bits [n][k] -> (int8 [n][k], bf16 scales [n][k/128])"""
    w = _c(w, np.uint16)
    q = np.empty((n, k), np.int8)
    s = np.empty((n, k // 128), np.uint16)
    lib().or_quantize_w8(_p(w), n, k, _p(q), _p(s))
    return q, s


def w8_pos(row, c, k):
    return lib().or_w8_pos(row, c, k)


def tile_w8(q, s, n, k, per_channel):
    q = _c(q, np.int8)
    s = _c(s, np.uint16)
    dq = np.empty(n * k, np.uint8)
    ds = np.empty(n if per_channel else n * (k // 128), np.uint16)
    lib().or_tile_w8(_p(q), _p(s), n, k, int(per_channel), _p(dq), _p(ds))
    return dq, ds


def dequant_w8(q, s, n, k, per_channel, sdt):
    q = _c(q, np.int8)
    s = _c(s, np.uint16)
    out = np.empty((n, k), np.uint16)
    lib().or_dequant_w8(_p(q), _p(s), n, k, int(per_channel), int(sdt), _p(out))
    return out


# ---------------------------------------------------------------- Q8
def q8_pos(row, k, K):
    return lib().or_q8_pos(row, k, K)


def repack_q8(q, s, n, k):
    """compressed-tensors 8-bit int32 [n][k/4] (u = w + 128) + bf16 scales [n][k/128] -> (Q8 bytes [n*k],
    scales in the W4 layout)"""
    q = _c(q, np.int32)
    s = _c(s, np.uint16)
    dq = np.empty(n * k, np.uint8)
    ds = np.empty(n * (k // 128), np.uint16)
    lib().or_repack_q8(_p(q), _p(s), n, k, _p(dq), _p(ds))
    return dq, ds


def dequant_q8(q, s, n, k):
    """-> bf16 bits [n][k] of bf16_rn((u - 128) * s) from the compressed-tensors source"""
    q = _c(q, np.int32)
    s = _c(s, np.uint16)
    out = np.empty((n, k), np.uint16)
    lib().or_dequant_q8(_p(q), _p(s), n, k, _p(out))
    return out


# ---------------------------------------------------------------- MoE
def moe_route(logits, topk):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    sel = np.empty((T, topk), np.int32)
    w = np.empty((T, topk), np.float32)
    lib().or_moe_route(_p(logits), T, E, topk, _p(sel), _p(w))
    return sel, w


def moe_segment(sel, E):
    sel = _c(sel, np.int32)
    T, topk = sel.shape
    cnt = np.empty(E, np.int32)
    off = np.empty(E + 1, np.int32)
    lst = np.empty(T * topk, np.int32)
    inv = np.empty(T * topk, np.int32)
    lib().or_moe_segment(_p(sel), T, E, topk, _p(cnt), _p(off), _p(lst), _p(inv))
    return cnt, off, lst, inv


def silu_mul(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return (a / (np.float32(1) + np.exp(-a)) * b).astype(np.float32)


def moe_pack(gu_q, gu_s, dn_q, dn_s, E, H, I):
    """compressed-tensors experts -> the group records (uint8 bytes), restated from the reference loader
    (flash.cu:1555-1611): per (e, g) gather gate/up rows of group g, GLU-interleave, repack; gather down columns,
    repack. Record layout [gq][gs][dq][ds] (flash.h:203-218)."""
    ngrp = I // 128
    out = []
    for e in range(E):
        for g in range(ngrp):
            rows = np.concatenate([np.arange(g * 128, g * 128 + 128), I + np.arange(g * 128, g * 128 + 128)])
            q = gu_q[e][rows]
            s = gu_s[e][rows]
            qg, sg = glu_rows(q, s, 256, H)
            gq, gs = repack_w4(qg, sg, 256, H)
            dq_src = np.ascontiguousarray(dn_q[e][:, g * 16:(g + 1) * 16])
            ds_src = np.ascontiguousarray(dn_s[e][:, g:g + 1])
            dq, ds = repack_w4(dq_src, ds_src, H, 128)
            out += [gq.view(np.uint8), gs.view(np.uint8), dq.view(np.uint8), ds.view(np.uint8)]
    return np.concatenate(out)


def moe_ref(logits, x, gu_q, gu_s, dn_q, dn_s, topk, H, I, tokens=None, exact=False):
    """one MoE layer in float64: out[t] = sum_k w_k * down_e(silu(gate_e x) * up_e x) with (sel, w) from moe_route,
    on the weight operands the layer's kernels multiply: gate_up bf16_rn((u - 8) * s), down fp16_rn((u - 8) * s)
    (exact: the unrounded (u - 8) * s for both); no intermediate rounding; tokens: subset of rows (default all).
    Returns (out [len(tokens)][H], sel, w)."""
    sel, w = moe_route(logits, topk)
    T = logits.shape[0]
    tokens = np.arange(T) if tokens is None else np.asarray(tokens)
    xf = bf16_to_f32(x).astype(np.float64)
    cache = {}

    def deq(q, s, n, k, f16):
        if exact:
            return unpack_w4(q, n, k).astype(np.float64) * np.repeat(f16_to_f32(s), 128, axis=1)
        if f16:
            return dequant_w4_f16(q, s, n, k).astype(np.float64)
        return bf16_to_f32(dequant_w4(q, s, n, k, 1)).astype(np.float64)

    def expert(e):
        if e not in cache:
            cache[e] = (deq(gu_q[e], gu_s[e], 2 * I, H, False), deq(dn_q[e], dn_s[e], H, I, True))
        return cache[e]

    out = np.zeros((len(tokens), H))
    for r, t in enumerate(tokens):
        for k in range(topk):
            wgu, wdn = expert(int(sel[t, k]))
            gu = wgu @ xf[t]
            act = gu[:I] / (1 + np.exp(-gu[:I])) * gu[I:]
            out[r] += float(w[t, k]) * (wdn @ act)
    return out, sel, w


# ---------------------------------------------------------------- H16 (fp16-accumulate decode on XH activations)
def xh_pos(k):
    """column of activation k inside an XH row (reference src/kernels/gemv_h16.cuh:22-27): within each 64-k chunk
    the k bits b0..b5 move to b0 | b3<<1 | b4<<2 | b5<<3 | b1<<4 | b2<<5"""
    k = np.asarray(k, np.int64)
    return (k & ~63) | (k & 1) | ((k >> 2) & 14) | ((k & 6) << 3)


def to_xh(v):
    """fp32 values -> fp16 bits of clamp(v, -2047, 2047) / 16, round to nearest even (gemv_h16.cuh:28-30)"""
    c = np.clip(np.asarray(v, np.float32), np.float32(-2047), np.float32(2047)) * np.float32(0.0625)
    return c.astype(np.float16).view(np.uint16)


def xh_pack(x, ldxh=None):
    """bf16 bits [m][k] -> XH fp16 bits [m][ldxh] (gemv.cu:1530-1534 xh_pack); columns k..ldxh stay 0"""
    m, k = x.shape
    out = np.zeros((m, ldxh or k), np.uint16)
    out[:, xh_pos(np.arange(k))] = to_xh(bf16_to_f32(x))
    return out


def xh_values(xh, k):
    """XH fp16 bits [m][>= k] -> the stored values x / 16 in natural column order (float64)"""
    return np.ascontiguousarray(xh[:, xh_pos(np.arange(k))]).view(np.float16).astype(np.float64)


def gemv_h16(xv, w, s, wdiv=1, step=64):
    """the H16 decode arithmetic (gemv_h16.cuh:12-15 and xh_flush :59-67; Q8: gemv.cu:786-792): xv [m][k] the XH
    values (x / 16), w [n][k] the exact integer weights, s [n][k/128] the group scales (float). step = 64 (this
    build's kernels): every 64-k chunk's partial sum of xv * (w / wdiv) (wdiv = 16 for Q8) is formed exactly and
    rounded once to fp16; step = 16 (the reference's m16n8k16 fp16-accumulate MMA steps): the chunk's fp16 accumulator
    takes the exact sum of each 16-k step (k = 64 c + 16 j .. + 15) and is rounded to fp16 after every step. Then the
    chunk is added at scale * 16 * wdiv. Returns float64 [m][n]; the kernels add the flushed chunks in fp32."""
    xv = np.asarray(xv, np.float64)
    m, k = xv.shape
    wf = np.asarray(w, np.float64) / wdiv
    sf = np.asarray(s, np.float64) * (16.0 * wdiv)
    acc = np.zeros((m, wf.shape[0]))
    for c in range(k // 64):
        if step == 64:
            part = (xv[:, 64 * c:64 * c + 64] @ wf[:, 64 * c:64 * c + 64].T).astype(np.float16)
        else:
            part = np.zeros((m, wf.shape[0]), np.float16)
            for j in range(4):
                k0 = 64 * c + 16 * j
                part = (part.astype(np.float64) + xv[:, k0:k0 + 16] @ wf[:, k0:k0 + 16].T).astype(np.float16)
        acc += part.astype(np.float64) * sf[:, c // 2][None, :]
    return acc


# ---------------------------------------------------------------- fp16-accumulate prefill GEMM (gemm_h)
def x_to_h(x):
    """bf16 bits [t][k] -> (xh float64 [t][k], xs float32 [t]) of the reference's x_to_h_kernel (gemm.cu:262-289):
    xs = amax / 16 in fp32 (1 for a zero row), inv = fp32(1 / xs), xh = fp16_rn(fp32(x * inv))"""
    xf = bf16_to_f32(np.asarray(x, np.uint16))
    amax = np.abs(xf).max(axis=1)
    xs = np.where(amax > 0, amax / np.float32(16), np.float32(1)).astype(np.float32)
    inv = (np.float32(1) / xs).astype(np.float32)
    prod = (xf * inv[:, None]).astype(np.float32)
    return prod.astype(np.float16).astype(np.float64), xs


def gemm_h(xh, xs, w, s, step=64):
    """the fp16-accumulate prefill arithmetic (gemm.cu:236-461): xh [t][k] the fp16 activation values, xs [t] the
    token scales, w [n][k] the exact integer weights u - 8, s [n][k/128] the group scales (float). step = 64 (this
    build's kernel): every 64-k chunk's partial sum is formed exactly and rounded once to fp16; step = 16 (the
    reference's fp16-accumulate MMA steps): the chunk's fp16 accumulator is rounded after every 16-k step. Then the
    chunk is added at its group scale, and the token scale multiplies the sum. Returns float64 [t][n]."""
    xh = np.asarray(xh, np.float64)
    t, k = xh.shape
    sf = np.asarray(s, np.float64)
    acc = np.zeros((t, w.shape[0]))
    for c in range(k // 64):  # the weights are converted chunk by chunk (full-size matrices stay integer)
        if step == 64:
            part = (xh[:, 64 * c:64 * c + 64] @ np.asarray(w[:, 64 * c:64 * c + 64], np.float64).T).astype(np.float16)
        else:
            part = np.zeros((t, w.shape[0]), np.float16)
            for j in range(4):
                k0 = 64 * c + 16 * j
                part = (part.astype(np.float64) + xh[:, k0:k0 + 16] @ np.asarray(w[:, k0:k0 + 16], np.float64).T
                        ).astype(np.float16)
        acc += part.astype(np.float64) * sf[:, c // 2][None, :]
    return acc * np.asarray(xs, np.float64)[:, None]


# ---------------------------------------------------------------- W4A8 prefill GEMM (gemm_w4_i8)
def x_to_i8(x, G):
    """bf16 bits [t][k] -> (q int8 [t][k] in natural k order, sx float32 [t][k/G]) of the reference's x_to_i8_kernel
    (gemm.cu:540-594): per (token, G-group) amax; sx = bits(amax / 127) & ~3 in fp32 (1 for a zero group),
    inv = fp32(1 / sx) (0 for a zero group), q = rn(x * inv) clamped to [-127, 127]"""
    xf = bf16_to_f32(np.asarray(x, np.uint16))
    t, k = xf.shape
    xg = xf.reshape(t, k // G, G)
    amax = np.abs(xg).max(axis=2)
    sx = ((amax / np.float32(127)).astype(np.float32).view(np.uint32) & np.uint32(0xFFFFFFFC)).view(np.float32)
    sx = np.where(amax > 0, sx, np.float32(1)).astype(np.float32)
    inv = np.where(amax > 0, np.float32(1) / sx, np.float32(0)).astype(np.float32)
    prod = (xg * inv[:, :, None]).astype(np.float32)
    q = np.clip(np.rint(prod), -127, 127).astype(np.int8)
    return q.reshape(t, k), sx


def gemm_i8(q, sx, w, s, G):
    """the W4A8 product of the dequantized operands in float64: sum_k (q sx)[t][k] (w s)[n][k], q / sx from x_to_i8,
    w [n][k] the exact integer weights u - 8, s [n][k/128] the group scales (float); the reference's test
    emulation (tests/test_gemm_i8.py:52-61,124-129)"""
    t, k = q.shape
    xq = (np.asarray(q, np.float64).reshape(t, k // G, G) * np.asarray(sx, np.float64)[:, :, None]).reshape(t, k)
    out = np.zeros((t, w.shape[0]))
    sf = np.asarray(s, np.float64)
    for g in range(k // 128):  # the weights are converted group by group (full-size matrices stay integer)
        out += xq[:, 128 * g:128 * g + 128] @ (np.asarray(w[:, 128 * g:128 * g + 128], np.float64) * sf[:, g:g + 1]).T
    return out
