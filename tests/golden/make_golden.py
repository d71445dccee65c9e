"""Writes tests/golden/golden.npz: small frozen input/output vectors of the path (run from the repo root).

    python tests/golden/make_golden.py

Contents (all seeded; bit patterns stored as unsigned integers):
  * q8_pos_K{64,128}: byte positions of the Q8 layout for every (row, k) of a 16 x K tile, taken from the reference's
    own header (src/kernels/q8_layout.h:29-37) compiled into oracle/_ref/libq8ref.so by `make -C oracle ref` in a
    container where /root/reference exists. These pin the Q8 layout wherever the reference is absent.
  * w4_*: a 32 x 256 INT4 matrix in compressed-tensors form (q int32 [n][k/8], fp16 scales), its W4 repack (the
    layout of the reference's repack_w4, gemv.cu:515-549), its bf16 dequantization bf16_rn((u - 8) * s), three
    bf16 activation rows and their product against the dequantized weights in float64 (stored as float32), and the
    GLU interleave of the same matrix (gemv.cu:1151-1160).
  * w8_*: a 16 x 256 bf16 matrix, its RTN INT8 quantization (tools/quant_int8.py:78-99) and W8 tile
    (gemv.cu:1102-1113).
  * moe_*: router logits with planted ties, top-3 selection and weights (flash_kernels.cuh:4006-4089 tie rule:
    value desc, index asc) and the expert segmentation of the selection.
Everything except q8_pos comes from the oracle (oracle/), whose functions are pinned in tests/test_oracle.py
against independent checks; the fixture freezes those outputs so a later change to either the oracle or the HIP
path that alters them fails tests/test_golden.py.
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from qengine_amd import synth  # noqa: E402


def q8_table(K):
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libq8ref.so"))
    lib.ref_q8_pos.restype = ctypes.c_size_t
    lib.ref_q8_pos.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return np.array([[lib.ref_q8_pos(r, k, K) for k in range(K)] for r in range(16)], dtype=np.uint32)


def main():
    out = {}
    out["q8_pos_K64"] = q8_table(64)
    out["q8_pos_K128"] = q8_table(128)

    n, k = 32, 256
    q, s = synth.w4_host(n, k, seed=2024, sdt=1)
    dq, ds = oracle.repack_w4(q, s, n, k)
    wdq = oracle.dequant_w4(q, s, n, k, 1)
    xh = synth.x_host(3, k, seed=2025)
    y = oracle.bf16_to_f32(xh).astype(np.float64) @ oracle.bf16_to_f32(wdq).astype(np.float64).T
    gq, gs = oracle.glu_rows(q, s, n, k)
    out.update(w4_q=q.view(np.uint32), w4_s=s, w4_dq=dq, w4_ds=ds, w4_deq=wdq, w4_x=xh, w4_y=y.astype(np.float32),
               w4_glu_q=np.asarray(gq).view(np.uint32), w4_glu_s=np.asarray(gs))

    n8, k8 = 16, 256
    rng = np.random.default_rng(2026)
    wb = synth.np_bf16(rng.standard_normal((n8, k8)) * 0.02)
    q8, s8 = oracle.quantize_w8(wb, n8, k8)
    tq, ts = oracle.tile_w8(q8, s8, n8, k8, False)
    out.update(w8_w=wb, w8_q=q8.view(np.uint8), w8_s=s8, w8_tq=np.asarray(tq).view(np.uint8), w8_ts=np.asarray(ts))

    T, E, topk = 6, 16, 3
    lg = synth.logits_host(T, E, seed=2027)
    lg[1, 3] = lg[1, 7] = lg[1, 11] = 2.5  # three-way tie at the top: index order decides
    lg[4, :] = 0.0                          # all equal: experts 0, 1, 2
    sel, w = oracle.moe_route(lg, topk)
    seg = oracle.moe_segment(sel, E)
    out.update(moe_logits=lg, moe_sel=np.asarray(sel, np.int32), moe_w=np.asarray(w, np.float32))
    for i, a in enumerate(seg):
        out[f"moe_seg{i}"] = np.asarray(a)
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "golden.npz"), **out)
    print({k_: (v.shape, v.dtype.name) for k_, v in out.items()})


if __name__ == "__main__":
    main()
