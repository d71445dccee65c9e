"""Pins of the CPU oracle (oracle/qe_oracle.c) against checks that do not restate its own formulas:
library dtype conversions, the PTX ISA mma.m16n8k16 A-fragment table, hand-computed known answers, numpy
float64 matmul, brute-force ranking, invariants. CPU only."""
import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

import oracle
from qengine_amd import synth


# ------------------------------------------------------------------ 16-bit floats vs torch
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.4e38, 1e-40, np.inf, -np.inf],
                                 np.float32)]).astype(np.float32)
    ref = torch.from_numpy(a).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(a), ref)
    lib = oracle.lib()
    for v in a[:500]:
        assert lib.or_f32_to_bf16(float(v)) == torch.tensor([v]).bfloat16().view(torch.int16).numpy().view(np.uint16)[0]


def test_f16_decode_matches_numpy_all_patterns():
    lib = oracle.lib()
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = pats.view(np.float16).astype(np.float32)
    got = np.array([lib.or_f16_to_f32(int(p)) for p in pats[::7]], np.float32)
    r = ref[::7]
    ok = (got == r) | (np.isnan(got) & np.isnan(r))
    assert ok.all()


# ------------------------------------------------------------------ W4 format
def _ptx_a_fragment(e, lane):
    """(row, col) of element e (0..7) of the m16n8k16 .bf16 A fragment held by `lane` (PTX ISA, 'Matrix
    Fragments for mma.m16n8k16 with floating point type': a0,a1 row g; a2,a3 row g+8; a4,a5 row g col+8; a6,a7
    row g+8 col+8; col = 2 * (lane % 4) + (e & 1))"""
    g, t = lane // 4, lane % 4
    row = g + (8 if e in (2, 3, 6, 7) else 0)
    col = 2 * t + (e & 1) + (8 if e >= 4 else 0)
    return row, col


def _decode_w4_fragments(dq, n, k):
    """Independent decoder of the W4 layout: word (r, c, lane, kstep) is the A fragment of k-step `kstep`;
    register j of dequant_w4 (reference gemv.cu:25-36) holds nibble j (low half) and nibble j + 4 (high half),
    i.e. fragment element e = 2 j + hi comes from nibble slot j + 4 hi."""
    u = np.empty((n, k), np.int16)
    words = dq.reshape(n // 16, k // 64, 32, 4)
    for e in range(8):
        slot = (e >> 1) + 4 * (e & 1)
        nib = ((words >> np.uint32(4 * slot)) & np.uint32(15)).astype(np.int16)  # [r][c][lane][kstep]
        for lane in range(32):
            row, col = _ptx_a_fragment(e, lane)
            for ks in range(4):
                u[row::16, col + 16 * ks::64][: n // 16] = nib[:, :, lane, ks]
    return u


@pytest.mark.parametrize("n,k", [(16, 128), (32, 256), (48, 384)])
def test_repack_w4_round_trip_through_ptx_decoder(n, k):
    q, s = synth.w4_host(n, k, seed=n + k)
    dq, ds = oracle.repack_w4(q, s, n, k)
    u = _decode_w4_fragments(dq, n, k)
    assert np.array_equal(u - 8, oracle.unpack_w4(q, n, k))
    # scales: [n/16][G][16], row-in-tile fastest
    G = k // 128
    assert np.array_equal(ds.reshape(n // 16, G, 16).transpose(0, 2, 1).reshape(n, G), s)


def test_repack_w4_known_answer():
    """u(row, k) = (row + k) % 16 on one 16 x 128 tile: the first word (lane 0, k-step 0) holds, LSB first,
    (0,0)=0 (8,0)=8 (0,8)=8 (8,8)=0 (0,1)=1 (8,1)=9 (0,9)=9 (8,9)=1 -> 0x19910880 (slot order of the reference
    comment gemv.cu:532-537, computed by hand)."""
    n, k = 16, 128
    u = (np.arange(n)[:, None] + np.arange(k)[None, :]) % 16
    q = np.zeros((n, k // 8), np.uint32)
    for j in range(8):
        q |= u[:, j::8].astype(np.uint32) << np.uint32(4 * j)
    s = np.ones((n, 1), np.uint16)
    dq, _ = oracle.repack_w4(q.view(np.int32), s, n, k)
    assert dq[0] == 0x19910880
    # lane 5 (g = 1, t = 1), k-step 2: row 1, k0 = 32 + 2 = 34: (1,34)=3 (9,34)=11 (1,42)=11 (9,42)=3 (1,35)=4
    # (9,35)=12 (1,43)=12 (9,43)=4 -> 0x4CC43BB3
    assert dq[5 * 4 + 2] == 0x4CC43BB3


def test_repack_w4_is_a_bijection():
    n, k = 32, 256
    # every source nibble position gets a distinct 12-bit id split over three matrices; decode must invert
    ids = np.arange(n * k).reshape(n, k)
    for part in range(3):
        u = (ids >> (4 * part)) & 15
        q = np.zeros((n, k // 8), np.uint32)
        for j in range(8):
            q |= u[:, j::8].astype(np.uint32) << np.uint32(4 * j)
        dq, _ = oracle.repack_w4(q.view(np.int32), np.zeros((n, 2), np.uint16), n, k)
        assert np.array_equal(_decode_w4_fragments(dq, n, k), u)


def test_unpack_matches_reference_expression():
    """reference tests/test_gemv.py:13-15: ((wp[..., None] >> arange(0, 32, 4)) & 15) - 8"""
    n, k = 32, 256
    q, _ = synth.w4_host(n, k, seed=3)
    wp = torch.from_numpy(q)
    ref = (((wp.unsqueeze(-1) >> torch.arange(0, 32, 4, dtype=torch.int32)) & 15).reshape(n, k) - 8).numpy()
    assert np.array_equal(oracle.unpack_w4(q, n, k), ref.astype(np.int8))


@pytest.mark.parametrize("sdt", [0, 1])
def test_dequant_w4_closed_form(sdt):
    """bf16_rn((u - 8) * s) through torch: (unpack * s.repeat_interleave(128)).bfloat16() (test_gemv.py:36)"""
    n, k = 48, 384
    q, s = synth.w4_host(n, k, seed=5, sdt=sdt)
    w = torch.from_numpy(oracle.unpack_w4(q, n, k).astype(np.float32))
    sf = torch.from_numpy(oracle.scale_to_f32(s, sdt)).repeat_interleave(128, dim=1)
    ref = (w * sf).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.dequant_w4(q, s, n, k, sdt), ref)


def test_dequant_w4_f16_closed_form():
    """fp16_rn((u - 8) * s) (the MoE down operand) through torch: (unpack * s.repeat_interleave(128)).half(), with
    tiny scales (fp16 subnormal products) and large ones"""
    n, k = 48, 384
    q, s = synth.w4_host(n, k, seed=6, sdt=1)
    s[0, :] = np.array([1e-6], np.float16).view(np.uint16)[0]
    s[1, :] = np.array([4000.0], np.float16).view(np.uint16)[0]
    w = torch.from_numpy(oracle.unpack_w4(q, n, k).astype(np.float32))
    sf = torch.from_numpy(oracle.f16_to_f32(s)).repeat_interleave(128, dim=1)
    ref = (w * sf).half().float().numpy()
    got = oracle.dequant_w4_f16(q, s, n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_glu_rows_matches_interleave_closed_form():
    """reference tests/test_q8.py:75-79: stack([gate.reshape(-1, 8, k), up.reshape(-1, 8, k)], 1)"""
    n, k = 64, 256
    q, s = synth.w4_host(n, k, seed=7)
    dq, ds = oracle.glu_rows(q, s, n, k)
    qt = torch.from_numpy(q)
    ref = torch.stack([qt[: n // 2].reshape(-1, 8, k // 8), qt[n // 2:].reshape(-1, 8, k // 8)], 1).reshape(n, -1)
    assert np.array_equal(dq, ref.numpy())
    st = torch.from_numpy(s.view(np.int16))
    refs = torch.stack([st[: n // 2].reshape(-1, 8, 2), st[n // 2:].reshape(-1, 8, 2)], 1).reshape(n, -1)
    assert np.array_equal(ds.view(np.int16), refs.numpy())


def test_glu_epilogue_matches_torch_silu():
    rng = np.random.default_rng(1)
    y = rng.standard_normal((3, 64)).astype(np.float32) * 4
    act = oracle.bf16_to_f32(oracle.glu_epilogue(y))
    yt = torch.from_numpy(y).double().reshape(3, 4, 2, 8)
    ref = (torch.nn.functional.silu(yt[:, :, 0]) * yt[:, :, 1]).reshape(3, 32).numpy()
    assert np.allclose(act, ref, rtol=2 ** -8, atol=1e-6)


# ------------------------------------------------------------------ matmul
def test_matmul_bf16_vs_numpy_f64():
    rng = np.random.default_rng(2)
    m, n, k = 5, 48, 640
    x = synth.np_bf16(rng.standard_normal((m, k)))
    w = synth.np_bf16(rng.standard_normal((n, k)) * 0.05)
    y = oracle.matmul_bf16(x, w)
    xf, wf = oracle.bf16_to_f32(x).astype(np.float64), oracle.bf16_to_f32(w).astype(np.float64)
    ref = xf @ wf.T
    bound = k * 2 ** -23 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(y - ref) <= bound)


def test_matmul_bf16_brute_force_tiny():
    x = synth.np_bf16(np.array([[1.0, 2.0, -3.0, 0.5]], np.float32))
    w = synth.np_bf16(np.array([[1.0, 1.0, 1.0, 1.0], [0.25, -1.0, 2.0, 4.0]], np.float32))
    assert np.array_equal(oracle.matmul_bf16(x, w), np.array([[0.5, -5.75]], np.float32))


# ------------------------------------------------------------------ W8
def test_quantize_w8_matches_reference_torch_expression():
    """reference tests/test_w8.py:6-9"""
    n, k = 32, 256
    rng = np.random.default_rng(4)
    wb = synth.np_bf16(rng.standard_normal((n, k)) * 0.02)
    wb[3, :128] = 0  # an all-zero group (scale 0)
    q, s = oracle.quantize_w8(wb, n, k)
    g = torch.from_numpy(oracle.bf16_to_f32(wb)).view(n, k // 128, 128)
    sc = (g.abs().amax(-1) / 127).bfloat16()
    scf = sc.float()
    qref = torch.clamp(torch.round(g / torch.where(scf > 0, scf, 1).unsqueeze(-1)), -127, 127)
    assert np.array_equal(q, qref.reshape(n, k).numpy().astype(np.int8))
    assert np.array_equal(s, sc.view(torch.int16).numpy().view(np.uint16))


def _decode_w8_fragments(dq, n, k):
    """16-byte record of lane `ln` in slab (rt, sl): bytes 8 hs + e are elements a_e of the k-step hs fragment
    (reference gemv.cu:700-703 builds a0a1 / a2a3 from bytes 0-1 / 2-3 of each half), PTX A-fragment table."""
    out = np.empty((n, k), np.int8)
    rec = dq.view(np.int8).reshape(n // 16, k // 32, 32, 16)
    for lane in range(32):
        for hs in range(2):
            for e in range(8):
                row, col = _ptx_a_fragment(e, lane)
                out[row::16, 16 * hs + col::32][: n // 16] = rec[:, :, lane, 8 * hs + e]
    return out


@pytest.mark.parametrize("per_channel", [False, True])
def test_tile_w8_round_trip_through_ptx_decoder(per_channel):
    n, k = 32, 256
    q, s = synth.w8_host(n, k, seed=9, per_channel=per_channel)
    if not per_channel:
        s = s.reshape(n, k // 128)
    dq, ds = oracle.tile_w8(q, s, n, k, per_channel)
    assert np.array_equal(_decode_w8_fragments(dq, n, k), q)
    if per_channel:
        assert np.array_equal(ds, s)
    else:
        assert np.array_equal(ds.reshape(n // 16, 2, 16).transpose(0, 2, 1).reshape(n, 2), s)
    pos = {oracle.w8_pos(r, c, k) for r in range(n) for c in range(k)}
    assert len(pos) == n * k and max(pos) == n * k - 1


@pytest.mark.parametrize("per_channel", [False, True])
def test_dequant_w8_closed_form(per_channel):
    n, k = 32, 256
    q, s = synth.w8_host(n, k, seed=10, per_channel=per_channel)
    sf = oracle.f16_to_f32(s)
    sf = sf[:, None] if per_channel else np.repeat(sf.reshape(n, k // 128), 128, axis=1)
    ref = torch.from_numpy(q.astype(np.float32) * sf).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.dequant_w8(q, s, n, k, per_channel, 1), ref)


# ------------------------------------------------------------------ MoE
def test_moe_route_brute_force_with_ties():
    T, E, topk = 7, 64, 10
    lg = synth.logits_host(T, E, seed=11)
    lg[2, 5] = lg[2, 9] = lg[2, 40] = 3.0  # ties: lower index first
    lg[4, :] = 0.0                         # all equal: experts 0..9
    sel, w = oracle.moe_route(lg, topk)
    for t in range(T):
        order = np.lexsort((np.arange(E), -lg[t]))[:topk]
        assert np.array_equal(sel[t], order)
        ex = np.exp(lg[t, order].astype(np.float64) - lg[t, order[0]])
        assert np.allclose(w[t], ex / ex.sum(), rtol=1e-6)
        # equivalently the softmax over all E renormalised over the selection
        p = np.exp(lg[t].astype(np.float64) - lg[t].max())
        p /= p.sum()
        assert np.allclose(w[t], p[order] / p[order].sum(), rtol=1e-6)
    assert np.array_equal(sel[4], np.arange(10))
    assert list(sel[2][:3]) == [5, 9, 40]


def test_moe_segment_invariants():
    T, E, topk = 33, 40, 6
    sel, _ = oracle.moe_route(synth.logits_host(T, E, seed=12), topk)
    cnt, off, lst, inv = oracle.moe_segment(sel, E)
    flat = sel.ravel()
    assert cnt.sum() == T * topk and np.array_equal(cnt, np.bincount(flat, minlength=E))
    assert off[0] == 0 and np.array_equal(np.diff(off), cnt)
    assert np.array_equal(np.sort(lst), np.arange(T * topk))          # every pair exactly once
    assert np.array_equal(lst, np.argsort(flat, kind="stable"))       # expert-ordered, stable inside an expert
    assert np.array_equal(inv[lst], np.arange(T * topk))              # inverse map
    for e in range(E):
        assert np.all(flat[lst[off[e]:off[e + 1]]] == e)


def test_moe_pack_decodes_to_source_rows():
    """group record (e, g) (reference flash.h:203-218, loader flash.cu:1555-1611) decoded with the independent
    fragment decoder: gq rows = GLU tile order of gate rows [128g, 128g+128) and up rows I + [128g, 128g+128),
    gs their scales; dq = down columns [128g, 128g+128) of all H rows, ds the matching scale column"""
    E, H, I = 2, 256, 256
    gq, gs, dq, ds = synth.moe_host(E, H, I, seed=4)
    rec = oracle.moe_pack(gq, gs, dq, ds, E, H, I)
    sizes = [256 * H // 2, 256 * (H // 128) * 2, H * 64, H * 2]
    assert rec.size == E * (I // 128) * sum(sizes)
    pos = 0
    for e in range(E):
        for g in range(I // 128):
            parts = []
            for sz in sizes:
                parts.append(rec[pos:pos + sz])
                pos += sz
            u = _decode_w4_fragments(parts[0].view(np.uint32), 256, H)
            s = parts[1].view(np.uint16).reshape(16, H // 128, 16).transpose(0, 2, 1).reshape(256, H // 128)
            src_u = oracle.unpack_w4(gq[e], 2 * I, H) + 8
            for dr in range(256):  # GLU tile order: per 16 rows 8 gate + 8 up
                t, j = dr // 16, dr % 16
                sr = 128 * g + 8 * t + j if j < 8 else I + 128 * g + 8 * t + (j - 8)
                assert np.array_equal(u[dr], src_u[sr]) and np.array_equal(s[dr], gs[e][sr])
            ud = _decode_w4_fragments(parts[2].view(np.uint32), H, 128)
            assert np.array_equal(ud, oracle.unpack_w4(dq[e], H, I)[:, 128 * g:128 * g + 128] + 8)
            assert np.array_equal(parts[3].view(np.uint16), ds[e][:, g])


def _moe_layer_torch(lg, xh, gq, gs, dq, ds, topk, H, I, plant=None):
    """one MoE layer composed independently of the oracle, in float64 torch:
      * routing: numpy lexsort on (-logit, expert index) (value desc, index asc: flash_kernels.cuh:4006-4089), weights
        softmax(logits) renormalised over the selection;
      * experts: the reference test's unpack ((q >> 4 j) & 15) - 8 (tests/test_gemv.py:13-15) times the fp16 group
        scale, rounded by torch to bf16 for gate_up (tests/test_gemv.py:36) and to fp16 for down (the operands the
        layer's kernels multiply); rows [0, I) of gate_up are the gate, [I, 2I) the up (the loader's "gate rows, then
        up rows", flash.cu:1564-1565);
      * out[t] = sum_k w_k * W_down (silu(W_gate x) * (W_up x)) (the routing weight scales the activation,
        flash_kernels.cuh:6185; down is linear, so that equals scaling the expert output).
    plant: a deliberate mistake, to show that the comparison can fail: "swap" (silu on the up half), "w_in_silu"
    (silu(w gate) up), "no_renorm" (softmax over all experts, not renormalised), "ties_high" (ties broken by the
    higher index), "drop_k" (the last selected expert left out)."""
    import torch.nn.functional as F
    T, E = lg.shape
    x = torch.from_numpy(oracle.bf16_to_f32(xh).astype(np.float64))

    def deq(q, s, n, k, half=False):
        wp = torch.from_numpy(q)
        u = ((wp.unsqueeze(-1) >> torch.arange(0, 32, 4, dtype=torch.int32)) & 15).reshape(n, k) - 8
        sf = torch.from_numpy(s.view(np.float16).astype(np.float32)).repeat_interleave(128, dim=1)
        w = u.float() * sf
        return (w.half() if half else w.bfloat16()).double()

    out = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        idx = np.arange(E)
        order = np.lexsort((E - idx if plant == "ties_high" else idx, -lg[t].astype(np.float64)))[:topk]
        p = np.exp(lg[t].astype(np.float64) - lg[t].max())
        p /= p.sum()
        wk = p[order] if plant == "no_renorm" else p[order] / p[order].sum()
        for j, e in enumerate(order[:topk - 1] if plant == "drop_k" else order):
            wgu = deq(gq[e], gs[e], 2 * I, H)
            gate, up = wgu[:I] @ x[t], wgu[I:] @ x[t]
            if plant == "swap":
                gate, up = up, gate
            if plant == "w_in_silu":
                act = F.silu(wk[j] * gate) * up
            else:
                act = F.silu(gate) * up * wk[j]
            out[t] += deq(dq[e], ds[e], H, I, half=True) @ act
    return out.numpy()


@pytest.mark.parametrize("topk,ties", [(1, False), (2, True), (3, False)])
def test_moe_ref_matches_independent_torch_layer(topk, ties):
    """oracle.moe_ref (the only checker of the MoE layer) against the independent float64 torch composition above.
    topk = 1: every routing weight is exactly 1; topk = 2 with three tied top logits: the two lowest-index ones are
    selected with weights exactly 0.5 (the k-sum and the tie rule); topk = 3: general weights (the oracle's fp32
    routing weights, 1e-7 relative). Each planted mistake moves the result far past the agreement bound."""
    E, H, I, T = 8, 256, 128, 4
    gq, gs, dq, ds = synth.moe_host(E, H, I, seed=17 + topk)
    lg = synth.logits_host(T, E, seed=23 + topk)
    if ties:
        for t in range(T):
            lg[t, [1, 4, 6]] = lg[t].max() + 0.5
    xh = synth.x_host(T, H, seed=29 + topk)
    got, sel, w = oracle.moe_ref(lg, xh, gq, gs, dq, ds, topk, H, I)
    want = _moe_layer_torch(lg, xh, gq, gs, dq, ds, topk, H, I)
    rms = np.sqrt(np.mean(want ** 2))
    bound = 1e-12 if topk <= 2 else 1e-6
    assert np.abs(got - want).max() <= bound * rms, float(np.abs(got - want).max() / rms)
    if topk == 1:
        assert np.all(w == 1.0)
    if ties:
        assert np.all(sel == [1, 4]) and np.all(w == 0.5)
    plants = ["swap", "no_renorm", "drop_k"] + (["w_in_silu", "ties_high"] if ties else [])
    for plant in plants:
        bad = _moe_layer_torch(lg, xh, gq, gs, dq, ds, topk, H, I, plant=plant)
        assert np.abs(got - bad).max() > 0.05 * rms, (plant, float(np.abs(got - bad).max() / rms))


# ---------------------------------------------------------------- Q8 layout (reference src/kernels/q8_layout.h)
_REF_DIR = os.path.join(os.path.dirname(oracle.__file__), "_ref")


def test_q8_pos_known_answers_and_bijection():
    """positions written from the layout comment (q8_layout.h:5-12): word 2 s + hi of lane (g, t) of tile r and
    32-k chunk c holds row 16 r + g + 8 hi, bytes i = k 32 c + 16 s + 2 t + {0, 8, 1, 9}[i]"""
    K = 256
    kat = {(0, 0): 0, (0, 8): 1, (0, 1): 2, (0, 9): 3, (8, 0): 4, (0, 16): 8, (8, 16): 12,
           (0, 2): 16, (1, 0): 64, (0, 32): 512, (16, 0): (K // 32) * 512, (17, 35): (K // 32) * 512 + 512 + 4 * 16 + 16 + 2}
    for (r, k), pos in kat.items():
        assert oracle.q8_pos(r, k, K) == pos, (r, k)
    n = 32
    pos = [oracle.q8_pos(r, k, K) for r in range(n) for k in range(K)]
    assert sorted(pos) == list(range(n * K))


@pytest.mark.skipif(not os.path.exists(os.path.join(_REF_DIR, "libq8ref.so")), reason="oracle/_ref not built")
def test_q8_pos_matches_reference_header():
    ref = ctypes.CDLL(os.path.join(_REF_DIR, "libq8ref.so"))
    ref.ref_q8_pos.restype = ctypes.c_size_t
    ref.ref_q8_pos.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    for n, K in ((64, 256), (48, 512)):
        for r in range(n):
            for k in range(K):
                assert oracle.q8_pos(r, k, K) == ref.ref_q8_pos(r, k, K), (r, k, K)


@pytest.mark.skipif(not os.path.exists(os.path.join(_REF_DIR, "q8_layout_unit")), reason="oracle/_ref not built")
def test_q8_reference_unit_test_passes():
    """the reference's own known-answer test of the Q8 layout (tests/q8_layout_unit.cpp), built from its sources"""
    out = subprocess.run([os.path.join(_REF_DIR, "q8_layout_unit")], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "ok (0 failures)" in out.stdout, out.stdout


def test_repack_q8_places_signed_weights():
    """compressed-tensors source (byte b of word j = k 4 j + b, u = w + 128) -> Q8 byte at q8_pos = w (int8)"""
    n, k = 32, 256
    rng = np.random.default_rng(3)
    w = rng.integers(-128, 128, size=(n, k)).astype(np.int32)
    u = (w + 128).astype(np.uint32).reshape(n, k // 4, 4)
    q = (u[..., 0] | (u[..., 1] << 8) | (u[..., 2] << 16) | (u[..., 3] << 24)).view(np.int32)
    s = synth.np_bf16(np.abs(rng.standard_normal((n, k // 128))).astype(np.float32) * 0.01)
    dq, ds = oracle.repack_q8(q, s, n, k)
    for r in range(0, n, 7):
        for c in range(0, k, 5):
            assert dq[oracle.q8_pos(r, c, k)].astype(np.int8) == w[r, c]
    assert np.array_equal(ds.reshape(n // 16, k // 128, 16).transpose(0, 2, 1).reshape(n, k // 128), s)
    deq = oracle.dequant_q8(q, s, n, k)
    ref = synth.np_bf16(w.astype(np.float32) * np.repeat(oracle.bf16_to_f32(s), 128, axis=1))
    assert np.array_equal(deq, ref)


# ------------------------------------------------------------------ H16 (XH activations, fp16 chunk partials)
def test_xh_pos_matches_lane_kstep_statement():
    """gemv_h16.cuh:8-10: lane t of a token's quad reads halves [16 t, 16 t + 16) of a chunk, i.e. for k-step j the
    values at k = 16 j + {2t, 2t+1, 2t+8, 2t+9}; every 64-k chunk is a permutation of itself"""
    for base in (0, 64, 640):
        for t in range(4):
            for j in range(4):
                ks = base + 16 * j + np.array([2 * t, 2 * t + 1, 2 * t + 8, 2 * t + 9])
                assert list(oracle.xh_pos(ks)) == [base + 16 * t + 4 * j + e for e in range(4)]
    p = oracle.xh_pos(np.arange(64 * 7))
    assert np.array_equal(np.sort(p), np.arange(64 * 7))
    assert np.array_equal(p // 64, np.arange(64 * 7) // 64)


def test_xh_pack_matches_torch_clamp_and_half():
    rng = np.random.default_rng(5)
    m, k = 3, 256
    x = synth.np_bf16((rng.standard_normal((m, k)) * 10.0 ** rng.integers(-6, 4, (m, k))).astype(np.float32))
    x[0, :4] = synth.np_bf16(np.array([3000.0, -3000.0, 2047.0, -2048.0], np.float32))
    xh = oracle.xh_pack(x, ldxh=320)
    xt = torch.from_numpy(oracle.bf16_to_f32(x))
    want = (xt.clamp(-2047, 2047) / 16).half().view(torch.int16).numpy().view(np.uint16)
    p = oracle.xh_pos(np.arange(k))
    assert np.array_equal(xh[:, p], want)
    assert not xh[:, k:].any()
    assert np.array_equal(oracle.xh_values(xh, k), want.view(np.float16).astype(np.float64))


@pytest.mark.parametrize("wdiv", [1, 16])
def test_gemv_h16_exact_on_integer_inputs(wdiv):
    """x / 16 and w / wdiv small integers, power-of-two scales: every chunk partial is an integer below 2048 (exact in
    fp16), so the H16 arithmetic must equal the float64 product x . (w * s)^T exactly"""
    rng = np.random.default_rng(wdiv)
    m, n, k = 5, 24, 640
    xv = rng.integers(-3, 4, (m, k)).astype(np.float64)
    w = rng.integers(-7, 8, (n, k)) * wdiv
    s = 2.0 ** rng.integers(-12, -4, (n, k // 128))
    got = oracle.gemv_h16(xv, w, s, wdiv)
    want = (xv * 16) @ (w * np.repeat(s, 128, axis=1)).T
    assert np.array_equal(got, want)


@pytest.mark.parametrize("wdiv", [1, 16])
def test_gemv_h16_within_one_fp16_rounding_per_chunk(wdiv):
    """random XH values: |h16 - exact| <= sum over 64-k chunks of half an fp16 ulp of the chunk's magnitude bound,
    at that chunk's scale; and the rounding really happens (not equal to the exact product)"""
    rng = np.random.default_rng(10 + wdiv)
    m, n, k = 4, 32, 1024
    x = synth.np_bf16(rng.standard_normal((m, k)).astype(np.float32) * 3)
    xv = oracle.xh_values(oracle.xh_pack(x), k)
    w = rng.integers(-8, 8, (n, k)) if wdiv == 1 else rng.integers(-127, 128, (n, k))
    s = np.abs(rng.standard_normal((n, k // 128))) * 0.01
    got = oracle.gemv_h16(xv, w, s, wdiv)
    exact = (xv * 16) @ (w * np.repeat(s, 128, axis=1)).T
    mag = np.einsum("mci,nci->mcn", np.abs(xv).reshape(m, k // 64, 64), np.abs(w / wdiv).reshape(n, k // 64, 64))
    half_ulp = 2.0 ** (np.floor(np.log2(np.maximum(mag, 2.0 ** -14))) - 11)  # [m][chunks][n]
    bound = (half_ulp * (np.repeat(s, 2, axis=1).T * 16 * wdiv)[None]).sum(axis=1)
    assert np.all(np.abs(got - exact) <= bound)
    assert not np.array_equal(got, exact)
    assert np.abs(got - exact).max() > 1e-3 * bound.max()


@pytest.mark.parametrize("wdiv", [1, 16])
def test_gemv_h16_step16_within_four_roundings_per_chunk(wdiv):
    """the reference's accumulation (an fp16 rounding after every 16-k MMA step, step = 16): |h16 - exact| <= sum
    over 64-k chunks of 4 half fp16 ulps of the chunk's magnitude bound at its scale; exact on integer inputs; it
    differs from the once-per-chunk rounding (step = 64), so the two emulations are not the same function"""
    rng = np.random.default_rng(20 + wdiv)
    m, n, k = 4, 32, 1024
    x = synth.np_bf16(rng.standard_normal((m, k)).astype(np.float32) * 3)
    xv = oracle.xh_values(oracle.xh_pack(x), k)
    w = rng.integers(-8, 8, (n, k)) if wdiv == 1 else rng.integers(-127, 128, (n, k))
    s = np.abs(rng.standard_normal((n, k // 128))) * 0.01
    got = oracle.gemv_h16(xv, w, s, wdiv, step=16)
    exact = (xv * 16) @ (w * np.repeat(s, 128, axis=1)).T
    mag = np.einsum("mci,nci->mcn", np.abs(xv).reshape(m, k // 64, 64), np.abs(w / wdiv).reshape(n, k // 64, 64))
    half_ulp = 2.0 ** (np.floor(np.log2(np.maximum(mag, 2.0 ** -14))) - 11)
    bound = (4 * half_ulp * (np.repeat(s, 2, axis=1).T * 16 * wdiv)[None]).sum(axis=1)
    assert np.all(np.abs(got - exact) <= bound)
    assert not np.array_equal(got, oracle.gemv_h16(xv, w, s, wdiv, step=64))
    # small integers (x / 16 in -3..3, w in -8..7: every partial sum of a chunk is a multiple of 1 / wdiv below 1536 /
    # wdiv, 11 bits) with power-of-two scales: every partial is exact in fp16, so is the result
    xi = synth.np_bf16((rng.integers(-3, 4, (m, k)) * 16).astype(np.float32))
    xvi = oracle.xh_values(oracle.xh_pack(xi), k)
    wi = rng.integers(-8, 8, (n, k))
    si = 2.0 ** rng.integers(-6, -3, (n, k // 128)).astype(np.float64)
    assert np.array_equal(oracle.gemv_h16(xvi, wi, si, wdiv, step=16), (xvi * 16) @ (wi * np.repeat(si, 128, axis=1)).T)


def test_x_to_h_matches_torch():
    """x_to_h against torch's float32 arithmetic and fp16 conversion; a zero row takes xs = 1, xh = 0; a row whose
    amax is 16 keeps its values (xs = 1)"""
    rng = np.random.default_rng(7)
    t, k = 6, 384
    xf = rng.standard_normal((t, k)).astype(np.float32) * np.exp(rng.standard_normal((t, 1))).astype(np.float32) * 5
    xf[2] = 0
    xf[3] = np.clip(np.round(xf[3]), -15, 15)
    xf[3, 7] = -16
    x = synth.np_bf16(xf)
    xh, xs = oracle.x_to_h(x)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).float()
    amax = xt.abs().amax(1)
    sc = torch.where(amax > 0, amax / 16, torch.ones_like(amax))
    inv = 1.0 / sc
    want = (xt * inv[:, None]).half().double().numpy()
    assert np.array_equal(xs, sc.numpy()) and np.array_equal(xh, want)
    assert xs[2] == 1 and not xh[2].any()
    assert xs[3] == 1 and np.array_equal(xh[3], oracle.bf16_to_f32(x[3]).astype(np.float64))
    assert np.abs(xh).max() <= 16


def test_gemm_h_exact_on_integer_inputs():
    """xh small integers, power-of-two scales and token scales: every chunk partial is an integer below 2048 (exact
    in fp16), so gemm_h equals the float64 product exactly"""
    rng = np.random.default_rng(3)
    t, n, k = 5, 24, 640
    xh = rng.integers(-3, 4, (t, k)).astype(np.float64)
    xs = (2.0 ** rng.integers(-4, 3, t)).astype(np.float32)
    w = rng.integers(-8, 8, (n, k))
    s = 2.0 ** rng.integers(-12, -4, (n, k // 128))
    got = oracle.gemm_h(xh, xs, w, s)
    want = (xh * xs[:, None].astype(np.float64)) @ (w * np.repeat(s, 128, axis=1)).T
    assert np.array_equal(got, want)


def test_gemm_h_within_one_fp16_rounding_per_chunk():
    """random activations through x_to_h: |gemm_h - exact| <= sum over chunks of half an fp16 ulp of the chunk's
    magnitude bound at that chunk's scale (times the token scale); and the rounding really happens"""
    rng = np.random.default_rng(11)
    t, n, k = 4, 32, 1024
    x = synth.np_bf16(rng.standard_normal((t, k)).astype(np.float32) * 3)
    xh, xs = oracle.x_to_h(x)
    w = rng.integers(-8, 8, (n, k))
    s = np.abs(rng.standard_normal((n, k // 128))) * 0.01
    got = oracle.gemm_h(xh, xs, w, s)
    exact = (xh * xs[:, None].astype(np.float64)) @ (w * np.repeat(s, 128, axis=1)).T
    mag = np.einsum("mci,nci->mcn", np.abs(xh).reshape(t, k // 64, 64), np.abs(w).reshape(n, k // 64, 64).astype(np.float64))
    half_ulp = 2.0 ** (np.floor(np.log2(np.maximum(mag, 2.0 ** -14))) - 11)
    bound = (half_ulp * np.repeat(s, 2, axis=1).T[None]).sum(axis=1) * xs[:, None]
    assert np.all(np.abs(got - exact) <= bound)
    assert not np.array_equal(got, exact)


@pytest.mark.parametrize("G", [32, 64, 128])
def test_x_to_i8_matches_reference_emulation(G):
    """x_to_i8 against the reference test's torch emulation (tests/test_gemm_i8.py:52-61, restated: amax, / 127.0,
    the low two mantissa bits cleared, 1 / sc, round, clamp); a zero group gives sx = 1, q = 0; a group whose
    amax is 127 * 2^e has sx = 2^e and q = x / 2^e exactly"""
    rng = np.random.default_rng(G)
    t, k = 5, 512
    xf = rng.standard_normal((t, k)).astype(np.float32) * np.exp(rng.standard_normal((t, 1))).astype(np.float32) * 4
    xf[1, :G] = 0
    xf[2, :G] = np.clip(np.round(xf[2, :G] * 10), -100, 100) * np.float32(0.25)
    xf[2, 3] = 127 * 0.25
    x = synth.np_bf16(xf)
    q, sx = oracle.x_to_i8(x, G)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).float().reshape(t, k // G, G)
    amax = xt.abs().amax(-1, keepdim=True)
    sc = (amax / 127.0).view(torch.int32) & ~3
    sc = torch.where(amax > 0, sc.view(torch.float32), torch.ones_like(amax))
    inv = torch.where(amax > 0, 1.0 / sc, torch.zeros_like(amax))
    want = torch.round(xt * inv).clamp(-127, 127).reshape(t, k).numpy().astype(np.int8)
    assert np.array_equal(q, want) and np.array_equal(sx, sc.reshape(t, k // G).numpy())
    assert sx[1, 0] == 1 and not q[1, :G].any()
    assert sx[2, 0] == 0.25 and np.array_equal(q[2, :G].astype(np.float32) * 0.25, oracle.bf16_to_f32(x[2, :G]))


def test_gemm_i8_brute_force():
    """gemm_i8 = the scalar triple loop over the dequantized int8 operands on a tiny shape"""
    rng = np.random.default_rng(1)
    t, n, k, G = 3, 5, 256, 64
    q = rng.integers(-127, 128, (t, k)).astype(np.int8)
    sx = rng.random((t, k // G)).astype(np.float32)
    w = rng.integers(-8, 8, (n, k))
    s = rng.random((n, k // 128))
    got = oracle.gemm_i8(q, sx, w, s, G)
    want = np.zeros((t, n))
    for i in range(t):
        for j in range(n):
            want[i, j] = sum(float(q[i, kk]) * float(sx[i, kk // G]) * float(w[j, kk]) * s[j, kk // 128] for kk in range(k))
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def _rn_f32(v):
    """an exact rational -> the nearest float32, ties to even (normal and subnormal range, no overflow)"""
    from fractions import Fraction
    if v == 0:
        return np.float32(0)
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** max(e - 23, -149)
    q, r = divmod(a, ulp)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return np.float32(float(q * ulp) * (1 if v > 0 else -1))


@pytest.mark.parametrize("per_channel", [False, True])
def test_rows_w8a8_exact_rational(per_channel):
    """rows_w8a8 = the per-group steps in exact rational arithmetic on a tiny shape: integer sum, one float32
    rounding of sum * sx, one of the fused multiply-add p * sw + y (k_rows_qt, src/flash/flash_pfq.cuh:637-641)"""
    from fractions import Fraction
    rng = np.random.default_rng(7 + per_channel)
    t, n, k = 3, 4, 384
    ng = k // 128
    xq = rng.integers(-127, 128, (t, k)).astype(np.int8)
    sx = ((rng.random((t, ng)) * 0.05 + 1e-3).astype(np.float32).view(np.uint32) & np.uint32(0xFFFFFFFC)).view(np.float32)
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sw = oracle.bf16_to_f32(synth.np_bf16((rng.standard_normal((n,) if per_channel else (n, ng)) * 0.01).astype(np.float32)))
    got = oracle.rows_w8a8(xq, sx, w, sw, per_channel)
    for i in range(t):
        for j in range(n):
            y = np.float32(0)
            for g in range(ng):
                s = int(np.dot(xq[i, 128 * g:128 * g + 128].astype(np.int64), w[j, 128 * g:128 * g + 128].astype(np.int64)))
                p = _rn_f32(Fraction(s) * Fraction(float(sx[i, g])))
                swg = sw[j] if per_channel else sw[j, g]
                y = _rn_f32(Fraction(float(p)) * Fraction(float(swg)) + Fraction(float(y)))
            assert got[i, j] == y, (i, j, got[i, j], y)


def test_rows_w8a8_integer_inputs_exact():
    """power-of-two scales and small integers: every partial result is a multiple of 2^-13 below 2^7 (20 bits), so
    every rounding is exact and rows_w8a8 equals the float64 product"""
    rng = np.random.default_rng(3)
    t, n, k = 6, 10, 512
    xq = rng.integers(-20, 21, (t, k)).astype(np.int8)
    w = rng.integers(-20, 21, (n, k)).astype(np.int8)
    sx = (2.0 ** rng.integers(-6, -4, (t, k // 128))).astype(np.float32)
    sw = (2.0 ** rng.integers(-7, -5, (n, k // 128))).astype(np.float32)
    got = oracle.rows_w8a8(xq, sx, w, sw, False)
    xd = (xq.astype(np.float64).reshape(t, k // 128, 128) * sx[:, :, None]).reshape(t, k)
    wd = (w.astype(np.float64).reshape(n, k // 128, 128) * sw[:, :, None]).reshape(n, k)
    assert np.array_equal(got.astype(np.float64), xd @ wd.T)
