"""Typed torch wrappers over the C-ABI (the reference's W4 / W8 structs and entry points, gemv.cuh:17-200).

Tensors are device tensors; 16-bit scales are torch.float16 (QE_SCALE_F16) or torch.bfloat16. Every wrapper
checks shapes on the host before calling into the library, which checks them again (fatal abort).
"""
import ctypes
from dataclasses import dataclass

import torch

from .qe import call

SCALE_F16 = 1
OUT_BF16 = 2
GLU = 4
W8_PER_CHANNEL = 8


class QeConfig(ctypes.Structure):
    """include/qe_kernels.h qe_config_t"""
    _fields_ = [("skinny_min_m", ctypes.c_int), ("w8_mfma_min_m", ctypes.c_int), ("batch_invariant", ctypes.c_int),
                ("gemm_tune", ctypes.c_int), ("gemm_h16", ctypes.c_int), ("reserved", ctypes.c_int * 3)]


def get_config():
    from .qe import lib
    c = QeConfig()
    lib().qe_get_config(ctypes.byref(c))
    return {"skinny_min_m": c.skinny_min_m, "w8_mfma_min_m": c.w8_mfma_min_m, "batch_invariant": c.batch_invariant,
            "gemm_tune": c.gemm_tune, "gemm_h16": c.gemm_h16}


def set_config(**kw):
    """update the library's kernel policy (qe_set_config); returns the previous settings"""
    from .qe import lib
    old = get_config()
    c = QeConfig()
    lib().qe_get_config(ctypes.byref(c))
    for key, v in kw.items():
        setattr(c, key, int(v))
    lib().qe_set_config(ctypes.byref(c))
    return old


def _stream():
    # a pointer-sized argument: an int would be passed as a 32-bit c_int
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _scale_flag(s):
    if s.dtype == torch.float16:
        return SCALE_F16
    if s.dtype == torch.bfloat16:
        return 0
    raise TypeError(f"scales must be float16 or bfloat16, got {s.dtype}")


@dataclass
class W4:
    """INT4 g128 matrix in the W4 fragment layout (q: uint8 [n*k/2], s: [n*k/128] 16-bit)."""
    q: torch.Tensor
    s: torch.Tensor
    n: int
    k: int
    glu: bool = False

    @property
    def flags(self):
        return _scale_flag(self.s) | (GLU if self.glu else 0)


@dataclass
class W8:
    """INT8 matrix in the W8 layout (q: uint8 [n*k]); s: [n] (per channel) or [n*k/128] (group 128)."""
    q: torch.Tensor
    s: torch.Tensor
    n: int
    k: int
    per_channel: bool = True

    @property
    def flags(self):
        return _scale_flag(self.s) | (W8_PER_CHANNEL if self.per_channel else 0)


def repack_w4(q, s, glu=False):
    """compressed-tensors int32 [n][k/8] + scales [n][k/128] -> W4 (on the default stream, as the reference)."""
    n, k = q.shape[0], q.shape[1] * 8
    assert q.dtype == torch.int32 and q.is_contiguous() and s.shape == (n, k // 128) and s.is_contiguous()
    assert n % 16 == 0 and k % 128 == 0
    dq = torch.empty(n * k // 2, dtype=torch.uint8, device=q.device)
    ds = torch.empty(n * (k // 128), dtype=s.dtype, device=q.device)
    call("qe_repack_w4", q, s, n, k, dq, ds)
    return W4(dq, ds, n, k, glu)


def glu_rows(q, s, bits=4):
    """[gate 0..I)[up 0..I) rows -> GLU tile order (8 gate, 8 up per 16-row tile)."""
    n = q.shape[0]
    k = q.shape[1] * 32 // bits
    dq = torch.empty_like(q)
    ds = torch.empty_like(s)
    call("qe_glu_rows", q, s, n, k, dq, ds, bits)
    return dq, ds


def dequant_w4(w: W4):
    out = torch.empty(w.n, w.k, dtype=torch.bfloat16, device=w.q.device)
    call("qe_dequant_w4", w.q, w.s, w.n, w.k, _scale_flag(w.s), out, _stream())
    return out


def _out(m, n, out_bf16, glu, device):
    if glu:
        return torch.empty(m, n // 2, dtype=torch.bfloat16, device=device)
    return torch.empty(m, n, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=device)


def gemv_w4(w: W4, x, out_bf16=False, y=None):
    """decode GEMV / skinny GEMM, m = x.shape[0] in 1..16"""
    m = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(m, w.n, out_bf16, w.glu, x.device) if y is None else y
    call("qe_gemv_w4_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), m,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def xh_pack(x, ldxh=None):
    """bf16 [m][k] -> the XH layout [m][ldxh] fp16 (x / 16, |x| clamped to 2047, columns of each 64-k chunk permuted);
    reference hook qe_xh_pack"""
    m, k = x.shape
    ldxh = k if ldxh is None else ldxh
    assert x.dtype == torch.bfloat16 and x.is_contiguous() and k % 64 == 0 and ldxh >= k and ldxh % 64 == 0
    xh = torch.zeros(m, ldxh, dtype=torch.float16, device=x.device)
    call("qe_xh_pack", x, k, m, xh, ldxh)
    return xh


def gemv_w4h(w: W4, x, yh=False):
    """H16 decode GEMV on bf16 activations (reference hook qe_gemv_w4h, bf16 scales): packs x into an XH workspace,
    then fp16 chunk partials flushed into fp32. -> (y, xh, yh): y fp32 [m][n] (GLU: bf16 act [m][n/2]), yh the XH
    copy of y when asked for"""
    m = x.shape[0]
    assert w.s.dtype == torch.bfloat16 and x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.is_contiguous()
    y = _out(m, w.n, False, w.glu, x.device)
    xh = torch.empty(m, w.k, dtype=torch.float16, device=x.device)
    yo = torch.empty(m, w.n // 2 if w.glu else w.n, dtype=torch.float16, device=x.device) if yh else None
    call("qe_gemv_w4h", w.q, w.s, w.n, w.k, x, y, m, int(w.glu), xh, yo)
    return y, xh, yo


def gemv_w4hx(w: W4, xh, out_bf16=False, yh=None, y=None):
    """H16 decode GEMV on activations already in the XH layout (qe_gemv_w4h_ex: any scale dtype, strides, stream)"""
    m = xh.shape[0]
    assert xh.dtype == torch.float16 and xh.shape[1] >= w.k and xh.stride(1) == 1
    y = _out(m, w.n, out_bf16, w.glu, xh.device) if y is None else y
    call("qe_gemv_w4h_ex", w.q, w.s, w.n, w.k, xh, xh.stride(0), y, y.stride(0), m,
         w.flags | (OUT_BF16 if out_bf16 else 0), yh, 0 if yh is None else yh.stride(0), _stream())
    return y


def gemm_w4(w: W4, x, out_bf16=False, y=None):
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, w.glu, x.device) if y is None else y
    call("qe_gemm_w4_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def gemm_w4h(w: W4, x, out_bf16=False, y=None):
    """prefill GEMM with the reference's fp16-accumulate numerics (qe_gemm_w4h_ex)"""
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, w.glu, x.device) if y is None else y
    call("qe_gemm_w4h_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def gemm_w4_i8(w: W4, x, G=64, out_bf16=False, y=None):
    """W4A8 prefill GEMM, activation group G (qe_gemm_w4_i8_ex)"""
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, w.glu, x.device) if y is None else y
    call("qe_gemm_w4_i8_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t, G,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def gemm_w4_choice(w: W4, x, cfg, ks, out_bf16=False, y=None):
    """prefill GEMM with a given (tile configuration, split) instead of the tuner's; returns (y, split applied)"""
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, w.glu, x.device) if y is None else y
    from .qe import lib
    lib().qe_gemm_w4_choice.restype = ctypes.c_int
    r = call("qe_gemm_w4_choice", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
             w.flags | (OUT_BF16 if out_bf16 else 0), cfg, ks, _stream())
    return y, bool(r)


def matmul_w4_onepass(w: W4, x, out_bf16=False, y=None):
    """the one-pass decode GEMM (qe_matmul_w4_onepass_ex) for 1..64 rows (the decode numerics: unrounded weights);
    returns y, or None if the shape does not fit it"""
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, w.glu, x.device) if y is None else y
    from .qe import lib
    lib().qe_matmul_w4_onepass_ex.restype = ctypes.c_int
    r = call("qe_matmul_w4_onepass_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
             w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y if r else None


def matmul_w4(w: W4, x, out_bf16=False, y=None):
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, w.glu, x.device) if y is None else y
    call("qe_matmul_w4_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def tile_w8(q, s, per_channel=True):
    """row-major int8 [n][k] + scales ([n] per channel, else [n][k/128]) -> W8 layout"""
    n, k = q.shape
    assert q.dtype == torch.int8 and q.is_contiguous() and n % 16 == 0 and k % 128 == 0
    dq = torch.empty(n * k, dtype=torch.uint8, device=q.device)
    ds = torch.empty(n if per_channel else n * (k // 128), dtype=s.dtype, device=q.device)
    call("qe_tile_w8", q, s, n, k, int(per_channel), dq, ds, _stream())
    return W8(dq, ds, n, k, per_channel)


def quantize_w8(w):
    """RTN INT8 group 128 of a bf16 [n][k] matrix (reference qe_quantize_w8)"""
    n, k = w.shape
    dq = torch.empty(n * k, dtype=torch.uint8, device=w.device)
    ds = torch.empty(n * (k // 128), dtype=torch.bfloat16, device=w.device)
    call("qe_quantize_w8", w, n, k, dq, ds)
    return W8(dq, ds, n, k, False)


def dequant_w8(w: W8):
    out = torch.empty(w.n, w.k, dtype=torch.bfloat16, device=w.q.device)
    call("qe_dequant_w8", w.q, w.s, w.n, w.k, w.flags, out, _stream())
    return out


def gemv_w8(w: W8, x, out_bf16=False, y=None):
    m = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(m, w.n, out_bf16, False, x.device) if y is None else y
    call("qe_gemv_w8_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), m,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def gemm_w8(w: W8, x, out_bf16=False, y=None):
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, False, x.device) if y is None else y
    call("qe_gemm_w8_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def gemm_w8a8(w: W8, x, out_bf16=False, y=None):
    """W8A8 row GEMM, the reference's prefill numerics for INT8 matrices (k_x_to_r8 + k_rows_qt;
    qe_gemm_w8a8_ex): bit-identical to its arithmetic"""
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = _out(t, w.n, out_bf16, False, x.device) if y is None else y
    call("qe_gemm_w8a8_ex", w.q, w.s, w.n, w.k, x, x.stride(0), y, y.stride(0), t,
         w.flags | (OUT_BF16 if out_bf16 else 0), _stream())
    return y


def rows8(w: W8, x, y=None):
    """the reference's Worker::rows8 dispatch (qe_rows8): W8A8 for m >= 64, k <= 4096 and an 8-element row
    stride, else the W8A16 GEMM; fp32 out"""
    m = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.stride(1) == 1
    y = torch.empty(m, w.n, dtype=torch.float32, device=x.device) if y is None else y
    call("qe_rows8", w.q, w.s, w.n, w.k, w.flags, x, x.stride(0), y, y.stride(0), m, _stream())
    return y


@dataclass
class Q8:
    """INT8 layer weights in the reference's Q8 byte order (src/kernels/q8_layout.h), bf16 group-128 scales"""
    q: torch.Tensor
    s: torch.Tensor
    n: int
    k: int
    glu: bool = False


def repack_q8(q, s, glu=False):
    """compressed-tensors 8-bit int32 [n][k/4] (u = w + 128) + bf16 scales [n][k/128] -> Q8 (reference hooks
    qe_glu_rows8 / qe_repack_q8)"""
    n, k = q.shape[0], q.shape[1] * 4
    assert s.dtype == torch.bfloat16 and s.shape == (n, k // 128)
    if glu:
        q2, s2 = torch.empty_like(q), torch.empty_like(s)
        call("qe_glu_rows8", q.contiguous(), s.contiguous(), n, k, q2, s2)
        q, s = q2, s2
    dq = torch.empty(n * k, dtype=torch.uint8, device=q.device)
    ds = torch.empty(n * (k // 128), dtype=torch.bfloat16, device=q.device)
    call("qe_repack_q8", q.contiguous(), s.contiguous(), n, k, dq, ds)
    return Q8(dq, ds, n, k, glu)


def gemv_q8(w: Q8, x, h16=False, yh=False):
    """decode GEMV (any m): fp32 [m][n], or the GLU bf16 activation [m][n/2] (reference hook qe_gemv_q8).
    h16: the fp16-accumulate XH numerics; returns (y, xh workspace, yh or None) then, else y"""
    m = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.is_contiguous()
    assert h16 or not yh
    y = _out(m, w.n, False, w.glu, x.device)
    if not h16:
        call("qe_gemv_q8", w.q, w.s, w.n, w.k, x, y, m, int(w.glu), 0, None, None)
        return y
    xh = torch.empty(m, w.k, dtype=torch.float16, device=x.device)
    yo = torch.empty(m, w.n // 2 if w.glu else w.n, dtype=torch.float16, device=x.device) if yh else None
    call("qe_gemv_q8", w.q, w.s, w.n, w.k, x, y, m, int(w.glu), 1, xh, yo)
    return y, xh, yo


def gemm_q8(w: Q8, x):
    """prefill GEMM: fp32 [t][n], or the GLU bf16 activation [t][n/2] (reference hook qe_gemm_q8)"""
    t = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.shape[1] == w.k and x.is_contiguous()
    y = _out(t, w.n, False, w.glu, x.device)
    call("qe_gemm_q8", w.q, w.s, w.n, w.k, x, y, t, int(w.glu), 0, 0)
    return y


class MoE:
    """One MoE layer of E INT4 experts in the group-record format (see include/qe_kernels.h)."""

    def __init__(self, records, E, topk, H, I):
        self.records, self.E, self.topk, self.H, self.I = records, E, topk, H, I
        self._ws = None
        self._old_ws = []  # outgrown workspaces stay alive: a captured HIP graph may still point at them

    @staticmethod
    def pack(gu_q, gu_s, dn_q, dn_s, topk):
        """gate_up int32 [E][2I][H/8] + fp16 [E][2I][H/128]; down int32 [E][H][I/8] + fp16 [E][H][I/128]"""
        E, I2, h8 = gu_q.shape
        H, I = h8 * 8, I2 // 2
        from .qe import lib
        lib().qe_moe_record_bytes.restype = ctypes.c_size_t
        rb = lib().qe_moe_record_bytes(H, I)
        recs = torch.empty(E * rb, dtype=torch.uint8, device=gu_q.device)
        call("qe_moe_pack_w4", gu_q, gu_s, dn_q, dn_s, E, H, I, recs, _stream())
        return MoE(recs, E, topk, H, I)

    def workspace(self, T):
        from .qe import lib
        lib().qe_moe_workspace_bytes.restype = ctypes.c_size_t
        nb = lib().qe_moe_workspace_bytes(T, self.E, self.topk, self.H, self.I)
        if self._ws is None or self._ws.numel() < nb:
            if self._ws is not None:
                self._old_ws.append(self._ws)
            self._ws = torch.empty(nb, dtype=torch.uint8, device=self.records.device)
        return self._ws, nb

    def __call__(self, logits, x, out_bf16=False, out=None):
        T = x.shape[0]
        assert logits.dtype == torch.float32 and logits.shape == (T, self.E) and x.shape == (T, self.H)
        ws, nb = self.workspace(T)
        if out is None:
            out = torch.empty(T, self.H, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=x.device)
        call("qe_moe_w4", logits, x, self.records, T, self.E, self.topk, self.H, self.I, out,
             OUT_BF16 if out_bf16 else 0, ws, ctypes.c_size_t(nb), _stream())
        return out


def moe_route(logits, topk):
    T, E = logits.shape
    sel = torch.empty(T, topk, dtype=torch.int32, device=logits.device)
    w = torch.empty(T, topk, dtype=torch.float32, device=logits.device)
    call("qe_moe_route", logits, T, E, topk, sel, w, _stream())
    return sel, w


def moe_segment(sel, w, E, chunk):
    T, topk = sel.shape
    dev = sel.device
    P = T * topk
    off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    slot_pair = torch.empty(P, dtype=torch.int32, device=dev)
    slot_tok = torch.empty(P, dtype=torch.int32, device=dev)
    slot_w = torch.empty(P, dtype=torch.float32, device=dev)
    inv = torch.empty(P, dtype=torch.int32, device=dev)
    jobs = torch.empty(2 * ((P + chunk - 1) // chunk + min(E, P)), dtype=torch.int32, device=dev)
    njobs = torch.empty(1, dtype=torch.int32, device=dev)
    call("qe_moe_segment", sel, w, T, E, topk, chunk, off, slot_pair, slot_tok, slot_w, inv, jobs, njobs, _stream())
    return dict(off=off, slot_pair=slot_pair, slot_tok=slot_tok, slot_w=slot_w, inv=inv, jobs=jobs, njobs=njobs)


# ---------------------------------------------------------------- on-disk weights (safetensors)
class SafeTensorsFile:
    """a memory-mapped .safetensors file (qe_st_open; the reference's SafeTensors, src/safetensors.h)"""

    def __init__(self, path):
        from .qe import lib
        L = lib()
        L.qe_st_open.restype = ctypes.c_void_p
        L.qe_st_name.restype = ctypes.c_char_p
        L.qe_st_count.restype = ctypes.c_int
        L.qe_st_tensor.restype = ctypes.c_int
        self._lib = L
        self.h = ctypes.c_void_p(L.qe_st_open(str(path).encode()))

    def close(self):
        if self.h:
            self._lib.qe_st_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def names(self):
        return [self._lib.qe_st_name(self.h, i).decode() for i in range(self._lib.qe_st_count(self.h))]

    def info(self, name):
        """-> (dtype, shape, nbytes, address) or None"""
        dt = ctypes.create_string_buffer(12)
        shape = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int()
        data = ctypes.c_void_p()
        nb = ctypes.c_size_t()
        if not self._lib.qe_st_tensor(self.h, name.encode(), dt, shape, ctypes.byref(nd), ctypes.byref(data),
                                      ctypes.byref(nb)):
            return None
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value)), nb.value, data.value

    def _specs(self, rows):
        names = (ctypes.c_char_p * len(rows))(*[r[0].encode() for r in rows])
        r0 = (ctypes.c_int * len(rows))(*[int(r[1]) for r in rows])
        r1 = (ctypes.c_int * len(rows))(*[int(r[2]) for r in rows])
        return names, r0, r1

    def w4_dims(self, rows, c0=-1, c1=-1):
        """rows: [(name, r0, r1), ...] -> (n, k, bits, sdt) of the matrix load_w4 builds"""
        names, r0, r1 = self._specs(rows)
        out = [ctypes.c_int() for _ in range(4)]
        self._lib.qe_load_w4_dims(self.h, names, r0, r1, len(rows), c0, c1, *[ctypes.byref(o) for o in out])
        return tuple(o.value for o in out)

    def load_w4(self, rows, c0=-1, c1=-1, glu=False, device="cuda"):
        """the reference's Worker::load_w4: -> W4 (4-bit) or Q8 (8-bit) on the device"""
        n, k, bits, sdt = self.w4_dims(rows, c0, c1)
        names, r0, r1 = self._specs(rows)
        dq = torch.empty(n * k * bits // 8, dtype=torch.uint8, device=device)
        ds = torch.empty(n * (k // 128), dtype=torch.float16 if sdt == SCALE_F16 else torch.bfloat16, device=device)
        self._lib.qe_load_w4(self.h, names, r0, r1, len(rows), c0, c1, int(glu), ctypes.c_void_p(dq.data_ptr()),
                             ctypes.c_void_p(ds.data_ptr()), _stream())
        return Q8(dq, ds, n, k, glu) if bits == 8 else W4(dq, ds, n, k, glu)
