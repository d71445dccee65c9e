// extern "C" entry points of libqe_kernels.so (declared in include/qe_kernels.h).
// Reference-named hooks keep the reference's signatures and semantics (src/capi.cpp:10-171): device
// pointers, default stream, bf16 scales, fp32 outputs, fatal abort on a violated precondition.
// Build-defined *_ex entry points take an explicit stream, row strides and flags (QeFlags).
#include "qe_api.hpp"
#include "gemm_tune.hpp"
#include "../../include/qe_kernels.h"

#include <algorithm>
#include <atomic>

[[noreturn]] void qe_fatal_check() {
    fflush(stdout);
    fflush(stderr);
    abort();
}

[[noreturn]] void qe_fatal_hip(hipError_t err, const char* what, const char* file, int line) {
    fprintf(stderr, "HIP error %d (%s) in %s at %s:%d\n", (int)err, hipGetErrorString(err), what, file, line);
    qe_fatal_check();
}

namespace {
std::atomic<int> g_out_bf16{0};
std::atomic<int> g_sk_maxparts{0};
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline W4 mk_w4(const void* q, const void* s, int n, int k, bool glu, int sdt) {
    W4 w;
    w.q = reinterpret_cast<const uint4*>(q);
    w.s = reinterpret_cast<const uint16_t*>(s);
    w.n = n;
    w.k = k;
    w.glu = glu;
    w.sdt = sdt;
    return w;
}
inline W8 mk_w8(const void* q, const void* s, int n, int k, bool per_channel, int sdt) {
    W8 w;
    w.q = reinterpret_cast<const uint4*>(q);
    w.s = reinterpret_cast<const uint16_t*>(s);
    w.n = n;
    w.k = k;
    w.per_channel = per_channel;
    w.sdt = sdt;
    return w;
}
}  // namespace

void gemm_set_out_bf16(bool on) { g_out_bf16.store(on ? 1 : 0); }
bool gemm_out_bf16() { return g_out_bf16.load() != 0; }
void gemm_set_sk_maxparts(int n) { g_sk_maxparts.store(n > 0 ? n : 0); }
int gemm_sk_maxparts() { return g_sk_maxparts.load(); }

extern "C" {

int qe_abi_version(void) { return QE_ABI_VERSION; }

void qe_get_config(qe_config_t* cfg) {
    CHECK(cfg != nullptr, "qe_get_config: null");
    const QeConfig& c = qe_config();
    *cfg = qe_config_t{};
    cfg->skinny_min_m = c.skinny_min_m;
    cfg->w8_mfma_min_m = c.w8_mfma_min_m;
    cfg->batch_invariant = c.batch_invariant;
    cfg->gemm_tune = c.gemm_tune;
    cfg->gemm_h16 = c.gemm_h16;
}

void qe_set_config(const qe_config_t* cfg) {
    CHECK(cfg != nullptr, "qe_set_config: null");
    QeConfig c;
    c.skinny_min_m = cfg->skinny_min_m;
    c.w8_mfma_min_m = cfg->w8_mfma_min_m;
    c.batch_invariant = cfg->batch_invariant;
    c.gemm_tune = cfg->gemm_tune;
    c.gemm_h16 = cfg->gemm_h16;
    CHECK(cfg->reserved[0] == 0 && cfg->reserved[1] == 0 && cfg->reserved[2] == 0, "qe_set_config: reserved fields must be 0");
    qe_config_set(c);
}

void qe_gemm_tune_file(const char* path) { gemm_tune_file(path); }
void qe_gemm_tune_clear(void) { gemm_table_clear(); }
int qe_gemm_tune_entries(void) { return (int)gemm_table_size(); }
void qe_gemm_reserve(size_t bytes) { gemm_reserve(bytes, 0); }
void qe_gemm_h_reserve(int k, int t) { gemm_h_reserve(k, t, 0); }
void qe_gemm_i8_reserve(int k, int t) { gemm_i8_reserve(k, t, 0); }
void qe_gemm_reserve_s(size_t bytes, void* stream) { gemm_reserve(bytes, as_stream(stream)); }
void qe_gemm_h_reserve_s(int k, int t, void* stream) { gemm_h_reserve(k, t, as_stream(stream)); }
void qe_gemm_i8_reserve_s(int k, int t, void* stream) { gemm_i8_reserve(k, t, as_stream(stream)); }
int qe_workspace_count(int kind) { return stream_ws_count(kind); }

// W4A8 (reference src/capi.cpp:104-113): ci (tile candidate) and ks (kernel variant) select among the reference's
// CUDA kernels; this build has one kernel per activation group and ignores them
void qe_gemm_w4_i8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t, int G, int ci,
                   int ks) {
    (void)ci;
    (void)ks;
    gemm_w4_i8(mk_w4(q, s, n, k, false, kScaleBF16), x, k, y, n, t, G, gemm_out_bf16(), 0);
}
void qe_gemm_w4_i8_glu(const void* q, const void* s, int n, int k, const uint16_t* x, void* act, int t, int G, int ci,
                       int ks) {
    (void)ci;
    (void)ks;
    gemm_w4_i8(mk_w4(q, s, n, k, true, kScaleBF16), x, k, act, n / 2, t, G, false, 0);
}
void qe_gemm_w4_i8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                      int G, int flags, void* st) {
    gemm_w4_i8(mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y,
               ldy, t, G, (flags & QE_OUT_BF16) != 0, as_stream(st));
}

int qe_matmul_w4_onepass_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy,
                            int m, int flags, void* stream) {
    const W4 w = mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16);
    if (!wdec_w4_fits(w, x, ldx, m)) return 0;
    wdec_w4(w, x, ldx, y, ldy, m, (flags & QE_OUT_BF16) != 0, as_stream(stream));
    return 1;
}

int qe_gemm_w4_choice(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                      int flags, int cfg, int ks, void* stream) {
    const W4 w = mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16);
    gemm_w4_choice(w, x, ldx, y, ldy, t, (flags & QE_OUT_BF16) != 0, cfg, ks, as_stream(stream));
    return ks > 1 && gemm_split_applies(cfg, n, k, t, ks) ? 1 : 0;
}

void qe_read_probe(const void* q, int n, int k, uint32_t* sink, void* stream) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && q && sink, "read_probe %d %d", n, k);
    read_probe_w4(q, n, k, sink, reinterpret_cast<hipStream_t>(stream));
}

float qe_clock_probe_mhz(void* stream) { return clock_probe_mhz(reinterpret_cast<hipStream_t>(stream)); }

// ---------------------------------------------------------------- reference-named hooks
void qe_gemv_workspace_init(void) {
    gemv_workspace_init();
    moe_scratch_ptr();  // the device's scratch address, resolved at set-up rather than on the first no-alloc call
}

void qe_repack_w4(const int32_t* q, const uint16_t* s, int n, int k, void* dq, void* ds) {
    repack_w4(q, s, n, k, reinterpret_cast<uint4*>(dq), reinterpret_cast<uint16_t*>(ds), 0);
}

void qe_gemv_w4(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m) {
    gemv_workspace_init();
    matmul_w4(mk_w4(q, s, n, k, false, kScaleBF16), x, k, y, n, m, false, 0);
}

void qe_gemv_w4g(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu) {
    gemv_workspace_init();
    CHECK(m >= 1 && m <= kMaxGemvW4Tokens, "qe_gemv_w4g m %d", m);
    matmul_w4(mk_w4(q, s, n, k, glu != 0, kScaleBF16), x, k, y, glu ? n / 2 : n, m, false, 0);
}

// the reference's skinny_w4 takes 1..32 rows (src/kernels/skinny.cu:572) and equals its GEMV bit for bit; here it is
// the decode dispatch of qe_gemv_w4g itself (matmul_w4: 1..16 rows the decode GEMV / skinny kernel, 17..32 the
// one-pass kernel where the dispatch picks it, else the 32-row skinny launch), so the bits are equal by construction. 17..32
// rows that neither of those one-launch kernels takes (x not 16-byte aligned, K slicing) return 0: unsupported, the
// caller falls back to qe_gemv_w4 as the reference's callers do.
int qe_skinny_w4(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu) {
    if (m < 1 || m > kWideRows || n <= 0 || k <= 0 || n % 16 != 0 || k % 128 != 0 || k % 8 != 0) return 0;
    const W4 w = mk_w4(q, s, n, k, glu != 0, kScaleBF16);
    if (m > kMaxGemvRows) {
        const bool onepass = !qe_config().batch_invariant && wdec_w4_pick(w, x, k, m);
        if (!onepass && !skinny_w4_wide_fits(w, x, k)) return 0;
    }
    gemv_workspace_init();
    matmul_w4(w, x, k, y, glu ? n / 2 : n, m, false, 0);
    return 1;
}

void qe_gemv_w4_s(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, void* st) {
    gemv_workspace_init();
    matmul_w4(mk_w4(q, s, n, k, false, kScaleBF16), x, k, y, n, m, false, as_stream(st));
}

void qe_gemm_w4(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t) {
    gemm_w4(mk_w4(q, s, n, k, false, kScaleBF16), x, k, y, n, t, gemm_out_bf16(), 0);
}

void qe_gemm_w4_t(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t) {
    gemm_w4(mk_w4(q, s, n, k, false, kScaleBF16), x, k, y, n, t, gemm_out_bf16(), 0, true);
}

void qe_gemm_w4_s(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t, void* st) {
    gemm_w4(mk_w4(q, s, n, k, false, kScaleBF16), x, k, y, n, t, gemm_out_bf16(), as_stream(st));
}

void qe_gemm_set_out_bf16(int on) { gemm_set_out_bf16(on != 0); }
void qe_gemm_set_sk_maxparts(int n) { gemm_set_sk_maxparts(n); }

void qe_xh_pack(const uint16_t* x, int k, int m, void* xh, int ldxh) {
    xh_pack(x, k, k, m, reinterpret_cast<uint16_t*>(xh), ldxh, 0);
}

void qe_gemv_w4h(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu, void* xh_ws,
                 void* yh) {
    CHECK(xh_ws != nullptr, "qe_gemv_w4h: needs the XH workspace xh_ws [m][k] fp16");
    gemv_workspace_init();
    xh_pack(x, k, k, m, reinterpret_cast<uint16_t*>(xh_ws), k, 0);
    const int ldy = glu ? n / 2 : n;
    gemv_h16(reinterpret_cast<const uint4*>(q), reinterpret_cast<const uint16_t*>(s), n, k, kScaleBF16, false, glu != 0,
             reinterpret_cast<const uint16_t*>(xh_ws), k, y, ldy, m, false, reinterpret_cast<uint16_t*>(yh), ldy, 0);
}

void qe_gemv_w4hx(const void* q, const void* s, int n, int k, const uint16_t* xh, float* y, int m, int glu, int ldx) {
    gemv_workspace_init();
    gemv_h16(reinterpret_cast<const uint4*>(q), reinterpret_cast<const uint16_t*>(s), n, k, kScaleBF16, false, glu != 0,
             xh, ldx, y, glu ? n / 2 : n, m, false, nullptr, 0, 0);
}

// the reference's wide H16 GEMV hook (src/capi.cpp:72-77, gemv_w4hx: 9..64 rows, false when unsupported): here 1 when
// the rows run as one launch (m <= 32 with the conditions of gemv_h16_one_launch), else 0 and nothing is written
int qe_gemv_w4hxx(const void* q, const void* s, int n, int k, const uint16_t* xh, float* y, int m, int glu, int ldx) {
    if (!gemv_h16_one_launch(n, k, false, xh, ldx, m)) return 0;
    gemv_workspace_init();
    gemv_h16(reinterpret_cast<const uint4*>(q), reinterpret_cast<const uint16_t*>(s), n, k, kScaleBF16, false, glu != 0,
             xh, ldx, y, glu ? n / 2 : n, m, false, nullptr, 0, 0);
    return 1;
}

void qe_gemv_w4h_ex(const void* q, const void* s, int n, int k, const uint16_t* xh, int ldx, void* y, int ldy, int m,
                    int flags, void* yh, int ldyh, void* stream) {
    gemv_workspace_init();
    gemv_h16(reinterpret_cast<const uint4*>(q), reinterpret_cast<const uint16_t*>(s), n, k,
             (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16, false, (flags & QE_GLU) != 0, xh, ldx, y, ldy, m,
             (flags & QE_OUT_BF16) != 0, reinterpret_cast<uint16_t*>(yh), ldyh, as_stream(stream));
}

void qe_quantize_w8(const uint16_t* w, int n, int k, void* dq, void* ds) {
    quantize_w8(w, n, k, reinterpret_cast<uint4*>(dq), reinterpret_cast<uint16_t*>(ds), 0);
}

void qe_gemv_w8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m) {
    gemv_workspace_init();
    const W8 w = mk_w8(q, s, n, k, false, kScaleBF16);
    for (int r0 = 0; r0 < m; r0 += kMaxGemvRows) {
        const int mm = m - r0 < kMaxGemvRows ? m - r0 : kMaxGemvRows;
        gemv_w8(w, x + (size_t)r0 * k, k, y + (size_t)r0 * n, n, mm, false, 0);
    }
}

void qe_glu_rows(const int32_t* q, const uint16_t* s, int n, int k, int32_t* dq, uint16_t* ds, int bits) {
    glu_interleave_rows(q, s, n, k, dq, ds, 0, bits);
}

// ---- Q8 (INT8 layer weights in the q8_layout.h byte order) ----
void qe_repack_q8(const int32_t* q, const uint16_t* s, int n, int k, void* dq, void* ds) {
    repack_q8(q, s, n, k, reinterpret_cast<uint4*>(dq), reinterpret_cast<uint16_t*>(ds), 0);
}

void qe_glu_rows8(const int32_t* q, const uint16_t* s, int n, int k, int32_t* dq, uint16_t* ds) {
    glu_interleave_rows(q, s, n, k, dq, ds, 0, 8);
}

void qe_gemv_q8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu, int h16,
                void* xh_ws, void* yh) {
    CHECK(!h16 || xh_ws != nullptr, "qe_gemv_q8: h16 needs the XH workspace xh_ws [m][k] fp16");
    CHECK(h16 || yh == nullptr, "qe_gemv_q8: yh (the XH copy) is an output of the h16 path");
    gemv_workspace_init();
    const int ldy = glu ? n / 2 : n;
    if (h16) {
        xh_pack(x, k, k, m, reinterpret_cast<uint16_t*>(xh_ws), k, 0);
        gemv_h16(reinterpret_cast<const uint4*>(q), reinterpret_cast<const uint16_t*>(s), n, k, kScaleBF16, true,
                 glu != 0, reinterpret_cast<const uint16_t*>(xh_ws), k, y, ldy, m, false,
                 reinterpret_cast<uint16_t*>(yh), ldy, 0);
        return;
    }
    W8 w = mk_w8(q, s, n, k, false, kScaleBF16);
    w.q8 = true;
    w.glu = glu != 0;
    const size_t esz = glu ? 2 : 4;
    for (int r0 = 0; r0 < m; r0 += kMaxGemvRows) {
        const int mm = m - r0 < kMaxGemvRows ? m - r0 : kMaxGemvRows;
        gemv_w8(w, x + (size_t)r0 * k, k, reinterpret_cast<char*>(y) + (size_t)r0 * ldy * esz, ldy, mm, false, 0);
    }
}

void qe_gemm_q8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t, int glu, int G, int ci) {
    (void)ci;
    if (G > 0) {  // W8A8 with activation group G (the reference's gemm_w4_i8 on a Q8 matrix)
        gemm_w4_i8(mk_w4(q, s, n, k, glu != 0, kScaleBF16), x, k, y, glu ? n / 2 : n, t, G, !glu && gemm_out_bf16(), 0,
                   true);
        return;
    }
    W8 w = mk_w8(q, s, n, k, false, kScaleBF16);
    w.q8 = true;
    w.glu = glu != 0;
    gemm_w8(w, x, k, y, glu ? n / 2 : n, t, !glu && gemm_out_bf16(), 0);
}

// ---------------------------------------------------------------- build-defined entry points
void qe_dequant_w4(const void* q, const void* s, int n, int k, int flags, uint16_t* out, void* st) {
    dequant_w4(mk_w4(q, s, n, k, false, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), out, as_stream(st));
}

void qe_gemv_w4_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                   int flags, void* st) {
    gemv_workspace_init();
    gemv_w4(mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y,
            ldy, m, (flags & QE_OUT_BF16) != 0, as_stream(st));
}

void qe_gemm_w4_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                   int flags, void* st) {
    gemm_w4(mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y,
            ldy, t, (flags & QE_OUT_BF16) != 0, as_stream(st));
}

void qe_gemm_w4h_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                    int flags, void* st) {
    gemm_w4h(mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y,
             ldy, t, (flags & QE_OUT_BF16) != 0, as_stream(st));
}

void qe_matmul_w4_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                     int flags, void* st) {
    gemv_workspace_init();
    matmul_w4(mk_w4(q, s, n, k, (flags & QE_GLU) != 0, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y,
              ldy, m, (flags & QE_OUT_BF16) != 0, as_stream(st));
}

void qe_tile_w8(const int8_t* w, const uint16_t* s, int n, int k, int per_channel, void* dq, void* ds, void* st) {
    tile_w8(w, s, n, k, reinterpret_cast<uint4*>(dq), reinterpret_cast<uint16_t*>(ds), per_channel != 0,
            as_stream(st));
}

void qe_dequant_w8(const void* q, const void* s, int n, int k, int flags, uint16_t* out, void* st) {
    const bool pc = (flags & QE_W8_PER_CHANNEL) != 0;
    dequant_w8(mk_w8(q, s, n, k, pc, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), out, as_stream(st));
}

void qe_gemv_w8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                   int flags, void* st) {
    gemv_workspace_init();
    const bool pc = (flags & QE_W8_PER_CHANNEL) != 0;
    gemv_w8(mk_w8(q, s, n, k, pc, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y, ldy, m,
            (flags & QE_OUT_BF16) != 0, as_stream(st));
}

void qe_gemm_w8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                   int flags, void* st) {
    const bool pc = (flags & QE_W8_PER_CHANNEL) != 0;
    gemm_w8(mk_w8(q, s, n, k, pc, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y, ldy, t,
            (flags & QE_OUT_BF16) != 0, as_stream(st));
}

void qe_gemm_w8a8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                     int flags, void* st) {
    const bool pc = (flags & QE_W8_PER_CHANNEL) != 0;
    gemm_w8a8(mk_w8(q, s, n, k, pc, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16), x, ldx, y, ldy, m,
              (flags & QE_OUT_BF16) != 0, as_stream(st));
}

// Worker::rows8 (reference src/flash/flash.cu:369-411): W8A8 for m >= 64 rows, k <= 4096 (the reference pre-pass's
// row staging limit, RQ_KMAX) and 8-element row strides, else its gemv_w8_rows (flash.cu:351-366): the W8A16 row GEMM
// for 16-byte aligned rows, else the W8A16 GEMV over blocks of up to 16 rows; fp32 out
void qe_rows8(const void* q, const void* s, int n, int k, int flags, const uint16_t* x, int ldx, float* y, int ldy,
              int m, void* st) {
    const bool pc = (flags & QE_W8_PER_CHANNEL) != 0;
    const W8 w = mk_w8(q, s, n, k, pc, (flags & QE_SCALE_F16) ? kScaleF16 : kScaleBF16);
    CHECK(m >= 1, "rows8: m = %d", m);
    if (m >= 64 && k <= 4096 && ldx % 8 == 0) {
        gemm_w8a8(w, x, ldx, y, ldy, m, false, as_stream(st));
    } else if (ldx % 8 == 0 && ((uintptr_t)x & 15) == 0) {
        gemm_w8(w, x, ldx, y, ldy, m, false, as_stream(st));
    } else {
        for (int r0 = 0; r0 < m; r0 += kMaxGemvRows)
            gemv_w8(w, x + (size_t)r0 * ldx, ldx, y + (size_t)r0 * ldy, ldy, std::min(kMaxGemvRows, m - r0), false,
                    as_stream(st));
    }
}

}  // extern "C"
