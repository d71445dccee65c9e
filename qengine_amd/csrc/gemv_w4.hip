// INT4 decode GEMV / skinny GEMM instantiations (kernel: gemv_impl.hpp).
#include "gemv_impl.hpp"

using namespace qe_gemv;

static void gemv_check(int n, int k, const void* x, int ldx, int ldy, int m, bool glu) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && m >= 1 && m <= kMaxGemvRows, "gemv %d %d %d", n, k, m);
    CHECK(ldx >= k && ldx % 2 == 0 && ((uintptr_t)x & 3) == 0, "gemv ldx %d (even, >= k, x 4-byte aligned)", ldx);
    CHECK(ldy >= (glu ? n / 2 : n), "gemv ldy %d", ldy);
}

void gemv_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    gemv_check(w.n, w.k, x, ldx, ldy, m, w.glu);
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    const QeConfig& cfg = qe_config();
    if (m == 1 && !cfg.batch_invariant && gemv1_w4(w, x, y, out, st)) return;  // 16-byte aligned x only
    // the matrix-core kernel for m >= skinny_min_m (every m with batch_invariant); rows that are not 16-byte aligned
    // take its 4-dword activation loads
    if (m >= cfg.skinny_min_m || cfg.batch_invariant) {
        skinny_w4_mfma(w, x, ldx, y, ldy, m, out, st);
        return;
    }
    if (w.sdt == kScaleF16) launch_gemv<kFmtW4, kScaleF16>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else launch_gemv<kFmtW4, kScaleBF16>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
}

bool gemv_h16_one_launch(int n, int k, bool q8, const uint16_t* xh, int ldx, int m) {
    return !q8 && m >= 1 && m <= kWideRows && n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && ldx >= k &&
           ldx % 64 == 0 && ((uintptr_t)xh & 15) == 0 && (m <= kMaxGemvRows || decode_groups(n, k) > 0);
}

void gemv_h16(const uint4* q, const uint16_t* s, int n, int k, int sdt, bool q8, bool glu, const uint16_t* xh, int ldx,
              void* y, int ldy, int m, bool out_bf16, uint16_t* yh, int ldyh, hipStream_t st) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && m >= 1, "gemv_h16 %d %d %d", n, k, m);
    CHECK(ldx >= k && ldx % 8 == 0 && ((uintptr_t)xh & 15) == 0, "gemv_h16: XH rows 16-byte aligned, ldx %d", ldx);
    CHECK(ldy >= (glu ? n / 2 : n), "gemv_h16 ldy %d", ldy);
    CHECK(!yh || (ldyh >= (glu ? n / 2 : n) && (glu ? n / 2 : n) % 64 == 0), "gemv_h16: yh needs %d columns, a "
          "multiple of 64 (ldyh %d)", glu ? n / 2 : n, ldyh);
    const int out = glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    const size_t esz = (glu || out_bf16) ? 2 : 4;
    // INT4 with an even K slicing: row blocks of up to 32 in one pass over the weights (the wide skinny kernel, the
    // rows' bits those of 16-row launches); else blocks of 16
    const int rb = !q8 && decode_groups(n, k) > 0 ? kWideRows : kMaxGemvRows;
    for (int r0 = 0; r0 < m; r0 += rb) {
        const int mm = m - r0 < rb ? m - r0 : rb;
        skinny_h16(q, s, n, k, sdt, q8, xh + (size_t)r0 * ldx, ldx, reinterpret_cast<char*>(y) + (size_t)r0 * ldy * esz,
                   ldy, mm, out, yh ? yh + (size_t)r0 * ldyh : nullptr, ldyh, st);
    }
}
