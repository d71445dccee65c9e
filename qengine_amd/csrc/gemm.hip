// Prefill GEMM (placeholder until the MFMA kernel lands) and the matmul() dispatch.
#include "qe_api.hpp"

void gemm_w4(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    (void)w; (void)x; (void)ldx; (void)c; (void)ldc; (void)t; (void)out_bf16; (void)st;
    CHECK(false, "gemm_w4: not available yet");
}

void gemm_w8(const W8& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    (void)w; (void)x; (void)ldx; (void)c; (void)ldc; (void)t; (void)out_bf16; (void)st;
    CHECK(false, "gemm_w8: not available yet");
}

void matmul_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    if (m > kMaxGemvW4Tokens) {
        gemm_w4(w, x, ldx, y, ldy, m, out_bf16, st);
        return;
    }
    const size_t esz = (w.glu || out_bf16) ? 2 : 4;
    for (int r0 = 0; r0 < m; r0 += kMaxGemvRows) {
        const int mm = m - r0 < kMaxGemvRows ? m - r0 : kMaxGemvRows;
        gemv_w4(w, x + (size_t)r0 * ldx, ldx, reinterpret_cast<char*>(y) + (size_t)r0 * ldy * esz, ldy, mm, out_bf16,
                st);
    }
}
