// INT8 decode GEMV / skinny GEMM instantiations (kernel: gemv_impl.hpp); the scale dtype is a run-time value.
#include "gemv_impl.hpp"

using namespace qe_gemv;

// smallest m that the matrix-core kernel takes: the config's w8_mfma_min_m if set, else 2, or 1 where the m = 1 slicing
// has >= 4 groups per wave (measured, N = 8192: m = 1 at K = 5120 (5-group slices) 10.9 -> 8.9 us on the matrix
// cores; at K = 2048 (2-group slices) the VALU GEMV is faster, 5.0 vs 6.0 us); batch_invariant: always 1
static int w8_mfma_min_m(int n, int k) {
    const QeConfig& cfg = qe_config();
    if (cfg.batch_invariant) return 1;
    if (cfg.w8_mfma_min_m > 0) return cfg.w8_mfma_min_m;
    return decode_groups(n, k) >= 4 ? 1 : 2;
}

void gemv_w8(const W8& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    CHECK(w.n > 0 && w.k > 0 && w.n % 16 == 0 && w.k % 128 == 0 && m >= 1 && m <= kMaxGemvRows, "gemv_w8 %d %d %d",
          w.n, w.k, m);
    CHECK(ldx >= w.k && ldx % 2 == 0 && ((uintptr_t)x & 3) == 0, "gemv_w8 ldx %d", ldx);
    CHECK(ldy >= (w.glu ? w.n / 2 : w.n), "gemv_w8 ldy %d", ldy);
    CHECK(!w.glu || w.q8, "gemv_w8: GLU is for Q8 matrices");
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    // m = 1 on per-channel records: the streaming matrix-core kernel (gemv1.hip) where it takes the shape (not under
    // batch_invariant, where m = 1 runs the batched rows' kernel)
    if (m == 1 && !qe_config().batch_invariant && gemv1_w8c(w, x, y, out, st)) return;
    // the matrix-core kernel from w8_mfma_min_m rows (rows that are not 16-byte aligned take its 4-dword loads)
    if (m >= w8_mfma_min_m(w.n, w.k)) {
        skinny_w8_mfma(w, x, ldx, y, ldy, m, out, st);
        return;
    }
    if (w.q8) launch_gemv<kFmtQ8, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else if (w.per_channel) launch_gemv<kFmtW8C, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else launch_gemv<kFmtW8G, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
}
