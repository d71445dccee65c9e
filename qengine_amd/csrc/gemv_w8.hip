// INT8 decode GEMV / skinny GEMM instantiations (kernel: gemv_impl.hpp); the scale dtype is a run-time value.
#include "gemv_impl.hpp"

using namespace qe_gemv;

void gemv_w8(const W8& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    CHECK(w.n > 0 && w.k > 0 && w.n % 16 == 0 && w.k % 128 == 0 && m >= 1 && m <= kMaxGemvRows, "gemv_w8 %d %d %d",
          w.n, w.k, m);
    CHECK(ldx >= w.k && ldx % 2 == 0 && ((uintptr_t)x & 3) == 0, "gemv_w8 ldx %d", ldx);
    CHECK(ldy >= (w.glu ? w.n / 2 : w.n), "gemv_w8 ldy %d", ldy);
    CHECK(!w.glu || w.q8, "gemv_w8: GLU is for Q8 matrices");
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    if (w.q8) launch_gemv<kFmtQ8, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else if (w.per_channel) launch_gemv<kFmtW8C, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else launch_gemv<kFmtW8G, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
}
