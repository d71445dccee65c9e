// Prefill GEMM on the W4 / W8 layouts for gfx950: C[t][n] = sum_k X[t][k] * W[n][k], bf16 MFMA, fp32 accumulate.
//
// The weights are dequantized once per block tile, in registers, to the reference's bf16 operand
// (bf16_rn((u - 8) * s) for INT4, bf16_rn(w * s) for INT8; reference gemm.cu:68-77) and staged in LDS next to the
// activation tile; v_mfma_f32_32x32x16_bf16 consumes both from LDS.
//   block: 256 threads (4 waves, 2 x 2), tile BM = 128 tokens x BN = 128 weight rows, BK = 64 (one W4 chunk)
//   wave: 64 x 64 = 2 x 2 MFMA 32x32 tiles, 4 k16 steps per BK
//   LDS: two stages of X [128][64] and W [128][64] bf16, rows of 128 B with the 16-byte chunks XOR-swizzled by
//        (row % 8) so the MFMA fragment reads (32 rows x 16 B per half-wave) spread over the banks
//   pipeline: the global loads of step k + 1 are issued before the MFMAs of step k; one barrier per step.
#include "mfma_tile.hpp"

namespace {

using namespace qe_tile;
constexpr int BM = 128, BN = 128, BK = 64, NTH = 256;
constexpr int kStageBytes = (BM + BN) * BK * 2;  // 32 KB

enum Fmt : int { kFmtW4 = 0, kFmtW8G = 1, kFmtW8C = 2 };
enum Out : int { kOutF32 = 0, kOutBF16 = 1, kOutGLU = 2 };

template <int FMT, int SDT>
__global__ void __launch_bounds__(NTH) gemm_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s,
                                                   int N, int K, const uint16_t* __restrict__ x, int ldx, int T,
                                                   void* __restrict__ c, int ldc, int out, int sdt) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n0 = blockIdx.x * BN, t0 = blockIdx.y * BM;
    const int G = K >> 7, KT = K / BK;

    // ---- X loads: 4 x 16 B per thread (row = idx / 8, chunk = idx % 8)
    u32x4_v xr[4];
    auto load_x = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = tid + i * NTH, r = idx >> 3, ch = idx & 7;
            const int tok = t0 + r;
            xr[i] = tok < T ? *reinterpret_cast<const u32x4_v*>(x + (size_t)tok * ldx + kt * BK + ch * 8)
                            : u32x4_v{0u, 0u, 0u, 0u};
        }
    };
    auto store_x = [&](char* xt) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = tid + i * NTH, r = idx >> 3, ch = idx & 7;
            *reinterpret_cast<u32x4_v*>(xt + swz(r, ch)) = xr[i];
        }
    };
    // ---- W loads. W4: one 16 B record per thread (tile tr = tid / 32 of 8, lane wl); W8: two (slabs)
    constexpr int WREC = FMT == kFmtW4 ? 1 : 2;
    const int tr = tid >> 5, wl = tid & 31, wg = wl >> 2, wt4 = wl & 3;
    const int wrow = tr * 16 + wg;  // rows wrow, wrow + 8 of the block tile
    const bool wvalid = n0 + tr * 16 < N;
    u32x4_v wr[WREC];
    uint16_t sr_lo, sr_hi;
    auto load_w = [&](int kt) {
        const size_t tile = (size_t)(n0 >> 4) + tr;
#pragma unroll
        for (int e = 0; e < WREC; e++) {
            const uint4* p = FMT == kFmtW4 ? q + (tile * (K >> 6) + kt) * 32 + wl
                                           : q + (tile * (K >> 5) + 2 * kt + e) * 32 + wl;
            wr[e] = wvalid ? __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p)) : u32x4_v{0u, 0u, 0u, 0u};
        }
        if (FMT == kFmtW8C) {
            sr_lo = wvalid ? s[n0 + wrow] : 0;
            sr_hi = wvalid ? s[n0 + wrow + 8] : 0;
        } else {
            const uint16_t* sp = s + (tile * G + (kt >> 1)) * 16;
            sr_lo = wvalid ? sp[wg] : 0;
            sr_hi = wvalid ? sp[wg + 8] : 0;
        }
    };
    auto store_w = [&](char* wtile) {
        const float s_lo = scale_rt<SDT>(sr_lo, sdt), s_hi = scale_rt<SDT>(sr_hi, sdt);
        if constexpr (FMT == kFmtW4) {
#pragma unroll
            for (int j = 0; j < 4; j++) dq_w4_word(wr[0][j], s_lo, s_hi, wtile, wrow, 16 * j + 2 * wt4);
        } else {
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int d = 0; d < 4; d++)  // slab e covers k 32 e .. 32 e + 31; dword d: k step d / 2, half d % 2
                    dq_w8_dword(wr[e][d], s_lo, s_hi, wtile, wrow, 32 * e + 16 * (d >> 1) + 8 * (d & 1) + 2 * wt4);
        }
    };

    // ---- MFMA tiles: wave (wm, wn) owns tokens wm*64 .. +64, rows wn*64 .. +64
    const int wm = wave >> 1, wn = wave & 1;
    f32x16_v acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][b][r] = 0.f;

    load_x(0);
    load_w(0);
    for (int kt = 0; kt < KT; kt++) {
        char* xt = lds + (kt & 1) * kStageBytes;
        char* wt = xt + BM * BK * 2;
        store_x(xt);
        store_w(wt);
        __syncthreads();
        if (kt + 1 < KT) {
            load_x(kt + 1);
            load_w(kt + 1);
        }
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            // fragment of lane l: row l % 32, k = 16 ks + 8 (l / 32) .. + 8 -> chunk 2 ks + l / 32
            const int fr = lane & 31, fc = 2 * ks + (lane >> 5);
            bf16x8_v af[2], bfr[2];
#pragma unroll
            for (int a = 0; a < 2; a++)
                af[a] = *reinterpret_cast<const bf16x8_v*>(xt + swz(wm * 64 + a * 32 + fr, fc));
#pragma unroll
            for (int b = 0; b < 2; b++)
                bfr[b] = *reinterpret_cast<const bf16x8_v*>(wt + swz(wn * 64 + b * 32 + fr, fc));
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[b], acc[a][b], 0, 0, 0);
        }
    }

    // ---- epilogue: lane l holds column n = l % 32 of each 32 x 32 tile, rows 8 (r / 4) + 4 (l / 32) + r % 4
    const int cj = lane & 31, ci = 4 * (lane >> 5);
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int n = n0 + wn * 64 + b * 32 + cj;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int tok = t0 + wm * 64 + a * 32 + 8 * (r >> 2) + ci + (r & 3);
                const float v = acc[a][b][r];
                if (out == kOutGLU) {
                    // gate = row g, up = row g + 8 of the 16-row tile: lanes j and j + 8
                    const float up = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                        0, __builtin_bit_cast(int, v), 0x128 /* row_ror:8 */, 0xF, 0xF, false));
                    if ((cj & 15) < 8 && tok < T && n < N)
                        reinterpret_cast<uint16_t*>(c)[(size_t)tok * ldc + (n >> 4) * 8 + (cj & 7)] =
                            f32_to_bf16(silu_f32(v) * up);
                } else if (tok < T && n < N) {
                    if (out == kOutBF16) reinterpret_cast<uint16_t*>(c)[(size_t)tok * ldc + n] = f32_to_bf16(v);
                    else reinterpret_cast<float*>(c)[(size_t)tok * ldc + n] = v;
                }
            }
        }
}

template <int FMT, int SDT>
void launch_gemm(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, int t, void* c, int ldc,
                 int out, int sdt, hipStream_t st) {
    const dim3 grid((unsigned)((n + BN - 1) / BN), (unsigned)((t + BM - 1) / BM)), block(NTH);
    gemm_kernel<FMT, SDT><<<grid, block, 2 * kStageBytes, st>>>(q, s, n, k, x, ldx, t, c, ldc, out, sdt);
    HIP_CHECK(hipGetLastError());
}

void gemm_check(int n, int k, const void* x, int ldx, int ldc, int t, bool glu) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && t >= 1, "gemm %d %d %d", n, k, t);
    CHECK(ldx >= k && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0, "gemm ldx %d (multiple of 8, x 16-byte aligned)", ldx);
    CHECK(ldc >= (glu ? n / 2 : n), "gemm ldc %d", ldc);
    CHECK((size_t)t < (size_t)65535 * BM, "gemm t %d", t);
}

}  // namespace

void gemm_w4(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    gemm_check(w.n, w.k, x, ldx, ldc, t, w.glu);
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    if (w.sdt == kScaleF16) launch_gemm<kFmtW4, kScaleF16>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, st);
    else launch_gemm<kFmtW4, kScaleBF16>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, st);
}

void gemm_w8(const W8& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    gemm_check(w.n, w.k, x, ldx, ldc, t, false);
    const int out = out_bf16 ? kOutBF16 : kOutF32;
    if (w.per_channel) launch_gemm<kFmtW8C, -1>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, st);
    else launch_gemm<kFmtW8G, -1>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, st);
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
