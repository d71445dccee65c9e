/* qe_oracle.c - CPU restatement of the reference's weight-only quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (qengine_amd/, include/) links, loads or calls this code;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker / CPU baseline.
 *
 * Every function cites the reference file:line whose behaviour it restates. Parity pins (what checks each
 * function against something other than itself) are listed in oracle/__init__.py and tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ 16-bit floats */
/* float -> bf16, round to nearest even; NaN -> quiet NaN (the rounding of __float2bfloat16 / torch .bfloat16()) */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}
float or_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* IEEE binary16 -> float (exact, subnormals included) */
float or_f16_to_f32(uint16_t h) {
    const int sign = h >> 15, exp = (h >> 10) & 31, man = h & 1023;
    float v;
    if (exp == 0) v = ldexpf((float)man, -24);
    else if (exp == 31) v = man ? NAN : INFINITY;
    else v = ldexpf((float)(man | 1024), exp - 25);
    return sign ? -v : v;
}
static inline float scale_f32(uint16_t s, int sdt) { return sdt ? or_f16_to_f32(s) : or_bf16_to_f32(s); }

/* ------------------------------------------------------------------ W4 */
/* compressed-tensors INT4 source: int32 [n][k/8], nibble j (LSB first) of word c is k = 8c + j, u = w + 8
 * (reference gemv.cuh:148-151, tools/convert_flash_next.py:6-9, tests/test_gemv.py:13-15). Returns w = u - 8. */
void or_unpack_w4(const int32_t* src, int n, int k, int8_t* w) {
    for (int r = 0; r < n; r++)
        for (int c = 0; c < k; c++) {
            const uint32_t word = (uint32_t)src[(size_t)r * (k / 8) + c / 8];
            w[(size_t)r * k + c] = (int8_t)((int)((word >> (4 * (c % 8))) & 15u) - 8);
        }
}

/* compressed-tensors -> W4 fragment layout (reference gemv.cu:515-549): destination u32 idx = ((r*(k/64) + c)*32
 * + lane)*4 + j holds rows 16r + g (+8), k0 = 64c + 16j + 2t (g = lane/4, t = lane%4), nibble slots
 * (row,k0) (row+8,k0) (row,k0+8) (row+8,k0+8) (row,k0+1) (row+8,k0+1) (row,k0+9) (row+8,k0+9) LSB first.
 * Scales [n][k/128] -> [n/16][k/128][16]. */
void or_repack_w4(const int32_t* src_q, const uint16_t* src_s, int n, int k, uint32_t* dq, uint16_t* ds) {
    const int chunks = k / 64, G = k / 128;
    for (int r = 0; r < n / 16; r++)
        for (int c = 0; c < chunks; c++)
            for (int lane = 0; lane < 32; lane++)
                for (int j = 0; j < 4; j++) {
                    const int g = lane / 4, t = lane % 4;
                    const int row = 16 * r + g, k0 = 64 * c + 16 * j + 2 * t;
                    const int rows[8] = {row, row + 8, row, row + 8, row, row + 8, row, row + 8};
                    const int ks[8] = {k0, k0, k0 + 8, k0 + 8, k0 + 1, k0 + 1, k0 + 9, k0 + 9};
                    uint32_t word = 0;
                    for (int sl = 0; sl < 8; sl++) {
                        const uint32_t sw = (uint32_t)src_q[(size_t)rows[sl] * (k / 8) + ks[sl] / 8];
                        word |= ((sw >> (4 * (ks[sl] % 8))) & 15u) << (4 * sl);
                    }
                    dq[(((size_t)r * chunks + c) * 32 + lane) * 4 + j] = word;
                }
    for (int r = 0; r < n / 16; r++)
        for (int gi = 0; gi < G; gi++)
            for (int i = 0; i < 16; i++) ds[((size_t)r * G + gi) * 16 + i] = src_s[(size_t)(16 * r + i) * G + gi];
}

/* dequantized weight d = bf16_rn((u - 8) * s): the reference's bf16 operand (gemv.cu:25-36 + __hmul2 at
 * gemv.cu:187-191; gemm.cu:68-77; tests/test_gemv.py:36 rounds the same way). (u-8)*s is exact in fp32. */
void or_dequant_w4(const int32_t* src_q, const uint16_t* src_s, int n, int k, int sdt, uint16_t* out) {
    const int G = k / 128;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; r++)
        for (int c = 0; c < k; c++) {
            const uint32_t word = (uint32_t)src_q[(size_t)r * (k / 8) + c / 8];
            const int w = (int)((word >> (4 * (c % 8))) & 15u) - 8;
            out[(size_t)r * k + c] = or_f32_to_bf16((float)w * scale_f32(src_s[(size_t)r * G + c / 128], sdt));
        }
}

/* GLU row interleave (reference gemv.cu:1151-1160): destination row dr of tile dr/16, j = dr%16, takes source
 * row j < 8 ? 8*tile + j : n/2 + 8*tile + j - 8. wpr = int32 words per row (k/8 INT4, k/4 INT8). */
void or_glu_rows(const int32_t* sq, const uint16_t* ss, int n, int k, int wpr, int32_t* dq, uint16_t* ds) {
    const int G = k / 128;
    for (int dr = 0; dr < n; dr++) {
        const int tile = dr / 16, j = dr % 16;
        const int sr = j < 8 ? 8 * tile + j : n / 2 + 8 * tile + (j - 8);
        memcpy(dq + (size_t)dr * wpr, sq + (size_t)sr * wpr, (size_t)wpr * 4);
        memcpy(ds + (size_t)dr * G, ss + (size_t)sr * G, (size_t)G * 2);
    }
}

/* ------------------------------------------------------------------ matmul */
/* y[m][n] = sum_k x[m][k] * w[n][k], x and w bf16, fp32 accumulation in k order (per output; the arithmetic of
 * the reference's fp32 dequantize-then-matmul check, tests/test_gemv.py:45 `x.float() @ wref.T`).
 * nthreads <= 0: all available. */
void or_matmul_bf16(const uint16_t* x, const uint16_t* w, int m, int n, int k, float* y, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    float* xf = (float*)malloc((size_t)m * k * sizeof(float));
    for (size_t i = 0; i < (size_t)m * k; i++) xf[i] = or_bf16_to_f32(x[i]);
#pragma omp parallel
    {
        float* wf = (float*)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
        for (int r = 0; r < n; r++) {
            const uint16_t* wr = w + (size_t)r * k;
            for (int c = 0; c < k; c++) wf[c] = or_bf16_to_f32(wr[c]);
            for (int t = 0; t < m; t++) {
                const float* xr = xf + (size_t)t * k;
                float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, a4 = 0.f, a5 = 0.f, a6 = 0.f, a7 = 0.f;
                int c = 0;
                for (; c + 8 <= k; c += 8) {
                    a0 += xr[c] * wf[c]; a1 += xr[c + 1] * wf[c + 1];
                    a2 += xr[c + 2] * wf[c + 2]; a3 += xr[c + 3] * wf[c + 3];
                    a4 += xr[c + 4] * wf[c + 4]; a5 += xr[c + 5] * wf[c + 5];
                    a6 += xr[c + 6] * wf[c + 6]; a7 += xr[c + 7] * wf[c + 7];
                }
                float a = ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7));
                for (; c < k; c++) a += xr[c] * wf[c];
                y[(size_t)t * n + r] = a;
            }
        }
        free(wf);
    }
    free(xf);
}

/* GLU epilogue on a [m][n] fp32 product of a GLU-interleaved matrix (reference gemv.cu:62-72, gemm.cu:198-216):
 * act[t][tile*8 + g] = bf16(silu(y[t][16 tile + g]) * y[t][16 tile + g + 8]) */
void or_glu_epilogue(const float* y, int m, int n, uint16_t* act) {
    for (int t = 0; t < m; t++)
        for (int tile = 0; tile < n / 16; tile++)
            for (int g = 0; g < 8; g++) {
                const float gate = y[(size_t)t * n + 16 * tile + g], up = y[(size_t)t * n + 16 * tile + g + 8];
                act[(size_t)t * (n / 2) + tile * 8 + g] = or_f32_to_bf16(gate / (1.f + expf(-gate)) * up);
            }
}

/* ------------------------------------------------------------------ W8 */
/* RTN INT8 group 128 (reference gemv.cu:1085-1116, closed form tests/test_w8.py:6-9): scale = bf16(amax/127),
 * q = clamp(rint(v / scale), -127, 127) (0 when the scale is 0). q int8 [n][k] row-major, s bf16 [n][k/128]. */
void or_quantize_w8(const uint16_t* w, int n, int k, int8_t* q, uint16_t* s) {
    const int G = k / 128;
    for (int r = 0; r < n; r++)
        for (int gi = 0; gi < G; gi++) {
            float mx = 0.f;
            for (int c = 0; c < 128; c++) {
                const float v = fabsf(or_bf16_to_f32(w[(size_t)r * k + gi * 128 + c]));
                if (v > mx) mx = v;
            }
            const uint16_t sb = or_f32_to_bf16(mx / 127.f);
            const float sc = or_bf16_to_f32(sb);
            const float div = sc > 0.f ? sc : 1.f;
            for (int c = 0; c < 128; c++) {
                float qv = rintf(or_bf16_to_f32(w[(size_t)r * k + gi * 128 + c]) / div);
                if (qv > 127.f) qv = 127.f;
                if (qv < -127.f) qv = -127.f;
                q[(size_t)r * k + gi * 128 + c] = (int8_t)qv;
            }
            s[(size_t)r * G + gi] = sb;
        }
}

/* byte offset of (row, k) in the W8 layout [n/16][k/32][32][16] (reference gemv.cu:1102-1113, inverse
 * src/tools/qe_w8q.cu:34-45) */
size_t or_w8_pos(int row, int c, int k) {
    const int rt = row / 16, rr = row % 16, ks = c / 16, col = c % 16;
    const int tq = (col % 8) / 2, half = col / 8, odd = col % 2;
    const int ln = (rr % 8) * 4 + tq;
    const int ai = (half * 2 + rr / 8) * 2 + odd;
    return (((size_t)rt * (k / 32) + ks / 2) * 32 + ln) * 16 + (ks % 2) * 8 + ai;
}

/* row-major int8 + scales -> W8 layout (reference tile_w8_kernel gemv.cu:1464-1477). per_channel (this build's
 * extension, no reference): scales [n] kept as they are. */
void or_tile_w8(const int8_t* q, const uint16_t* s, int n, int k, int per_channel, uint8_t* dq, uint16_t* ds) {
    for (int r = 0; r < n; r++)
        for (int c = 0; c < k; c++) dq[or_w8_pos(r, c, k)] = (uint8_t)q[(size_t)r * k + c];
    if (per_channel) {
        memcpy(ds, s, (size_t)n * 2);
        return;
    }
    const int G = k / 128;
    for (int r = 0; r < n; r++)
        for (int gi = 0; gi < G; gi++) ds[((size_t)(r / 16) * G + gi) * 16 + r % 16] = s[(size_t)r * G + gi];
}

/* d = bf16_rn(w * s) (exact product in fp32), row-major; s [n] per channel or [n][k/128] */
void or_dequant_w8(const int8_t* q, const uint16_t* s, int n, int k, int per_channel, int sdt, uint16_t* out) {
    const int G = k / 128;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; r++)
        for (int c = 0; c < k; c++) {
            const float sc = scale_f32(per_channel ? s[r] : s[(size_t)r * G + c / 128], sdt);
            out[(size_t)r * k + c] = or_f32_to_bf16((float)q[(size_t)r * k + c] * sc);
        }
}

/* ------------------------------------------------------------------ Q8 (INT8 layer weights) */
/* Byte position of weight (row, k) of an [N][K] matrix in the Q8 layout (reference src/kernels/q8_layout.h:29-37):
 * q [N/16][K/32][32 lanes][16 B]; lane (g, t) of tile r, 32-k chunk c: word 2 s + hi = row 16 r + g + 8 hi,
 * byte i = k 32 c + 16 s + 2 t + {0, 8, 1, 9}[i]. Restated from the layout comment; pinned against the header
 * itself (oracle/_ref) and by bijection / known answers in the tests. */
size_t or_q8_pos(int row, int k, int K) {
    const int r = row / 16, rr = row % 16, g = rr % 8, hi = rr / 8;
    const int c = k / 32, s = (k / 16) % 2, kk = k % 16;
    const int t = (kk % 8) / 2;                 /* kk = 2 t + {0, 8, 1, 9} */
    const int i = (kk >= 8 ? 1 : 0) + 2 * (kk % 2);
    return (((size_t)r * (K / 32) + c) * 32 + g * 4 + t) * 16 + (2 * s + hi) * 4 + i;
}

/* compressed-tensors 8-bit (int32 [n][k/4], byte b of word j = k 4 j + b, stored u = w + 128; reference
 * tools/quant_int8.py:102-105) + bf16 group-128 scales [n][k/128] -> Q8 bytes (signed w) + W4 scale layout
 * (reference repack_q8 gemv.cu:940-957, 1377-1383) */
void or_repack_q8(const int32_t* q, const uint16_t* s, int n, int k, uint8_t* dq, uint16_t* ds) {
    for (int r = 0; r < n; r++)
        for (int c = 0; c < k; c++) {
            const uint32_t u = ((uint32_t)q[(size_t)r * (k / 4) + c / 4] >> (8 * (c % 4))) & 0xFFu;
            dq[or_q8_pos(r, c, k)] = (uint8_t)(u ^ 0x80u);
        }
    const int G = k / 128;
    for (int r = 0; r < n; r++)
        for (int gi = 0; gi < G; gi++) ds[((size_t)(r / 16) * G + gi) * 16 + r % 16] = s[(size_t)r * G + gi];
}

/* compressed-tensors 8-bit source -> bf16 [n][k] = bf16_rn((u - 128) * s) */
void or_dequant_q8(const int32_t* q, const uint16_t* s, int n, int k, uint16_t* out) {
    const int G = k / 128;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; r++)
        for (int c = 0; c < k; c++) {
            const int u = (int)(((uint32_t)q[(size_t)r * (k / 4) + c / 4] >> (8 * (c % 4))) & 0xFFu);
            out[(size_t)r * k + c] = or_f32_to_bf16((float)(u - 128) * or_bf16_to_f32(s[(size_t)r * G + c / 128]));
        }
}

/* ------------------------------------------------------------------ MoE */
/* Router (reference flash_kernels.cuh:4351-4399 k_topk_rows; 4006-4089 k_route): top-`topk` experts of each
 * row by logit, ties: lower index first; weights w_i = exp(l_i - l_max) / sum_sel exp(l_j - l_max) (softmax
 * renormalised over the selection, norm_topk_prob). */
void or_moe_route(const float* logits, int T, int E, int topk, int32_t* sel, float* w) {
    int* taken = (int*)calloc((size_t)E, sizeof(int));
    for (int t = 0; t < T; t++) {
        const float* l = logits + (size_t)t * E;
        memset(taken, 0, (size_t)E * sizeof(int));
        for (int kk = 0; kk < topk; kk++) {
            int bi = -1;
            for (int e = 0; e < E; e++)
                if (!taken[e] && (bi < 0 || l[e] > l[bi])) bi = e;
            taken[bi] = 1;
            sel[(size_t)t * topk + kk] = bi;
        }
        const float lmax = l[sel[(size_t)t * topk]];
        float tot = 0.f;
        for (int kk = 0; kk < topk; kk++) tot += expf(l[sel[(size_t)t * topk + kk]] - lmax);
        for (int kk = 0; kk < topk; kk++) w[(size_t)t * topk + kk] = expf(l[sel[(size_t)t * topk + kk]] - lmax) / tot;
    }
    free(taken);
}

/* Sort & segment (token, k) pairs by expert (reference k_jobs_pf flash_kernels.cuh:6007-6100): cnt[e], exclusive
 * offsets off[0..E], list[off[e] + i] = pair index t*topk + k of the i-th pair routed to e, inv[pair] = slot.
 * Order inside an expert: ascending pair index (this build's choice; the reference's atomics leave it
 * unspecified, flash_kernels.cuh:6049-6051). */
void or_moe_segment(const int32_t* sel, int T, int E, int topk, int32_t* cnt, int32_t* off, int32_t* list,
                    int32_t* inv) {
    memset(cnt, 0, (size_t)E * sizeof(int32_t));
    for (int i = 0; i < T * topk; i++) cnt[sel[i]]++;
    off[0] = 0;
    for (int e = 0; e < E; e++) off[e + 1] = off[e] + cnt[e];
    int32_t* fill = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    for (int i = 0; i < T * topk; i++) {
        const int e = sel[i];
        const int slot = off[e] + fill[e]++;
        list[slot] = i;
        inv[i] = slot;
    }
    free(fill);
}

/* W8A8 row GEMM (reference k_rows_qt, src/flash/flash_pfq.cuh:520-651; the activations quantized by the caller as
 * k_x_to_r8, :473-518, does): per (token t, row r) and 128-k group g in k order, sum = the exact integer dot product
 * of xq[t] and w[r] over the group, p = rn_f32((float)sum * sx[t][g]) and y = fmaf(p, sw[r][g], y). The reference
 * computes p as fma(M + sum, sx, -M sx) with M = 1.5 * 2^23 (an int32 accumulator started at M's bit pattern):
 * M sx is exact (sx has 22 significant bits) and (M + sum) sx - M sx = sum sx before the one rounding, so p is the
 * same. sw: [n][k/128] floats, or [n] with per_channel (the same scale in every group). nthreads <= 0: all. */
void or_rows_w8a8(const int8_t* xq, const float* sx, const int8_t* w, const float* sw, int per_channel, int m, int n,
                  int k, float* y, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    const int ng = k / 128;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; r++) {
        const int8_t* wr = w + (size_t)r * k;
        for (int t = 0; t < m; t++) {
            const int8_t* xr = xq + (size_t)t * k;
            float acc = 0.f;
            for (int g = 0; g < ng; g++) {
                int32_t sum = 0;
                for (int c = 128 * g; c < 128 * g + 128; c++) sum += (int32_t)xr[c] * (int32_t)wr[c];
                const float p = (float)sum * sx[(size_t)t * ng + g];
                acc = fmaf(p, per_channel ? sw[r] : sw[(size_t)r * ng + g], acc);
            }
            y[(size_t)t * n + r] = acc;
        }
    }
}

/* silu(a) * b in fp32 */
float or_silu_mul(float a, float b) { return a / (1.f + expf(-a)) * b; }
