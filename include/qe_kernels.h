/* qe_kernels.h - C-ABI of libqe_kernels.so, the MI355X (gfx950) weight-only quantized matmul path.
 *
 * Every pointer argument is a DEVICE pointer unless stated; `stream` is a hipStream_t (NULL = default
 * stream). 16-bit floats cross the ABI as raw uint16_t bit patterns. A violated shape precondition prints
 * "check failed ..." to stderr and aborts (the reference's convention, src/common.h:27-36); the one
 * exception is qe_skinny_w4, which returns 0 for an unsupported shape (reference src/capi.cpp:79-83).
 *
 * Weight layouts are the reference's (src/kernels/gemv.cuh:7-16,33-40):
 *   W4 q: [N/16][K/64][32 lanes][4 x u32] repacked nibbles (u = w + 8), s: [N/16][K/128][16] 16-bit scales
 *   W8 q: [N/16][K/32][32 lanes][16 bytes] int8; s: group 128 -> [N/16][K/128][16]; per channel -> [N]
 * Preconditions: n % 16 == 0, k % 128 == 0, x rows 4-byte aligned with an even stride.
 */
#ifndef QE_KERNELS_H
#define QE_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QE_ABI_VERSION 1

/* flags of the *_ex entry points */
#define QE_SCALE_F16 1      /* scales are fp16 (default bf16) */
#define QE_OUT_BF16 2       /* y is bf16 (round to nearest even), default fp32 */
#define QE_GLU 4            /* GLU matrix (8 gate + 8 up rows per tile): y = bf16 silu(gate) * up, n / 2 cols */
#define QE_W8_PER_CHANNEL 8 /* W8 with one scale per output row, s = [N] (group = K) */

int qe_abi_version(void);

/* Kernel policy of this build, set explicitly (the reference reads scattered environment variables: QE_SKINNY*,
 * QE_GEMV_NW_*, src/kernels/gemv.cu:1349-1357, skinny.cu:563-570). Process-wide; set it before capturing graphs.
 *   skinny_min_m    smallest row count the W4 decode GEMV sends to the matrix-core skinny kernel (default 2)
 *   w8_mfma_min_m   the same for INT8 / Q8; 0 = automatic (1 where the m = 1 K slices hold >= 4 groups, else 2)
 *   batch_invariant 1: every decode row is computed by the same kernel whatever the row count, so a row's bits do
 *                   not depend on the batch (the reference's skinny == GEMV contract, skinny.cu:1-14); 0 (default):
 *                   m = 1 takes the faster m = 1 kernel, equal to the batched rows within 1e-5 * rms
 *   gemm_tune       1: every prefill GEMM times its candidates (tile configuration x split of the last partial round)
 *                   once per (shape, token bucket), outside graph capture, and keeps the fastest (as qe_gemm_w4_t
 *                   always does); 0 (default): a stored choice if any, else the cost model
 *   gemm_h16        1: the W4 prefill GEMM entry points (qe_gemm_w4*, the GEMM leg of qe_matmul_w4_ex) run the
 *                   reference's fp16-accumulate numerics (qe_gemm_w4h_ex below; the reference's QE_GEMM_H16 with
 *                   W4A8 off, src/kernels/gemm.cu:3360-3362,4047-4070); 0 (default): the bf16 MFMA GEMM
 * Out-of-range values abort with a "check failed" message. No counterpart function in the reference. */
typedef struct qe_config {
    int skinny_min_m;
    int w8_mfma_min_m;
    int batch_invariant;
    int gemm_tune;
    int gemm_h16;
    int reserved[3];
} qe_config_t;
void qe_get_config(qe_config_t* cfg);
void qe_set_config(const qe_config_t* cfg);

/* GEMM tuning table (reference TuneStore, src/kernels/gemm.cu:4116-4348, QE_TUNE_FILE): path = a text file that
 * holds the measured choices per device; entries already in it are loaded (a file of another build is ignored) and
 * every new choice rewrites it, so later processes reuse the choices (bit-identical results across restarts).
 * NULL or "": in memory only. qe_gemm_tune_clear forgets the choices (in memory; the file is left as it is). */
void qe_gemm_tune_file(const char* path);
void qe_gemm_tune_clear(void);
int qe_gemm_tune_entries(void);
/* Library-owned workspaces of the prefill GEMMs (the split-K partial sums, the fp16-accumulate and W4A8 / W8A8
 * pre-pass buffers) are kept per (device, stream): calls on one stream share a buffer (they run in order), calls on
 * two streams of a device use two, so concurrent streams (or graphs replayed on two streams) never overwrite each
 * other's workspace (the reference keeps them thread_local, src/kernels/gemm.cu:3258-3368). A buffer grows on a call
 * outside graph capture; during capture it is not grown (the GEMM then runs unsplit; a pre-pass aborts with a message).
 * qe_gemm_reserve sizes the split-K workspace of the current device's default stream before capturing (the
 * reference's gemm_reserve_ws); qe_gemm_reserve_s that of `stream`. */
void qe_gemm_reserve(size_t bytes);
void qe_gemm_reserve_s(size_t bytes, void* stream);
/* test hook: how many workspace buffers of a kind (0 split-K, 1 W4A8 / W8A8 pre-pass, 2 fp16-accumulate pre-pass)
 * the library holds, over all devices and streams. No counterpart in the reference. */
int qe_workspace_count(int kind);
/* Prefill GEMM with the reference's fp16-accumulate numerics (gemm_h_kernel + x_to_h_kernel,
 * src/kernels/gemm.cu:236-461): activations scaled per token to |x| <= 16 (xs = amax / 16) and rounded to fp16,
 * weights as the exact integers u - 8 in fp16, each 64-k chunk's partial rounded to fp16 (once; the reference rounds
 * after every 16-k MMA step, so the bits are not the reference's) and scaled by its group scale into fp32, the token
 * scale in the epilogue. flags: QE_SCALE_F16, QE_OUT_BF16, QE_GLU (y = the bf16
 * activation [t][n / 2]). The pre-pass buffer (t * (2 k + 4) bytes) is the library's, one per (device, stream),
 * grown on first use; qe_gemm_h_reserve(k, t) sizes the default stream's, qe_gemm_h_reserve_s that of `stream`,
 * before graph capture (a capture that needs more aborts with a message).
 * No single counterpart function in the reference (its gemm_w4 picks this path by QE_GEMM_H16); also reached
 * through qe_gemm_w4* with qe_config_t.gemm_h16 = 1. */
void qe_gemm_w4h_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                    int flags, void* stream);
void qe_gemm_h_reserve(int k, int t);
void qe_gemm_h_reserve_s(int k, int t, void* stream);
/* W4A8 prefill GEMM, the reference's default prefill numerics (gemm_w4_i8 = x_to_i8_kernel + gemm_i8*_kernel,
 * src/kernels/gemm.cu:463-594,4513-4518): activations quantized per (token, G-group), G = 32, 64 or 128, to int8
 * with sx = amax / 127 (two lowest mantissa bits cleared) and q = rn(x / sx); weights as the exact int8 u - 8;
 * int32 dot products per G-group on the int8 matrix cores, added at sx * sw in fp32. qe_gemm_w4_i8 replaces
 * reference src/capi.cpp:104 (y fp32 [t][n], or bf16 after qe_gemm_set_out_bf16(1); bf16 scales), qe_gemm_w4_i8_glu
 * src/capi.cpp:109 (act bf16 [t][n/2] of a GLU matrix); ci / ks (the reference's tile candidate and kernel variant)
 * are accepted and ignored. qe_gemm_w4_i8_ex: strides, stream, flags QE_SCALE_F16 / QE_OUT_BF16 / QE_GLU. The
 * pre-pass buffer (t * (k + k / 8) bytes) is the library's, one per (device, stream), grown on first use;
 * qe_gemm_i8_reserve(k, t) sizes the default stream's, qe_gemm_i8_reserve_s that of `stream`, before graph capture. */
void qe_gemm_w4_i8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t, int G, int ci,
                   int ks);
void qe_gemm_w4_i8_glu(const void* q, const void* s, int n, int k, const uint16_t* x, void* act, int t, int G, int ci,
                       int ks);
void qe_gemm_w4_i8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                      int G, int flags, void* stream);
void qe_gemm_i8_reserve(int k, int t);
void qe_gemm_i8_reserve_s(int k, int t, void* stream);
/* test hook: qe_gemm_w4_ex with a given choice instead of the tuner's (cfg 0: 256 x 256 tiles, 1: 256 x 128; ks: K
 * ranges of the last partial round's tiles, 1 / 2 / 4); returns 1 if that split applies to the shape (else it runs
 * unsplit and returns 0). The reference's QE_GEMM_FORCE (src/kernels/gemm.cu:4376-4394). */
int qe_gemm_w4_choice(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                      int flags, int cfg, int ks, void* stream);
/* test hook: the one-pass decode GEMM of qe_matmul_w4_ex for m = 1..64 rows whatever the dispatch would pick (the
 * weights read once for all rows, as the reference's wide decode GEMVs, src/kernels/gemv_x.cu:902-980; this build's
 * decode numerics: the exact products (u - 8) x summed in fp32 and scaled once per 128-k group). Returns 0 without
 * running when the shape does not fit it (n % 64, x not 16-byte aligned or ldx % 8, K / 64 not an even number of
 * steps per wave), else 1. */
int qe_matmul_w4_onepass_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy,
                            int m, int flags, void* stream);

/* Measurement helper (no reference counterpart): streams the n*k/2 record bytes of a W4 matrix with the launch shape
 * of the m = 1 decode GEMV (n/16 blocks, its K slices) and does nothing else, the HBM read floor that GEMV is held
 * against. sink: n/16 dwords (written only on a 2^-32 chance, so the loads cannot be dropped). */
void qe_read_probe(const void* q, int n, int k, uint32_t* sink, void* stream);
/* Measurement helper (no reference counterpart): the shader clock in MHz, counted by one lane over 50 us of the
 * constant-rate wall clock (clock64 / wall_clock64); synchronizes the stream and allocates 16 bytes. The bench reports
 * it beside the GEMV time, which follows the clock of the box it runs on. */
float qe_clock_probe_mhz(void* stream);

/* ---- reference-named hooks (src/capi.cpp): bf16 scales, fp32 outputs, default stream ---- */

/* Library set-up for the current device (CU count, the address of the device's scratch array used by
 * qe_moe_w4_noalloc); call once per device before any graph capture. Replaces gemv_workspace_init, reference
 * src/capi.cpp:131 / gemv.cuh:51. */
void qe_gemv_workspace_init(void);

/* compressed-tensors int32 [n][k/8] (nibbles LSB first, u = w + 8) + scales [n][k/128] -> W4 layout
 * (dq: n*k/2 bytes, ds: n*k/128 16-bit). Replaces reference src/capi.cpp:13 (repack_w4, gemv.cu:1686-1694). */
void qe_repack_w4(const int32_t* q, const uint16_t* s, int n, int k, void* dq, void* ds);

/* y[m][n] (fp32, stride n) = x[m][k] (bf16, stride k) . W^T; any m (1..16 rows: the decode GEMV; 17..64: the
 * one-pass decode GEMM where the shape fits it and it is the faster choice (N >= 64 x the CU count, K without an even
 * slicing of the skinny kernel, more than 48 rows on matrices of >= ~26 M weights), else the skinny kernel's 32- and
 * 16-row launches, which batch_invariant always takes; the prefill GEMM above, as qe_matmul_w4_ex).
 * Replaces reference src/capi.cpp:47 (gemv_w4, gemv.cu:1585). */
void qe_gemv_w4(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m);

/* as qe_gemv_w4; glu != 0: y is the bf16 activation [m][n/2] = bf16(silu(gate) * up).
 * Replaces reference src/capi.cpp:52. */
void qe_gemv_w4g(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu);

/* skinny GEMM, bit-identical to qe_gemv_w4g for every row count (it is qe_gemv_w4g's decode dispatch); m = 1..32
 * (the reference's skinny_w4 range, skinny.cu:572): 17..32 rows run as one launch (the one-pass kernel where the
 * dispatch picks it, else the wide skinny kernel), which needs 16-byte aligned rows and an even K slicing. Returns 0 (nothing
 * written) when the shape is unsupported, 1 when it ran. Replaces reference src/capi.cpp:79-83 (skinny_w4,
 * skinny.cu:572-604). */
int qe_skinny_w4(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu);

/* qe_gemv_w4 on an explicit stream. Replaces reference src/capi.cpp:101. */
void qe_gemv_w4_s(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, void* stream);

/* ---- H16 decode numerics (the reference's default decode, src/kernels/gemv_h16.cuh, gemv.cu:1537-1583) ----
 * XH layout: fp16 x / 16 with |x| clamped to 2047, the columns of each 64-k chunk permuted (k bits b0..b5 ->
 * b0 | b3<<1 | b4<<2 | b5<<3 | b1<<4 | b2<<5). Weights as exact integers in fp16, f16 MFMA over each 64-k chunk, the
 * chunk partial rounded to fp16, then added to fp32 at group scale x 16. Every row count gives the same bits per row.
 * Not bit-identical to the reference, which rounds its fp16 accumulator after every 16-k MMA step (here once per 64-k
 * chunk; the difference is bounded by the tests). Replaces reference src/capi.cpp:55-66. */
/* bf16 x [m][k] -> XH [m][ldxh] (k % 64 == 0) */
void qe_xh_pack(const uint16_t* x, int k, int m, void* xh, int ldxh);
/* packs x into xh_ws [m][k] fp16, then the H16 GEMV; glu: y is the bf16 act [m][n/2]; yh (optional): XH copy of y */
void qe_gemv_w4h(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu, void* xh_ws,
                 void* yh);
/* x already XH, stride ldx */
void qe_gemv_w4hx(const void* q, const void* s, int n, int k, const uint16_t* xh, float* y, int m, int glu, int ldx);
/* the wide H16 GEMV (reference src/capi.cpp:72-77, gemv_w4hx): returns 1 when the m rows ran as one launch, 0 (nothing
 * written) when unsupported: m 1..32 (17..32 rows need an even K slicing; the reference's 33..64 return 0 here, its
 * callers then take qe_gemv_w4hx), ldx % 64 == 0, xh 16-byte aligned. Bit-identical to qe_gemv_w4hx. */
int qe_gemv_w4hxx(const void* q, const void* s, int n, int k, const uint16_t* xh, float* y, int m, int glu, int ldx);
/* build-defined: scales dtype / output bf16 / GLU by flags, explicit strides and stream, optional yh [m][ldyh] */
void qe_gemv_w4h_ex(const void* q, const void* s, int n, int k, const uint16_t* xh, int ldx, void* y, int ldy, int m,
                    int flags, void* yh, int ldyh, void* stream);

/* prefill GEMM: c[t][n] (fp32, or bf16 after qe_gemm_set_out_bf16(1)) = x[t][k] . W^T.
 * Replaces reference src/capi.cpp:84 (gemm_w4, gemm.cu:4361). */
void qe_gemm_w4(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t);
/* the tuned entry of the reference (src/capi.cpp:116); same kernel selection as qe_gemm_w4 here */
void qe_gemm_w4_t(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t);
/* qe_gemm_w4 on an explicit stream. Replaces reference src/capi.cpp:97. */
void qe_gemm_w4_s(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t, void* stream);
/* on != 0: later non-GLU GEMM calls write bf16 (round to nearest even) into y viewed as bf16 [t][n].
 * Replaces reference src/capi.cpp:114 (gemm_set_out_bf16, gemm.cu:4363-4375). */
void qe_gemm_set_out_bf16(int on);
/* run-time cap of the stream-K split: later prefill GEMM calls (W4, W8 / Q8 bf16-activation GEMMs) split the tiles
 * of their last partial round into at most n K ranges (n <= 0: no cap, the default; splits here are 1, 2 or 4, so
 * n = 1 turns the split off and n = 2 or 3 allows 2). Applies to the cost model's, the tuner's and a stored choice
 * alike (a stored split above the cap runs as the largest allowed one). Replaces reference src/capi.cpp:115
 * (gemm_set_sk_maxparts, gemm.cu:3485-3496,4359). */
void qe_gemm_set_sk_maxparts(int n);

/* RTN INT8 group-128 quantization of a row-major bf16 [n][k] into the W8 layout: scale = bf16(amax/127),
 * q = clamp(rint(v/scale), -127, 127). Replaces reference src/capi.cpp:124 (quantize_w8, gemv.cu:1085-1116). */
void qe_quantize_w8(const uint16_t* w, int n, int k, void* dq, void* ds);

/* W8 (group 128, bf16 scales) GEMV, y fp32 [m][n], m = 1..64. Replaces reference src/capi.cpp:127. */
void qe_gemv_w8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m);

/* gate/up row interleave into the GLU tile order (8 gate rows, 8 up rows per tile) of a compressed-tensors
 * matrix, bits 4 (int32 [n][k/8]) or 8 (int32 [n][k/4]). Replaces reference src/capi.cpp:23 (qe_glu_rows8) and
 * glu_interleave_rows (gemv.cu:1371-1375) for both widths. */
void qe_glu_rows(const int32_t* q, const uint16_t* s, int n, int k, int32_t* dq, uint16_t* ds, int bits);

/* ---- Q8: INT8 layer weights in the reference's Q8 byte order (src/kernels/q8_layout.h:1-37), bf16 group-128 scales
 * in the W4 scale layout ---- */

/* compressed-tensors 8-bit int32 [n][k/4] (byte b of word j = k 4j + b, u = w + 128) + bf16 [n][k/128] -> Q8 (dq:
 * n * k bytes, ds: W4 scale layout). Replaces reference src/capi.cpp:19 (repack_q8, gemv.cu:940-957,1377-1383). */
void qe_repack_q8(const int32_t* q, const uint16_t* s, int n, int k, void* dq, void* ds);

/* gate/up row interleave of an 8-bit compressed-tensors matrix (GLU layout, before qe_repack_q8).
 * Replaces reference src/capi.cpp:23 (glu_interleave_rows, bits 8). */
void qe_glu_rows8(const int32_t* q, const uint16_t* s, int n, int k, int32_t* dq, uint16_t* ds);

/* decode GEMV of a Q8 matrix, y fp32 [m][n] (glu: the bf16 activation [m][n/2]), any m (row blocks of 16).
 * Replaces reference src/capi.cpp:28. h16 = 1: the H16 numerics (x packed into xh_ws [m][k] fp16 in the XH layout,
 * w / 16 in fp16, f16 MFMA per 64-k chunk rounded to fp16, flushed into fp32 at scale x 256), and yh (if not NULL)
 * receives the outputs again in the XH layout [m][n or n/2] (n or n/2 a multiple of 64); h16 = 0: fp32 accumulation of
 * bf16 products, xh_ws unused, yh must be NULL. */
void qe_gemv_q8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int m, int glu, int h16,
                void* xh_ws, void* yh);

/* prefill GEMM of a Q8 matrix, y fp32 [t][n] (or bf16 after qe_gemm_set_out_bf16(1); glu: the bf16 activation
 * [t][n/2]). Replaces reference src/capi.cpp:41. G > 0: W8A8 with activation group G (32, 64, 128; the reference's
 * gemm_w4_i8 on a Q8 matrix: int8 activations per (token, G-group) as in qe_gemm_w4_i8, the Q8 bytes as the int8
 * weights); G = 0: the bf16 MFMA GEMM on bf16_rn(w * s) tiles. ci (the reference's tile candidate) is ignored. */
void qe_gemm_q8(const void* q, const void* s, int n, int k, const uint16_t* x, float* y, int t, int glu, int G, int ci);

/* ---- build-defined entry points (no reference counterpart; BASELINE workloads: fp16 scales, bf16 out) ---- */

/* W4 -> bf16 row-major [n][k], d = bf16_rn((u - 8) * s) (the reference's dequantized weight, gemv.cu:25-36,
 * gemm.cu:68-77, tests/test_gemv.py:36). flags: QE_SCALE_F16. */
void qe_dequant_w4(const void* q, const void* s, int n, int k, int flags, uint16_t* out, void* stream);

/* decode GEMV / skinny GEMM, m = 1..16, x rows of stride ldx, y rows of stride ldy.
 * flags: QE_SCALE_F16 | QE_OUT_BF16 | QE_GLU. Deterministic. m = 1 runs the m = 1 matrix-core kernel (gemv1),
 * m = 2..16 the matrix-core skinny kernel, whose rows are bit-identical for every m in 2..16 (a row does not depend
 * on the other rows of the batch); the two kernels agree to ~1e-6 relative (fp32 sums in another order), and with
 * qe_config_t.batch_invariant set m = 1 takes the skinny kernel too. Activation rows that are not 16-byte aligned
 * (x, or ldx not a multiple of 8) take the VALU decode kernel for every m. */
void qe_gemv_w4_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                   int flags, void* stream);

/* prefill GEMM (bf16 MFMA), any t >= 1. flags: QE_SCALE_F16 | QE_OUT_BF16 | QE_GLU. */
void qe_gemm_w4_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                   int flags, void* stream);

/* GEMV for m <= 64 (row blocks of 16), GEMM above: the reference's matmul() dispatch (gemv.cuh:187-190) with the
 * decode range widened from 32 to 64 rows (measured faster on MI355X; every row of a 1..64-row call has the bits it
 * has alone). */
void qe_matmul_w4_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                     int flags, void* stream);

/* row-major int8 [n][k] + scales -> W8 layout; per_channel: s is [n] (copied), else [n][k/128] */
void qe_tile_w8(const int8_t* w, const uint16_t* s, int n, int k, int per_channel, void* dq, void* ds, void* stream);

/* W8 -> bf16 row-major [n][k], d = bf16_rn(w * s). flags: QE_SCALE_F16 | QE_W8_PER_CHANNEL. */
void qe_dequant_w8(const void* q, const void* s, int n, int k, int flags, uint16_t* out, void* stream);

/* INT8 W8A16 GEMV (m = 1..16) / GEMM (any t). flags: QE_SCALE_F16 | QE_OUT_BF16 | QE_W8_PER_CHANNEL. */
void qe_gemv_w8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                   int flags, void* stream);
void qe_gemm_w8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int t,
                   int flags, void* stream);

/* W8A8 row GEMM of a W8 matrix, the reference's prefill numerics for INT8 matrices (k_x_to_r8 + k_rows_qt,
 * src/flash/flash_pfq.cuh:473-651): the activations are quantized per (row, 128-k group), sx = amax / 127 with the
 * two lowest mantissa bits cleared (1 for a zero group), q = rn(x * fp32(1 / sx)); each group's int8 x int8 dot
 * product is summed exactly in int32 and y = fma(rn(float(sum) * sx), sw, y) over the groups in k order, the
 * reference's arithmetic to the bit. Group-128 or per-channel (QE_W8_PER_CHANNEL) scales, QE_SCALE_F16,
 * QE_OUT_BF16; any m >= 1, k % 128 == 0. The pre-pass buffer (m * (k + k / 8) bytes) is the one of qe_gemm_w4_i8
 * (qe_gemm_i8_reserve sizes it). qe_rows8 is the reference's dispatch, Worker::rows8 (src/flash/flash.cu:369-411):
 * W8A8 for m >= 64, k <= 4096 and ldx % 8 == 0, else the W8A16 GEMM of qe_gemm_w8_ex for 16-byte aligned rows and
 * the W8A16 GEMV of qe_gemv_w8_ex (blocks of 16 rows) otherwise; y fp32. */
void qe_gemm_w8a8_ex(const void* q, const void* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                     int flags, void* stream);
void qe_rows8(const void* q, const void* s, int n, int k, int flags, const uint16_t* x, int ldx, float* y, int ldy,
              int m, void* stream);

/* ---- MoE grouped INT4 expert layer (one GPU, every expert local). No reference C-ABI exists for it: it replaces
 * Worker::moe (reference src/flash/flash.cu:4842-5020) and its kernels k_topk_rows / k_jobs_pf / k_moe_* with the
 * expert weights in the Flash-Next group-record format (src/flash/flash.h:203-218, fp16 scales): record (e, g) =
 * [gq: 256 GLU rows x H W4][gs][dq: H rows x 128 W4][ds], NGRP = I / 128 records per expert, expert-major. ---- */

/* top-k routing: sel int32 [T][topk], w fp32 [T][topk] = exp(l_i - l_max) / sum_sel exp(l_j - l_max); ties: lower
 * expert index first (reference k_topk_rows, flash_kernels.cuh:4351-4399). E <= 1024, topk <= 32. */
void qe_moe_route(const float* logits, int T, int E, int topk, int32_t* sel, float* w, void* stream);

/* sort & segment (token, k) pairs by expert (reference k_jobs_pf, flash_kernels.cuh:6007-6100): off [E+1]; per slot
 * (expert-major, ascending pair t*topk+k inside an expert): slot_pair, slot_tok, slot_w; inv [T*topk] = slot of a
 * pair; jobs int32 [2 * n] = (expert, first row) of `chunk`-row jobs, njobs [1]. Deterministic. topk <= 16. */
void qe_moe_segment(const int32_t* sel, const float* w, int T, int E, int topk, int chunk, int32_t* off,
                    int32_t* slot_pair, int32_t* slot_tok, float* slot_w, int32_t* inv, int32_t* jobs, int32_t* njobs,
                    void* stream);

/* device workspace of qe_moe_w4 for these sizes, and the bytes of one expert's records */
size_t qe_moe_workspace_bytes(int T, int E, int topk, int H, int I);
size_t qe_moe_record_bytes(int H, int I);

/* one MoE layer: out [T][H] (fp32, or bf16 with QE_OUT_BF16) = sum_k w_k * down_e(silu(gate_e x) * up_e x) for the
 * top-k experts e of each token; logits fp32 [T][E], x bf16 [T][H]. H % 512 == 0, I % 128 == 0. Numerics: gate_up
 * multiplies x by bf16_rn((u - 8) s), the activation silu(gate) up w_k is kept as fp16 of act / 16, down multiplies it
 * by fp16_rn((u - 8) s) and each (token, k) result is kept as an fp16 slot (value / 16), summed in k order in fp32
 * (the reference's fp16 intermediates, flash_kernels.cuh:6185,6308,6421-6482); deterministic. */
void qe_moe_w4(const float* logits, const uint16_t* x, const void* records, int T, int E, int topk, int H, int I,
               void* out, int flags, void* workspace, size_t ws_bytes, void* stream);

/* allocation-free qe_moe_w4: no counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the workspace is the
 * library's own per-device scratch array of QE_MOE_SCRATCH_BYTES (held by every GPU that loads the library until the
 * process ends). Sizes whose qe_moe_workspace_bytes exceeds it are rejected (abort with a message). Calls on one GPU
 * share the array: calls that overlap on one GPU (two streams) race. Nothing in it needs clearing between calls. */
#define QE_MOE_SCRATCH_BYTES (8 << 20)
void qe_moe_w4_noalloc(const float* logits, const uint16_t* x, const void* records, int T, int E, int topk, int H,
                       int I, void* out, int flags, void* stream);

/* load time: compressed-tensors experts -> group records (reference loader, src/flash/flash.cu:1555-1611).
 * gate_up int32 [E][2I][H/8] (gate rows then up rows) + fp16 [E][2I][H/128]; down int32 [E][H][I/8] + fp16
 * [E][H][I/128]; records: E * qe_moe_record_bytes(H, I) bytes. One kernel on `stream` (stream-ordered, no
 * allocation, no synchronization). */
void qe_moe_pack_w4(const int32_t* gu_q, const uint16_t* gu_s, const int32_t* dn_q, const uint16_t* dn_s, int E, int H,
                    int I, void* records, void* stream);

/* ---- on-disk weights: .safetensors files (host, memory-mapped) and the quantized-matrix loader ----
 * qe_st_open maps a file and indexes its tensors by name (reference SafeTensors::open, src/safetensors.h:40; a
 * malformed file aborts with a message); qe_st_close unmaps it. qe_st_count / qe_st_name list the names (sorted);
 * qe_st_tensor is the reference's has / get (src/safetensors.h:41-42): 0 if absent, else the dtype string
 * ("I32", "BF16", ... up to 11 chars + NUL into dtype[12]), shape (up to 8 dims), the mapped bytes. Host only. */
void* qe_st_open(const char* path);
void qe_st_close(void* st);
int qe_st_count(void* st);
const char* qe_st_name(void* st, int i);
int qe_st_tensor(void* st, const char* name, char* dtype, int64_t* shape, int* ndim, const void** data,
                 size_t* nbytes);
/* A quantized matrix from compressed-tensors tensors <names[i]>.weight_packed (int32) / .weight_scale (bf16 or
 * fp16, per 128-k group): rows [r0[i], r1[i]) of each name in order, columns [c0, c1) (c0 < 0: all), bits per
 * weight from the packed width (4: W4 layout, dq n*k/2 bytes; 8: Q8 layout, n*k bytes; ds n*k/128 16-bit), GLU
 * (gate rows then up rows) interleaved per 16-row tile before the repack. Replaces reference Worker::load_w4
 * (src/model.cpp:994-1059). qe_load_w4_dims: the matrix's n, k, bits, scale dtype (0 bf16, 1 fp16) without loading
 * (host only); qe_load_w4 copies, interleaves and repacks on `stream` and returns when done. */
void qe_load_w4_dims(void* st, const char* const* names, const int* r0, const int* r1, int nspec, int c0, int c1,
                     int* n, int* k, int* bits, int* sdt);
void qe_load_w4(void* st, const char* const* names, const int* r0, const int* r1, int nspec, int c0, int c1, int glu,
                void* dq, void* ds, void* stream);

#ifdef __cplusplus
}
#endif
#endif
