// C++ kernel API of qengine_amd: the MI355X counterpart of the reference's kernel header
// (src/kernels/gemv.cuh:17-200). Same weight layouts, same argument meaning, hipStream_t instead of
// cudaStream_t. All pointers are device pointers; the caller owns weights, activations and outputs, the
// library owns its workspaces (qe_gemv_workspace_init, once per device before any graph capture).
#pragma once
#include "qe_common.hpp"

// W4 layout (symmetric INT4, group 128 along K, stored nibble u = w + 8), reference gemv.cuh:12-16:
//   q: [N/16][K/64][32 lanes][4 x u32]   s: [N/16][K/128][16] 16-bit (bf16 or fp16, `sdt`)
// glu: each 16-row tile holds 8 gate rows then the 8 matching up rows; the output is
// act[t][i] = bf16(silu(gate_i) * up_i) with n / 2 columns (gemv.cuh:20-22).
struct W4 {
    const uint4* q = nullptr;
    const uint16_t* s = nullptr;
    int n = 0, k = 0;
    bool glu = false;
    int sdt = kScaleBF16;
};
// W8 layout (symmetric INT8), reference gemv.cuh:33-40: q [N/16][K/32][32 lanes][16 bytes].
// group 128 (reference): s [N/16][K/128][16] bf16. per-channel (this build): s [N] fp16 (group = K).
// Q8 layout (reference q8_layout.h:1-37, INT8 layer weights): same [N/16][K/32][32][16 B] records, word 2 s + hi =
// row g + 8 hi, bytes i = k 32 c + 16 s + 2 t + {0, 8, 1, 9}[i]; group-128 scales in the W4 scale layout.
struct W8 {
    const uint4* q = nullptr;
    const uint16_t* s = nullptr;
    int n = 0, k = 0;
    bool per_channel = false;
    int sdt = kScaleBF16;
    bool q8 = false;   // Q8 byte order instead of W8
    bool glu = false;  // GLU matrix (Q8 layer weights)
};

// ---- layouts (load time) ----
void repack_w4(const int32_t* src_q, const uint16_t* src_s, int n, int k, uint4* dst_q, uint16_t* dst_s,
               hipStream_t st);
void glu_interleave_rows(const int32_t* src_q, const uint16_t* src_s, int n, int k, int32_t* dst_q,
                         uint16_t* dst_s, hipStream_t st, int bits = 4);
void dequant_w4(const W4& w, uint16_t* out, hipStream_t st);  // bf16 [n][k] = bf16_rn((u - 8) * s)
void quantize_w8(const uint16_t* src, int n, int k, uint4* dst_q, uint16_t* dst_s, hipStream_t st);
void tile_w8(const int8_t* src, const uint16_t* ssrc, int n, int k, uint4* dst_q, uint16_t* dst_s,
             bool per_channel, hipStream_t st);
void dequant_w8(const W8& w, uint16_t* out, hipStream_t st);  // bf16 [n][k] = bf16_rn(w * s)
// compressed-tensors 8-bit int32 [n][k/4] (u = w + 128) + [n][k/128] scales -> Q8 bytes + W4 scale layout
void repack_q8(const int32_t* src_q, const uint16_t* src_s, int n, int k, uint4* dst_q, uint16_t* dst_s,
               hipStream_t st);

// ---- decode GEMV / skinny GEMM (m = 1..16), VALU, deterministic split-K ----
void gemv_workspace_init();
// y[m][n] = sum_k x[m][k] * W[n][k]; x bf16 rows of stride ldx; y fp32 (or bf16 with out_bf16, or the GLU
// bf16 activation) rows of stride ldy
void gemv_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st);
// skinny GEMM on the matrix cores (skinny.hip), m = 1..16; out: 0 fp32, 1 bf16, 2 GLU (bf16 act)
void skinny_w4_mfma(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, int out, hipStream_t st);
// 17..32 rows in one pass (INT4, x 16-byte aligned, ldx % 8 == 0); the rows' bits equal the 16-row launches'
void skinny_w4_wide(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st);
bool skinny_w4_wide_fits(const W4& w, const uint16_t* x, int ldx);
// one pass over the weights for 1..64 rows (wdec.hip): the decode numerics (exact (u - 8) x products, group scale on
// the fp32 sums) on the 32 x 32 matrix cores, K split over the waves of a block, fixed-order sums; n % 64 == 0, x
// 16-byte aligned, ldx % 8 == 0 and the K steps even per wave (wdec_w4_fits)
bool wdec_w4_fits(const W4& w, const uint16_t* x, int ldx, int m);
// the dispatch's choice for 17..64 rows outside batch_invariant: fits, and faster than the skinny kernel's launches
bool wdec_w4_pick(const W4& w, const uint16_t* x, int ldx, int m);
void wdec_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st);
// the same kernel on W8 / Q8 records (GLU for Q8): m = 1..16, x 16-byte aligned, ldx % 8 == 0
void skinny_w8_mfma(const W8& w, const uint16_t* x, int ldx, void* y, int ldy, int m, int out, hipStream_t st);
// m = 1 decode GEMV on the matrix cores (gemv1.hip); false when the shape takes the VALU GEMV (uneven K slices,
// x not 16-byte aligned). out as for skinny_w4_mfma
bool gemv1_w4(const W4& w, const uint16_t* x, void* y, int out, hipStream_t st);
// m = 1 on W8 per-channel records on the matrix cores (gemv1.hip); false when it does not take the shape (Q8 or group
// scales, GLU, x not 16-byte aligned, no K slicing)
bool gemv1_w8c(const W8& w, const uint16_t* x, void* y, int out, hipStream_t st);
// H16 decode numerics (the reference's gemv_w4h, gemv_h16.cuh): XH activations (xh_pack), m = 1..16 per launch,
// W4 or Q8 (q8) records; out as for skinny_w4_mfma; yh: optional XH copy of the outputs [m][ldyh]
void xh_pack(const uint16_t* x, int ldx, int k, int m, uint16_t* xh, int ldxh, hipStream_t st);
void skinny_h16(const uint4* q, const uint16_t* s, int n, int k, int sdt, bool q8, const uint16_t* xh, int ldx, void* y,
                int ldy, int m, int out, uint16_t* yh, int ldyh, hipStream_t st);
// any m (16-row launches); checks the shapes
// whether gemv_h16 runs m rows as one launch (INT4, m <= 32, XH rows 64-element strided and 16-byte aligned, and for
// 17..32 rows an even K slicing): the reference's wide H16 GEMV contract (gemv_w4hx, false when unsupported)
bool gemv_h16_one_launch(int n, int k, bool q8, const uint16_t* xh, int ldx, int m);
void gemv_h16(const uint4* q, const uint16_t* s, int n, int k, int sdt, bool q8, bool glu, const uint16_t* xh, int ldx,
              void* y, int ldy, int m, bool out_bf16, uint16_t* yh, int ldyh, hipStream_t st);
// the m = 1 GEMV's record stream with no arithmetic (its HBM read floor); falls back to 4-group slices where the
// GEMV has no even slicing
void read_probe_w4(const void* q, int n, int k, uint32_t* sink, hipStream_t st);
float clock_probe_mhz(hipStream_t st);  // the shader clock over 50 us of wall clock (synchronizes st)
// Kernel policy, set explicitly by the caller (qe_set_config) instead of scattered environment reads:
//   skinny_min_m    smallest row count gemv_w4 sends to the matrix-core skinny kernel (default 2)
//   w8_mfma_min_m   the same for INT8 / Q8 (0 = automatic: 1 where the m = 1 slicing has >= 4 groups, else 2)
//   batch_invariant 1: m = 1 also runs the skinny kernel, so a row's bits do not depend on how many rows are in the
//                   call (m = 1..16 per launch; larger m in 16-row launches of the same kernel); 0 (default): m = 1
//                   runs the faster m = 1 kernel, whose fp32 summation order differs (results within 1e-5 * rms)
//   gemm_tune       1: every prefill GEMM call times its candidates once per (shape, token bucket) (outside graph
//                   capture) and keeps the fastest; 0 (default): stored choices, else the cost model
struct QeConfig {
    int skinny_min_m = 2;
    int w8_mfma_min_m = 0;
    int batch_invariant = 0;
    int gemm_tune = 0;
    int gemm_h16 = 0;
};
const QeConfig& qe_config();
void qe_config_set(const QeConfig& c);
void gemv_w8(const W8& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st);

// ---- library-owned workspaces, one per (kind, device, stream) (workspace.cpp) ----
enum WsKind : int { kWsSplit = 0, kWsI8 = 1, kWsH = 2, kWsDec = 3, kNumWs = 4 };
// the buffer of (kind, current device, st), at least `bytes`: grown outside graph capture (the outgrown one kept
// allocated); nullptr during capture when it is too small. kWsDec buffers (the one-pass decode's tail counters and
// sums) are zero-filled when allocated; the kernel leaves its counters zero.
void* stream_ws(int kind, size_t bytes, hipStream_t st);
// the stream's tail workspace of the decode kernels (kWsDec, one size for every shape): dec_tail_ctr_bytes() of
// counters (one per tail tile or slab, at most one per CU), then the tail parts' sums (up to 2 x 32 x 64 floats per
// CU); nullptr during a graph capture on a stream that has none yet
char* dec_tail_ws(hipStream_t st);
size_t dec_tail_ctr_bytes();
void stream_ws_reserve(int kind, size_t bytes, hipStream_t st);
int stream_ws_count(int kind);  // buffers of that kind allocated so far (all devices and streams)

// ---- prefill GEMM (bf16 MFMA on dequantized tiles staged in LDS) ----
// tuned: time the candidates on the first call of a (shape, token bucket) outside graph capture (also when the
// config's gemm_tune is set); otherwise the stored choice, else the cost model
void gemm_w4(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st,
             bool tuned = false);
void gemm_w8(const W8& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st,
             bool tuned = false);
// a given choice (tile configuration 0: 256 x 256, 1: 256 x 128; ks K ranges of the last partial round, 1 = none);
// falls back to ks = 1 where the split does not apply (gemm_split_applies false) or has no workspace
void gemm_w4_choice(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, int cfg, int ks,
                    hipStream_t st);
bool gemm_split_applies(int cfg, int n, int k, int t, int ks);
// the reference's fp16-accumulate prefill numerics (gemm_h.hip); gemm_h_reserve sizes its pre-pass buffer
void gemm_w4h(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st);
void gemm_h_reserve(int k, int t, hipStream_t st);
// the reference's W4A8 prefill numerics (gemm_i8.hip): activation group G in {32, 64, 128}
// q8: the matrix is in the Q8 layout (signed int8 weights, W8A8)
void gemm_w4_i8(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, int G, bool out_bf16, hipStream_t st,
                bool q8 = false);
void gemm_i8_reserve(int k, int t, hipStream_t st);
// the reference's W8A8 row GEMM of a W8 matrix (k_x_to_r8 + k_rows_qt), on the same pre-pass buffer
void gemm_w8a8(const W8& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st);
void gemm_set_out_bf16(bool on);
// reserve the split-K workspace of (the current device, st) (grown on demand otherwise, never during graph capture)
void gemm_reserve(size_t bytes, hipStream_t st);
bool gemm_out_bf16();
// run-time cap of the split count of the prefill GEMMs' last partial round (0 or less: no cap, i.e. up to 4)
void gemm_set_sk_maxparts(int n);
int gemm_sk_maxparts();

// GEMV for m <= 32 (split into row blocks of 16), GEMM above (reference gemv.cuh:187-190)
void matmul_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st);

int qe_num_cus();
// device address of the MoE scratch array on the current device (moe.hip; resolved once per device)
void* moe_scratch_ptr();

// ---- grouped prefill GEMMs of the MoE layer (moe_pf.hip: weights dequantized in registers) ----
// Jobs are (expert, first row) pairs over the expert-sorted slots, kMoePfRows rows each (moe.hip's segmentation).
// mode 1, gate_up: act[slot][I] = bf16(silu(gate) * up * slot_w[slot]) from the records' GLU rows over x[token];
// mode 2, down: slot_out[slot][H] = bf16(act[slot] . down) over the records' down columns.
constexpr int kMoePfRows = 128;
struct MoePfArgs {
    const char* recs = nullptr;      // expert-major group records
    size_t rec = 0, gg_q = 0, gg_s = 0, gd_q = 0;  // record bytes and part offsets
    int ngrp = 0, H = 0, I = 0;
    const uint16_t* a = nullptr;     // mode 1: x [T][H]; mode 2: act [slots][I]
    const int32_t* off = nullptr;    // [E + 1] first slot of each expert
    const int32_t* slot_tok = nullptr;
    const float* slot_w = nullptr;
    const int32_t* jobs = nullptr;   // [max_jobs][2]
    const int32_t* njobs = nullptr;
    uint16_t* out = nullptr;         // mode 1: act; mode 2: slot_out
    int max_jobs = 0;
};
void moe_pf_gemm(int mode, const MoePfArgs& a, hipStream_t st);
