// Decode GEMV and skinny GEMM (m = 1..16 rows) on the W4 / W8 fragment layouts, for gfx950.
//
// Design (memory-bound: the packed weights are streamed once from HBM; the VALU work per byte is the other
// limit, so the inner loop is counted in instructions):
//   * one block per 16-row tile; wave w of the block owns K slice w (NG 128-k groups). A wave-load is
//     64 lanes x 16 B = 1 KB, contiguous in the layout (W4: one group of the tile, W8: half a group). All weight
//     loads of the slice are issued first (non-temporal), then the activations are staged.
//   * activation staging: lane L of a wave loads dword `slot` (L % 8) of lane class c = L / 8 of each group
//     and stores it at LDS position L, so a class's 8 dwords are contiguous (two ds_read_b128 per lane and
//     group, broadcast across the 8 lanes of a row pair) and the class sum is a 3-step DPP reduction.
//   * nibbles become bf16 by placing them in the mantissa of 128.0 (0x4300 -> 128 + u exactly, v_perm_b32),
//     v_dot2_f32_bf16 accumulates (128 + u) * x in fp32; per group the bias is removed with the staged class
//     sum and the group scale applied: acc += s * (a - 136 X). INT8 bytes (XOR 0x80 -> u = w + 128) go through
//     v_cvt_f32_ubyte + v_cvt_pk_bf16 (exact), bias 128.
//   * reduction: lanes of one row within a half-wave by DPP quad swaps, then half-waves and slices through LDS
//     in a fixed order. No global atomics, no workspace; results are deterministic and independent of m
//     ("batch == alone", the reference's skinny / GEMV contract, skinny.cu:1-14): the slicing depends on (n, k)
//     only.
#pragma once
#include "qe_api.hpp"

namespace qe_gemv {

typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));

enum Fmt : int { kFmtW4 = 0, kFmtW8G = 1, kFmtW8C = 2, kFmtQ8 = 3 };
enum Out : int { kOutF32 = 0, kOutBF16 = 1, kOutGLU = 2 };
constexpr int kMaxWaves = 8;      // K slices per block (even slicing)
constexpr int kGenericNG = 16;    // max groups per slice of the generic (uneven slices) variant
constexpr int kMaxWavesGeneric = 16;  // K slices per block of the generic variant: K <= 16 * 16 * 128 = 32768

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a), __builtin_bit_cast(bf16x2_v, b), c,
                                           false);
}
__device__ __forceinline__ u32x4_v ld_stream(const uint4* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p));
}
// Nibbles to bf16: t holds one nibble in the low half of each byte (t & 0xF0F0F0F0 == 0); v_perm_b32 with 0x43 as
// the high byte of each half gives the bf16 pairs 128 + u exactly: bytes (0, 2) and bytes (1, 3) of t. No inline
// asm for VALU work anywhere in these kernels: the compiler's MFMA hazard checks (VALU writes to registers an
// in-flight MFMA still reads) do not look into asm operands.
__device__ __forceinline__ uint32_t bf16x2_b02(uint32_t t) { return __builtin_amdgcn_perm(0x43434343u, t, 0x04020400u); }
__device__ __forceinline__ uint32_t bf16x2_b13(uint32_t t) { return __builtin_amdgcn_perm(0x43434343u, t, 0x04030401u); }
constexpr uint32_t kNib = 0x0F0F0F0Fu;
// the same with the fp16 magic 0x64 (1024 + u) and packed fp16 arithmetic (v_pk_add_f16 / v_pk_fma_f16; packed fp16
// is not the packed fp32 these kernels avoid): the exact integer u - 8, and for bytes u = w + 128, w / 16
__device__ __forceinline__ uint32_t f16x2_b02(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04020400u); }
__device__ __forceinline__ uint32_t f16x2_b13(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04030401u); }
__device__ __forceinline__ uint32_t f16x2_sub1032(uint32_t p) {
    const f16x2_v v = __builtin_bit_cast(f16x2_v, p) - f16x2_v{(_Float16)1032.f, (_Float16)1032.f};
    return __builtin_bit_cast(uint32_t, v);
}
// XH activation layout (reference gemv_h16.cuh:1-30): x / 16 in fp16 with |x| clamped to 2047 first, the columns of
// every 64-k chunk permuted: k bits b0..b5 -> p = b0 | b3 << 1 | b4 << 2 | b5 << 3 | b1 << 4 | b2 << 5, which is
// p = 16 t + 4 j + e for k = 16 j + 2 t + {0, 1, 8, 9}[e]: the class-major order the decode kernels stage
__device__ __forceinline__ int xh_pos(int k) { return (k & ~63) | (k & 1) | ((k >> 2) & 14) | ((k & 6) << 3); }
// The magnitude is scaled and rounded, then the sign is put back by hand: hipcc folds a scale-and-convert into
// v_fma_mixlo_f16 with a +0 addend, which turns -0 into +0. NaN clamps to -2047 (what fmaxf(NaN, -2047) gives).
__device__ __forceinline__ uint16_t to_xh(float v) {
    const float c = v == v ? v : -2047.f;
    const uint16_t mag = __builtin_bit_cast(uint16_t, (_Float16)(fminf(fabsf(c), 2047.f) * 0.0625f));
    return mag | static_cast<uint16_t>((__builtin_bit_cast(uint32_t, c) >> 16) & 0x8000u);
}
__device__ __forceinline__ uint32_t f16x2_q8(uint32_t p) {
    const f16x2_v v = __builtin_bit_cast(f16x2_v, p) * f16x2_v{(_Float16)0.0625f, (_Float16)0.0625f} -
                      f16x2_v{(_Float16)72.f, (_Float16)72.f};
    return __builtin_bit_cast(uint32_t, v);
}
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                     false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8

// x dword (within a 128-k group, 0..63) of slot `sl` of lane class `c` (c = 4 h + t)
template <int FMT>
__device__ __forceinline__ int x_dword(int c, int sl) {
    const int h = c >> 2, t = c & 3;
    if constexpr (FMT == kFmtW4) return 32 * h + 8 * (sl >> 1) + 4 * (sl & 1) + t;  // pair at 64h + 16j + 2t (+8b)
    else return 16 * (2 * (sl >> 2) + h) + 4 * (sl & 3) + t;  // W8: load e = sl/4, dword d = sl%4
}

// inverse of x_dword: LDS position 8 c + sl of the class-major staging that holds dword d (0..63) of a group
template <int FMT>
__device__ __forceinline__ int x_slot(int d) {
    if constexpr (FMT == kFmtW4) {  // d = 32 h + 8 (sl / 2) + 4 (sl % 2) + t
        const int c = 4 * (d >> 5) + (d & 3), sl = 2 * ((d >> 3) & 3) + ((d >> 2) & 1);
        return 8 * c + sl;
    } else {  // d = 16 (2 (sl / 4) + h) + 4 (sl % 4) + t
        const int q = d >> 4, r = d & 15;
        const int c = 4 * (q & 1) + (r & 3), sl = 4 * (q >> 1) + (r >> 2);
        return 8 * c + sl;
    }
}

template <int SDT>
__device__ __forceinline__ float scale_rt(uint16_t v, int sdt) {
    if constexpr (SDT >= 0) return scale_to_f32<SDT>(v);
    else return sdt == kScaleF16 ? scale_to_f32<kScaleF16>(v) : scale_to_f32<kScaleBF16>(v);
}

// One block computes the 16 rows of one weight tile for up to MT activation rows; wave w owns K slice w (NG
// groups, NG == 0: ng groups, <= kGenericNG). The caller supplies, per wave, the first weight record of the slice
// (qp: uint4 of lane 0 of the slice's first group; W4: groups 64 uint4 apart, W8: 128), the slice's 16-bit scales
// (sp: [ng][16] rows of the tile, W8C: [16]) and, per activation row, the dword pointer of the slice's first group
// (xw[tok], 64 dwords per group). On return (after a barrier) red[S][2][MT][16] holds the partial sums; rsum()
// below adds them in a fixed order.
// SDT < 0: scale dtype chosen at run time (`sdt`). PF: the activations of every group are loaded up front; with
// even slices (NG > 0, "UP") as 16-byte pieces before all weights (xw rows 16-byte aligned), staged and summed per
// class while the weights are in flight, else interleaved with the weight loads of the same group (w_i, x_i, ...).
// !PF: loaded when the group is reached (large m).
// LDS (`lds`): per wave xl [XG][MT][64] u32 + xsum [XG][MT][8] + the slice's scales [NGM][16] half, then red
// (XG = NG groups when PF with even slices, else 1).
// qgs / sgs: uint4 / scale dwords from one group of the slice to the next (default: the W4 / W8 layouts, groups
// adjacent; the MoE down GEMV passes the record size, its K groups are in consecutive records).
template <int MT, int FMT, int SDT, int NG, bool PF>
__device__ __forceinline__ float* gemv_tile(uint32_t* lds, const uint4* __restrict__ qp, const uint16_t* __restrict__ sp,
                                            const uint32_t* const* xw, int m, int ng, int sdt, size_t qgs = 64 * (FMT == kFmtW4 ? 1 : 2),
                                            size_t sgs = 8) {
    constexpr int NGM = NG > 0 ? NG : kGenericNG;
    constexpr int LPG = FMT == kFmtW4 ? 1 : 2;  // wave-loads per group
    // UP: every group's activations are loaded before the weights and staged while the weights are in flight,
    // so a group's work after its weights arrive is the unpack and the dot products only
    constexpr bool UP = PF && NG > 0;
    constexpr int XG = UP ? NGM : 1;  // groups of activations staged at once
    const int S = blockDim.x >> 6;
    const int w = threadIdx.x >> 6, L = threadIdx.x & 63;
    constexpr int WSZ = XG * MT * 72 + NGM * 8;  // dwords of LDS per wave
    uint32_t* xl = lds + (size_t)w * WSZ;                             // [XG][MT][64]
    float* xsum = reinterpret_cast<float*>(xl + XG * MT * 64);        // [XG][MT][8]
    uint16_t* sl16 = reinterpret_cast<uint16_t*>(xl + XG * MT * 72);  // [NGM][16] scales of the slice
    float* red = reinterpret_cast<float*>(lds + (size_t)S * WSZ);  // [S][2][MT][16]
    const int g = (L >> 2) & 7, t = L & 3, h = L >> 5;
    if (NG > 0) ng = NG;

    // activation dword of this lane in the class-major staging: class c = L / 8, slot L % 8
    const int c_st = L >> 3, sl_st = L & 7;
    const int xoff = x_dword<FMT>(c_st, sl_st);
    auto ldx_group = [&](int tok, int i) { return tok < m ? xw[tok][i * 64 + xoff] : 0u; };

    // 1. loads, in the order they are consumed (vmcnt retires in order) and with no wait between them: (UP) the
    //    activation pieces, the slice's scales (one dword per lane), then the weight records group by group. The
    //    addresses are clamped rather than branched on (xw rows past m point at row 0), so no load has to
    //    complete before the weight stream starts; out-of-range values are dropped when staged. The LDS writes
    //    that consume the early loads come after the last weight load (sched_barrier), so waiting for them
    //    never waits for weights.
    const int ndw = FMT == kFmtW8C ? 8 : ng * 8;  // scale dwords of the slice
    u32x4_v wv[NGM][LPG];
    uint32_t xr[PF && !UP ? MT : 1][PF && !UP ? NGM : 1];
    // UP: piece p = L + 64 r (slices of more than 8 groups take two rounds): lane L loads dwords [8 p, 8 p + 8) of
    // each row's slice (NG groups x 64 dwords) with two 16-byte loads (the slice starts 16-byte aligned:
    // launch_gemv checks x and ldx)
    constexpr int XL = UP ? NGM * 8 : 1;  // activation pieces of the slice
    constexpr int XR = (XL + 63) / 64;
    u32x4_v xv[UP ? XR : 1][UP ? MT : 1][2];
    qp += L;
    if constexpr (UP) {
#pragma unroll
        for (int r = 0; r < XR; r++)
#pragma unroll
            for (int tok = 0; tok < MT; tok++) {
                const int pc = L + 64 * r < XL ? L + 64 * r : XL - 1;
                const u32x4_v* src = reinterpret_cast<const u32x4_v*>(xw[tok]) + 2 * pc;
                xv[r][tok][0] = src[0];
                xv[r][tok][1] = src[1];
            }
    }
    // scale dword p = L + 64 r (slices of more than 8 groups take two rounds)
    constexpr int SPR = FMT == kFmtW8C ? 1 : (NGM * 8 + 63) / 64;
    uint32_t sraw[SPR];
#pragma unroll
    for (int r = 0; r < SPR; r++) {
        const int ls = L + 64 * r < ndw ? L + 64 * r : ndw - 1;
        sraw[r] = reinterpret_cast<const uint32_t*>(sp)[(size_t)(ls >> 3) * sgs + (ls & 7)];
    }
#pragma unroll
    for (int i = 0; i < NGM; i++) {
        if (NG == 0 && i >= ng) break;
#pragma unroll
        for (int e = 0; e < LPG; e++) wv[i][e] = ld_stream(qp + (size_t)i * qgs + (size_t)e * 64);
        if constexpr (PF && !UP) {
#pragma unroll
            for (int tok = 0; tok < MT; tok++) xr[tok][i] = xw[tok][i * 64 + xoff];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < SPR; r++)
        if (L + 64 * r < ndw) reinterpret_cast<uint32_t*>(sl16)[L + 64 * r] = sraw[r];

    // 2. per group: stage x (class-major, class sums times the bias), then the dot products
    constexpr float bias = FMT == kFmtW4 ? 136.f : 128.f;
    const int cls = 4 * h + t;
    float acc_lo[MT], acc_hi[MT];
#pragma unroll
    for (int tok = 0; tok < MT; tok++) acc_lo[tok] = acc_hi[tok] = 0.f;
    // stage group i's activations at xl[i % XG] (class-major) with the class sums times the bias
    auto stage = [&](int i) {
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
            const uint32_t v = PF && !UP ? (tok < m ? xr[PF && !UP ? tok : 0][PF && !UP ? i : 0] : 0u)
                                         : ldx_group(tok, i);
            const int xi = (UP ? i : 0) * MT + tok;
            xl[xi * 64 + L] = v;
            float sm = dot2_bf16(v, 0x3F803F80u, 0.f);  // x_lo + x_hi (bf16 (1, 1))
            sm = dpp_add<kDppXor1>(sm);
            sm = dpp_add<kDppXor2>(sm);
            sm = dpp_add<kDppHalfMirror>(sm);
            if (sl_st == 0) xsum[xi * 8 + c_st] = bias * sm;
        }
    };
    if constexpr (UP) {
        // dword e of piece p is dword d = 8 (p % 8) + e of group p / 8, stored at its (class, slot) (x_slot, the
        // inverse of x_dword); then the lane of piece p adds up class p % 8 of group p / 8 (16 values, in order)
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const int pc = L + 64 * r, gi = pc >> 3, l8 = pc & 7;
            if (pc < XL) {
#pragma unroll
                for (int tok = 0; tok < MT; tok++)
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        xl[(gi * MT + tok) * 64 + x_slot<FMT>(8 * l8 + e)] = tok < m ? xv[r][tok][e >> 2][e & 3] : 0u;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const int pc = L + 64 * r, gi = pc >> 3, l8 = pc & 7;
            if (pc >= XL) continue;
#pragma unroll
            for (int tok = 0; tok < MT; tok++) {
                const u32x4_v* cl = reinterpret_cast<const u32x4_v*>(&xl[(gi * MT + tok) * 64 + l8 * 8]);
                const u32x4_v a0 = cl[0], a1 = cl[1];
                float sm = 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) sm = dot2_bf16(a0[e], 0x3F803F80u, sm);  // x_lo + x_hi (bf16 (1, 1))
#pragma unroll
                for (int e = 0; e < 4; e++) sm = dot2_bf16(a1[e], 0x3F803F80u, sm);
                xsum[(gi * MT + tok) * 8 + l8] = bias * sm;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int i = 0; i < NGM; i++) {
        if (NG == 0 && i >= ng) break;
        if constexpr (!UP) {
            // the wave's own LDS region; LDS operations of one wave complete in order
            __builtin_amdgcn_wave_barrier();
            stage(i);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        const int xg = (UP ? i : 0) * MT;  // first staged row of this group

        const int so = FMT == kFmtW8C ? 0 : i * 16;
        const float s_lo = scale_rt<SDT>(sl16[so + g], sdt);
        const float s_hi = scale_rt<SDT>(sl16[so + g + 8], sdt);
        // the dot2 chains start at -bias * X, so they end at sum (u - 8) x (or sum w x for INT8)
        float a_lo[MT], a_hi[MT];
#pragma unroll
        for (int tok = 0; tok < MT; tok++) a_lo[tok] = a_hi[tok] = -xsum[(xg + tok) * 8 + cls];
        if constexpr (FMT == kFmtW4) {
            uint32_t p[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t wd = wv[i][0][j];
                const uint32_t t0 = wd & kNib, t1 = (wd >> 4) & kNib;  // row g / row g + 8: k0, k0 + 8, k0 + 1, k0 + 9
                p[j][0] = bf16x2_b02(t0);  // row g,     k0, k0 + 1
                p[j][1] = bf16x2_b02(t1);  // row g + 8, k0, k0 + 1
                p[j][2] = bf16x2_b13(t0);  // row g,     k0 + 8, k0 + 9
                p[j][3] = bf16x2_b13(t1);  // row g + 8, k0 + 8, k0 + 9
            }
#pragma unroll
            for (int tok = 0; tok < MT; tok++) {
                const u32x4_v x0 = *reinterpret_cast<const u32x4_v*>(&xl[(xg + tok) * 64 + cls * 8]);
                const u32x4_v x1 = *reinterpret_cast<const u32x4_v*>(&xl[(xg + tok) * 64 + cls * 8 + 4]);
                const uint32_t xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    a_lo[tok] = dot2_bf16(p[j][0], xv[2 * j], a_lo[tok]);
                    a_lo[tok] = dot2_bf16(p[j][2], xv[2 * j + 1], a_lo[tok]);
                    a_hi[tok] = dot2_bf16(p[j][1], xv[2 * j], a_hi[tok]);
                    a_hi[tok] = dot2_bf16(p[j][3], xv[2 * j + 1], a_hi[tok]);
                }
            }
        } else if constexpr (FMT == kFmtQ8) {
            // word 2 s + hi of wave-load e: row g + 8 hi, bytes (k0, k0 + 8, k0 + 1, k0 + 9) with k0 = the x slot
            // 4 e + 2 s; bytes 0 / 2 pair with slot 4 e + 2 s, bytes 1 / 3 with 4 e + 2 s + 1
            uint32_t plo[2][4], phi[2][4];  // [e][2 s + b]
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int sq = 0; sq < 2; sq++) {
                    const uint32_t ug = wv[i][e][2 * sq] ^ 0x80808080u, uh = wv[i][e][2 * sq + 1] ^ 0x80808080u;
                    plo[e][2 * sq] = pack_bf16x2((float)(ug & 0xffu), (float)((ug >> 16) & 0xffu));
                    plo[e][2 * sq + 1] = pack_bf16x2((float)((ug >> 8) & 0xffu), (float)(ug >> 24));
                    phi[e][2 * sq] = pack_bf16x2((float)(uh & 0xffu), (float)((uh >> 16) & 0xffu));
                    phi[e][2 * sq + 1] = pack_bf16x2((float)((uh >> 8) & 0xffu), (float)(uh >> 24));
                }
#pragma unroll
            for (int tok = 0; tok < MT; tok++) {
                const u32x4_v x0 = *reinterpret_cast<const u32x4_v*>(&xl[(xg + tok) * 64 + cls * 8]);
                const u32x4_v x1 = *reinterpret_cast<const u32x4_v*>(&xl[(xg + tok) * 64 + cls * 8 + 4]);
                const uint32_t xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int e = 0; e < 2; e++)
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        a_lo[tok] = dot2_bf16(plo[e][d], xv[4 * e + d], a_lo[tok]);
                        a_hi[tok] = dot2_bf16(phi[e][d], xv[4 * e + d], a_hi[tok]);
                    }
            }
        } else {
            uint32_t plo[2][4], phi[2][4];
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t u = wv[i][e][d] ^ 0x80808080u;  // (g, k) (g, k+1) (g+8, k) (g+8, k+1)
                    plo[e][d] = pack_bf16x2((float)(u & 0xffu), (float)((u >> 8) & 0xffu));
                    phi[e][d] = pack_bf16x2((float)((u >> 16) & 0xffu), (float)(u >> 24));
                }
#pragma unroll
            for (int tok = 0; tok < MT; tok++) {
                const u32x4_v x0 = *reinterpret_cast<const u32x4_v*>(&xl[(xg + tok) * 64 + cls * 8]);
                const u32x4_v x1 = *reinterpret_cast<const u32x4_v*>(&xl[(xg + tok) * 64 + cls * 8 + 4]);
                const uint32_t xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int e = 0; e < 2; e++)
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        a_lo[tok] = dot2_bf16(plo[e][d], xv[4 * e + d], a_lo[tok]);
                        a_hi[tok] = dot2_bf16(phi[e][d], xv[4 * e + d], a_hi[tok]);
                    }
            }
        }
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
            acc_lo[tok] = fmaf(s_lo, a_lo[tok], acc_lo[tok]);
            acc_hi[tok] = fmaf(s_hi, a_hi[tok], acc_hi[tok]);
        }
    }

    // 3. rows g / g + 8: lanes t (DPP quad swaps), then half-waves and slices through LDS (rsum)
#pragma unroll
    for (int tok = 0; tok < MT; tok++) {
        float a = dpp_add<kDppXor1>(acc_lo[tok]);
        float b = dpp_add<kDppXor1>(acc_hi[tok]);
        a = dpp_add<kDppXor2>(a);
        b = dpp_add<kDppXor2>(b);
        if (t == 0) {
            red[((w * 2 + h) * MT + tok) * 16 + g] = a;
            red[((w * 2 + h) * MT + tok) * 16 + g + 8] = b;
        }
    }
    __syncthreads();
    return red;
}

// sum of row rr (0..15) for activation row tok over the S slices and both half-waves, in a fixed order
template <int MT>
__device__ __forceinline__ float rsum(const float* red, int S, int tok, int rr) {
    float v = 0.f;
    for (int ws = 0; ws < S; ws++) v += red[((ws * 2) * MT + tok) * 16 + rr] + red[((ws * 2 + 1) * MT + tok) * 16 + rr];
    return v;
}



// Plain decode GEMV: one block per 16-row tile of a tile-major matrix, K slices of NG groups.
template <int MT, int FMT, int SDT, int NG, bool PF>
__global__ void __launch_bounds__(64 * (NG > 0 ? kMaxWaves : kMaxWavesGeneric))
__attribute__((amdgpu_waves_per_eu(MT == 1 ? 6 : MT == 2 ? 5 : 1))) gemv_kernel(
    const uint4* __restrict__ q, const uint16_t* __restrict__ s, int N, int K, const uint16_t* __restrict__ x,
    int ldx, void* __restrict__ y, int ldy, int m, int out, int sdt) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6;
    const int tile = blockIdx.x, G = K >> 7;
    const int gb = NG > 0 ? w * NG : w * G / S;
    const int ng = NG > 0 ? NG : (w + 1) * G / S - gb;
    const uint4* qp = FMT == kFmtW4 ? q + ((size_t)tile * (K >> 6) + 2 * gb) * 32
                                    : q + ((size_t)tile * (K >> 5) + 4 * gb) * 32;
    const uint16_t* sp = FMT == kFmtW8C ? s + 16 * tile : s + ((size_t)tile * G + gb) * 16;
    const uint32_t* xw[MT];
#pragma unroll
    for (int tok = 0; tok < MT; tok++)
        xw[tok] = reinterpret_cast<const uint32_t*>(x) + (size_t)(tok < m ? tok : 0) * (ldx >> 1) + (size_t)gb * 64;
    const float* red = gemv_tile<MT, FMT, SDT, NG, PF>(lds, qp, sp, xw, m, ng, sdt);
    const int row0 = 16 * tile;
    if (out == kOutGLU) {
        for (int idx = threadIdx.x; idx < m * 8; idx += blockDim.x) {
            const int tok = idx >> 3, gg = idx & 7;
            reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 / 2 + gg] =
                f32_to_bf16(silu_f32(rsum<MT>(red, S, tok, gg)) * rsum<MT>(red, S, tok, gg + 8));
        }
    } else {
        for (int idx = threadIdx.x; idx < m * 16; idx += blockDim.x) {
            const int tok = idx >> 4, rr = idx & 15;
            const float v = rsum<MT>(red, S, tok, rr);
            if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 + rr] = f32_to_bf16(v);
            else reinterpret_cast<float*>(y)[(size_t)tok * ldy + row0 + rr] = v;
        }
    }
}

// dynamic LDS of gemv_tile for S waves (the layout described above gemv_tile)
template <int MT, int NG, bool PF>
constexpr size_t gemv_lds_bytes(int S) {
    constexpr int NGM = NG > 0 ? NG : kGenericNG;
    constexpr int XG = PF && NG > 0 ? NGM : 1;
    return (size_t)S * (XG * MT * 72 + NGM * 8) * 4 + (size_t)S * 2 * MT * 16 * 4;
}

// K slicing of a matrix: (groups per slice NG, slices S); NG = 0 means uneven slices (generic kernel).
// Depends on (n, k) only, so every row count of a matrix reduces in the same order.
struct Slicing {
    int ng, S;
};
Slicing gemv_slicing(int n, int k);
// slice size (groups per wave) of the matrix-core decode kernels, 0 when no even slicing fits (gemv.hip)
int decode_groups(int n, int k);

template <int FMT, int SDT>
void launch_gemv(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
                 int out, int sdt, hipStream_t st) {
    const Slicing sc = gemv_slicing(n, k);
    const int mt = m == 1 ? 1 : m == 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16;
    const int ngm = sc.ng > 0 ? sc.ng : kGenericNG;
    // activation prefetch registers; the up-front staging of even slices loads 16-byte pieces of x, so it needs
    // 16-byte aligned rows. The template launched follows pf, and its LDS is sized by that same template.
    const bool aligned = ((uintptr_t)x & 15) == 0 && ldx % 8 == 0;
    const bool pf = mt * ngm <= 16 && (aligned || sc.ng == 0);
    const dim3 grid((unsigned)(n / 16)), block(64 * sc.S);
#define QE_GEMV_K(MT_, NG_, PF_)                                                                          \
    gemv_kernel<MT_, FMT, SDT, NG_, PF_><<<grid, block, gemv_lds_bytes<MT_, NG_, PF_>(sc.S), st>>>( \
        q, s, n, k, x, ldx, y, ldy, m, out, sdt)
#define QE_GEMV_NG(MT_, PF_)                         \
    do {                                             \
        if (sc.ng == 8) QE_GEMV_K(MT_, 8, PF_);      \
        else if (sc.ng == 4) QE_GEMV_K(MT_, 4, PF_); \
        else if (sc.ng == 2) QE_GEMV_K(MT_, 2, PF_); \
        else QE_GEMV_K(MT_, 0, PF_);                 \
    } while (0)
#define QE_GEMV_PF(MT_)                 \
    do {                                \
        if (pf) QE_GEMV_NG(MT_, true);  \
        else QE_GEMV_NG(MT_, false);    \
    } while (0)
    if (mt == 1) QE_GEMV_PF(1);
    else if (mt == 2) QE_GEMV_PF(2);
    else if (mt == 4) QE_GEMV_PF(4);
    else if (mt == 8) QE_GEMV_NG(8, false);  // mt = 8 / 16: activations loaded per group
    else QE_GEMV_NG(16, false);
#undef QE_GEMV_PF
#undef QE_GEMV_NG
#undef QE_GEMV_K
    HIP_CHECK(hipGetLastError());
}

}  // namespace qe_gemv
