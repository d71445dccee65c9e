// Skinny GEMM (m = 2..16 activation rows) on the W4 layout, with the multiply-adds on the matrix cores.
//
// The VALU GEMV (gemv_impl.hpp) spends one v_dot2 per weight pair and activation row, so its cost grows with m.
// Here the weights are unpacked once per tile and group and v_mfma_f32_16x16x32_bf16 multiplies them by all 16
// (padded) activation rows at once:
//   * MFMA operand lanes: lane l = 16 q + i supplies A row i (the tile's row i) and B column i (activation row i)
//     for the k slots 8 q .. 8 q + 7; the output lane l holds column l % 16, rows 4 q .. 4 q + 3.
//   * The W4 record of lane (g, t) holds rows g and g + 8 at k = 64 c + 16 j + 2 t + {0, 1, 8, 9} (j = 0..3).
//     Lane 16 q + i of the wave loads the records (c, g = i % 8, t = q) of the group's two 64-k chunks and keeps the
//     rows of half i / 8: k slots of lane group q are then the k of record t = q, the same for every row, which
//     is what the B operand needs. Lanes i and i + 8 load the same two records (one 16-byte load each, merged by
//     the cache), so each lane unpacks 32 weights of its own row: t = (w >> 4 h) & 0x0F0F0F0F holds its nibbles
//     for k0, k0 + 8, k0 + 1, k0 + 9, and a byte permute with 0x43 gives the bf16 pairs (128 + u) of (k0, k0 + 1)
//     and (k0 + 8, k0 + 9).
//   * Activations are staged per group in the wave's LDS in class-major order (class c = 4 h + t holds the 8
//     dwords of k = 64 h + 16 j + 2 t (+8)), which is exactly the B operand: one ds_read_b128 per MFMA. They are
//     loaded as 16-byte pieces (every wave-level load instruction costs the address unit about the same, so 4-byte
//     loads per row made the activations, not the weights, the bound at MT >= 8).
//   * The bias 136 (u = w + 8 over the 128 of the magic) is removed by one more MFMA per k step with A = -136, in
//     a chain of its own that serves all of the wave's tiles: C = sum (128 + u) x + (-136 sum x) = sum (u - 8) x,
//     all products exact in fp32. The group scale is applied once per group: acc += s * C.
//   * A wave computes RT = 2 tiles (16-row tiles 2 b, 2 b + 1 of block b) where that pays: one activation load,
//     staging and B operand read serve both tiles' MFMAs.
//   * K slices per block are those of the m = 1 matrix-core kernel (decode_groups; gemv_slicing's uneven slices
//     where no even slicing fits) and the fixed-order LDS reduction makes the result deterministic; an activation
//     row's result does not depend on the other rows (MFMA columns are independent, the slicing depends on (n, k)
//     only, the tiles per wave do not change any tile's sums).
#include "gemv_impl.hpp"

namespace qe_skinny {
using namespace qe_gemv;

// Tiles per wave RT: the weight tiles of RT consecutive 16-row tiles share one wave's staged activations and B
// operand reads (the activation traffic per tile halves at RT = 2). Even slices can take RT = 2 (the host picks it
// in launch()), uneven slices (NG = 0) at MT = 2..8 (16 rows at RT = 2 spill: N = 5120, K = 17408 29.8 -> 55.9 us).
// Measured on uneven slices, RT = 1 -> 2: N = 5120, K = 17408, m = 2 / 4 / 8 15.7 / 16.3 / 21.6 -> 14.8 / 14.8 / 16.0
// us; K = 13824 13.0 / 13.7 / 17.6 -> 12.2 / 12.2 / 13.1 us; N = 8192, K = 17408, m = 8 24.5 -> 17.5 us. Weight
// groups in flight per wave D and the occupancy hint WPE, measured on the BASELINE shapes (K = 5120, 5-group slices;
// N = 5120 and 17408):
//   RT = 2: D = 2 on slices of <= 5 groups (WPE 4: <= 128 VGPRs), else D = 3 (MT = 8: 2)
//   RT = 1: D = 2 for MT <= 8 (MT = 2 / 4: 5 / 2.5 % faster than 3, 4 and 5 slower still), else 3; WPE 6 at
//   MT <= 4 on even slices of <= 5 groups
//   uneven slices: D = 2 at MT = 16 too (N = 5120, K = 13824 / 17408, m = 12: 22.7 / 27.0 -> 21.5 / 26.0 us; N = 8192,
//   K = 17408, m = 16: 32.0 -> 30.5 us)
template <int MT, int NG, int FMT>
constexpr int skinny_rt() {
    if (FMT != kFmtW4) return 1;
    return NG > 0 || (MT >= 2 && MT <= 8) ? 2 : 1;
}
template <int MT, int NG, int RT, int FMT>
constexpr int skinny_d() {
    constexpr int d = MT <= 8 || FMT != kFmtW4 || NG == 0 || (RT == 2 && NG <= 5) ? 2 : 3;
    return NG > 0 && NG < d ? NG : d;
}
template <int MT, int NG, int RT, int FMT>
constexpr int skinny_wpe() {  // minimum waves per SIMD asked of the register allocator
    return FMT != kFmtW4 ? 1 : MT > 16 ? 2 : RT == 2 ? (NG <= 5 ? 4 : 1) : (MT <= 4 && NG > 0 && NG <= 5 ? 6 : 1);
}

// UPX (MT <= 4 with even slices): every group's activations are loaded before the weights and staged in LDS
// while the weights are in flight. Else the activations of a group are loaded with its weights (x_j before w_j,
// so waiting for x_j never waits for w_j) and staged one group ahead into a double buffer. Weight records stream
// through a window of D groups.
template <int MT, int NG>
constexpr bool skinny_upx() {
    return MT <= 4 && NG > 0 && NG <= 8;
}
// staged activation rows (one row = one activation row's 64 dwords of a group) are kXStride dwords apart: the B
// operand reads of 8 consecutive lanes (8 rows, same offset in the row) then hit 8 disjoint groups of 4 banks; with
// 64 they all hit the same banks (an 8-way conflict per read at MT >= 8)
constexpr int kXStride = 68;
template <int MT, int NG, int RT>
constexpr int skinny_wsz() {  // dwords of LDS per wave: xl [UPX ? NGM : 2][MT][kXStride], scales [RT][NGM][16] half
    constexpr int NGM = NG > 0 ? NG : kGenericNG;
    constexpr int stage = (skinny_upx<MT, NG>() ? NGM : 2) * MT * kXStride + RT * NGM * 8;
    // after its loop a wave writes its partial sums [RT][max(MT, 16)][16] floats over its own (then dead) staging area
    constexpr int part = RT * (MT > 16 ? MT : 16) * 16;
    return stage > part ? stage : part;
}

// H16: the reference's fp16 decode numerics (XH activations x / 16 in fp16 already in class-major order, weights as
// exact integers in fp16 (Q8: w / 16), f16 MFMAs, every 64-k chunk's partial rounded to fp16 and flushed into fp32
// with the group scale x 16 (Q8 x 256)); W4 and Q8 only
// UA: activation rows only 4-byte aligned (x or ldx not 16-byte aligned): each 16-byte piece is loaded as 4 dwords
template <int MT, int SDT, int NG, int RT, int FMT, bool H16 = false, bool UA = false, int D = skinny_d<MT, NG, RT, FMT>(),
          int WPE = skinny_wpe<MT, NG, RT, FMT>()>
__global__ void __launch_bounds__(64 * (NG > 0 ? kMaxWaves : kMaxWavesGeneric))
__attribute__((amdgpu_waves_per_eu(WPE))) skinny_kernel(
    const uint4* __restrict__ q, const uint16_t* __restrict__ s, int N, int K, const uint16_t* __restrict__ x,
    int ldx, void* __restrict__ y, int ldy, int m, int out, int sdt, uint16_t* __restrict__ yh = nullptr, int ldyh = 0) {
    constexpr int NGM = NG > 0 ? NG : kGenericNG;
    constexpr bool UPX = skinny_upx<MT, NG>();
    constexpr int WSZ = skinny_wsz<MT, NG, RT>();
    // MT > 16 (the wide batch kernel): NB blocks of 16 activation rows, each the B operand of its own MFMAs against
    // the same A (weight) operand; every row's arithmetic is that of MT = 16 (MFMA columns are independent)
    constexpr int NB = MT > 16 ? MT / 16 : 1, MTR = MT > 16 ? MT : 16;
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    const int tile0 = blockIdx.x * RT, G = K >> 7;
    const int gb = NG > 0 ? w * NG : w * G / S;
    const int ng = NG > 0 ? NG : (w + 1) * G / S - gb;
    uint32_t* xl = lds + (size_t)w * WSZ;
    uint16_t* sl16 = reinterpret_cast<uint16_t*>(xl + (WSZ - RT * NGM * 8));
    float* red = reinterpret_cast<float*>(lds);  // wave w's [RT][16 tok][16 rows] at w * WSZ (its staging area)

    const int qg = L >> 4, i = L & 15;  // operand lane group, row / column within the tile
    const int g = i & 7, sh = 4 * (i >> 3);  // W4: nibble shift of row i's half (W8: byte pair 16 sh / 4)

    // Activation rows tok >= m (up to MT) load row m - 1 instead: no load sits under a branch, and those MFMA
    // columns are never stored (columns are independent).
    const size_t xs = (size_t)(ldx >> 1);  // dwords per activation row
    // !UPX: a group's activations are MT rows x 16 pieces of 16 bytes; lane L loads piece L % 16 of row xrow_of(e)
    // and stages its 4 dwords at their class-major positions (MT < 4: lanes of rows past MT load a duplicate and
    // stage nothing). A staging store covers 4 rows of 8 consecutive dwords (+32): MT >= 8 takes rows 2 apart
    // (2 x kXStride = 8 banks mod 64, so the 4 rows' spans are disjoint); rows 1 apart would overlap by 4 banks.
    constexpr int XP = MT >= 4 ? MT / 4 : 1;
    auto xrow_of = [&](int e) { return MT >= 8 ? (e & 1) + 2 * (L >> 4) + 8 * (e >> 1) : (L >> 4) + 4 * e; };
    auto ld16 = [&](const uint32_t* p) -> u32x4_v {
        if constexpr (UA) return u32x4_v{p[0], p[1], p[2], p[3]};
        else return *reinterpret_cast<const u32x4_v*>(p);
    };
    const uint32_t* xq[XP];  // dword pointers of this lane's pieces (16-byte aligned unless UA)
#pragma unroll
    for (int e = 0; e < XP; e++) {
        const int tp = xrow_of(e);
        xq[e] = reinterpret_cast<const uint32_t*>(x) + (size_t)(tp < m ? tp : m - 1) * xs + (size_t)gb * 64 + 4 * (L & 15);
    }
    auto ldxg = [&](u32x4_v* dst, int ii) {
#pragma unroll
        for (int e = 0; e < XP; e++) dst[e] = ld16(xq[e] + ii * 64);
    };
    auto stxg = [&](const u32x4_v* src, int buf) {
#pragma unroll
        for (int e = 0; e < XP; e++)
            if (MT >= 4 || (L >> 4) < MT) {
#pragma unroll
                for (int c = 0; c < 4; c++)
                    xl[(buf * MT + xrow_of(e)) * kXStride + (H16 ? 4 * (L & 15) + c : x_slot<kFmtW4>(4 * (L & 15) + c))] =
                        src[e][c];
            }
    };

    // 1. loads in consumption order, none waited for before the weight window is issued: the slice's scales (8
    //    dwords per group, dword p on lane p % 64, written to LDS once the window is in flight: a write right after
    //    the load waits one memory latency ahead of the weight stream); UPX every group's activations, then the first
    //    D groups of weight records; else (x_j, w_j) pairs for the first D groups. Lanes past the scales (and UPX
    //    pieces past the slice) load and store the last dword (piece) again: the stores are unconditional, so the
    //    compiler keeps each load where it is issued here.
    constexpr int PR = (NGM * 8 + 63) / 64;  // rounds of 64 scale dwords / activation pieces (slices of > 8 groups)
    uint32_t sraw[RT][PR];
    auto sidx = [&](int pr) {
        const int p = L + 64 * pr, lim = FMT == kFmtW8C ? 8 : ng * 8;
        return p < lim ? p : lim - 1;
    };
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(
            FMT == kFmtW8C ? s + (size_t)(tile0 + r) * 16 : s + ((size_t)(tile0 + r) * G + gb) * 16);
#pragma unroll
        for (int pr = 0; pr < PR; pr++) sraw[r][pr] = sp[sidx(pr)];
    }
    auto stage_scales = [&]() {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int pr = 0; pr < (FMT == kFmtW8C ? 1 : PR); pr++)
                reinterpret_cast<uint32_t*>(sl16)[r * NGM * 8 + sidx(pr)] = sraw[r][pr];
    };
    u32x4_v xr[UPX ? 1 : D][XP];  // activation register slots (per-group staging)
    // records of lane (g, t): W4 one per 64 k (two per group), W8 one per 32 k (four per group); 32 per record column
    constexpr int LPG = FMT == kFmtW4 ? 2 : 4;
    const size_t qts = (size_t)(K >> (FMT == kFmtW4 ? 6 : 5)) * 32;  // records per tile
    const uint4* qp = q + (size_t)tile0 * qts + (size_t)(LPG * gb) * 32 + 4 * g + qg;
    u32x4_v wv[D][RT][LPG];
    auto ldw = [&](int slot, int ii) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int e = 0; e < LPG; e++) wv[slot][r][e] = ld_stream(qp + r * qts + (size_t)ii * (32 * LPG) + 32 * e);
    };
    if constexpr (UPX) {
        // piece p = L + 64 pr: lane L loads dwords [8 p, 8 p + 8) of each row's slice (16-byte pieces; x and ldx
        // are 16-byte aligned) and stores dword 8 (p % 8) + e of group p / 8 at its class-major position
        constexpr int XL = NGM * 8;
        u32x4_v xv[PR][MT][2];
        const uint32_t* xs0 = reinterpret_cast<const uint32_t*>(x) + (size_t)gb * 64;
#pragma unroll
        for (int pr = 0; pr < PR; pr++) {
            const int lc = L + 64 * pr < XL ? L + 64 * pr : XL - 1;  // lanes past the slice reload its last piece
#pragma unroll
            for (int tok = 0; tok < MT; tok++) {
                const uint32_t* src = xs0 + (tok < m ? tok : m - 1) * xs + 8 * lc;
                xv[pr][tok][0] = ld16(src);
                xv[pr][tok][1] = ld16(src + 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ii = 0; ii < D; ii++)
            if (ii < ng) ldw(ii, ii);
        __builtin_amdgcn_sched_barrier(0);
        stage_scales();
#pragma unroll
        for (int pr = 0; pr < PR; pr++) {
            const int pc = L + 64 * pr < XL ? L + 64 * pr : XL - 1;
#pragma unroll
            for (int tok = 0; tok < MT; tok++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    xl[((pc >> 3) * MT + tok) * kXStride + (H16 ? 8 * (pc & 7) + e : x_slot<kFmtW4>(8 * (pc & 7) + e))] =
                        xv[pr][tok][e >> 2][e & 3];
        }
    } else {
#pragma unroll
        for (int ii = 0; ii < D; ii++) {
            if (ii < ng) {
                ldxg(xr[ii], ii);
                ldw(ii, ii);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        stage_scales();
        stxg(xr[0], 0);  // group 0 -> buffer 0
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // the bias as bf16 pairs: W4 -136 (u = w + 8 over the magic's 128), W8 -128 (u = w + 128)
    constexpr uint32_t kBias = FMT == kFmtW4 ? 0xC308C308u : 0xC300C300u;
    const bf16x8_v a_bias = __builtin_bit_cast(bf16x8_v, u32x4_v{kBias, kBias, kBias, kBias});
    f32x4_v acc[RT][NB];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) acc[r][nb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
    // groups in rounds of D (register slot d = group % D, a compile-time index). MT = 8 on slices of more than 5
    // groups keeps the rounds rolled: fully unrolled, the compiler hoists operand reads across the whole slice and
    // needs 200+ registers (2 waves per SIMD); the other shapes run faster fully unrolled
    constexpr int OUTER_UNROLL = MT == 8 && NG > 5 ? 1 : (NGM + D - 1) / D;
#pragma unroll OUTER_UNROLL
    for (int i0 = 0; i0 < NGM; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
        const int ii = i0 + d;
        if (ii >= ng) break;
        const int xrow = UPX ? ii * MT : (ii & 1) * MT;  // first staged row of this group
        if constexpr (!UPX) {
            // stage the next group's activations into the other buffer (read two groups ago, LDS operations of
            // a wave complete in order)
            if (ii + 1 < ng) stxg(xr[(d + 1) % D], (ii + 1) & 1);
        }
        u32x4_v rc[RT][LPG];
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int e = 0; e < LPG; e++) rc[r][e] = wv[d][r][e];
        // refill the window: group ii + D goes where group ii was, issued here (left to itself the scheduler sinks
        // these loads below the group's MFMAs, and the window drains before each refill)
        if (ii + D < ng) {
            if constexpr (!UPX) ldxg(xr[d], ii + D);
            ldw(d, ii + D);
        }
        __builtin_amdgcn_sched_barrier(0);
        // per k step: one B operand read (the group's activations) serves each tile's weight MFMA and one bias MFMA
        // (A = -136, the same for every row and tile): c_r + cb = sum (128 + u) x - 136 sum x = sum (u - 8) x
        f32x4_v c[RT][NB], cb[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            cb[nb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < RT; r++) c[r][nb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int mm = 0; mm < 4; mm++) {
            bf16x8_v bb[NB];  // the B operands (H16: the same bits as f16x8)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                // columns i >= MT read row 0 again: MFMA columns are independent and those are never stored
                const u32x4_v bv = *reinterpret_cast<const u32x4_v*>(&xl[(xrow + 16 * nb + (i < MT ? i : 0)) * kXStride +
                                                                        (4 * (mm >> 1) + qg) * 8 + 4 * (mm & 1)]);
                bb[nb] = __builtin_bit_cast(bf16x8_v, bv);
            }
            const int j0 = 2 * (mm & 1);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                u32x4_v a;
                if constexpr (FMT == kFmtW4 && H16) {
                    // fp16 (1024 + u) by the 0x64 magic, minus 1032: the exact integer w = u - 8
                    const u32x4_v rec = rc[r][mm >> 1];
                    const uint32_t t0 = (rec[j0] >> sh) & kNib, t1 = (rec[j0 + 1] >> sh) & kNib;
                    const uint32_t p[4] = {f16x2_b02(t0), f16x2_b13(t0), f16x2_b02(t1), f16x2_b13(t1)};
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) a[q4] = f16x2_sub1032(p[q4]);
                } else if constexpr (FMT == kFmtW4) {
                    const u32x4_v rec = rc[r][mm >> 1];
                    const uint32_t w0 = rec[j0], w1 = rec[j0 + 1];
                    const uint32_t t0 = (w0 >> sh) & kNib, t1 = (w1 >> sh) & kNib;  // row i: k0, k0 + 8, k0 + 1, k0 + 9
                    a = u32x4_v{bf16x2_b02(t0), bf16x2_b13(t0), bf16x2_b02(t1), bf16x2_b13(t1)};
                } else if constexpr (FMT == kFmtQ8 && H16) {
                    // bytes u = w + 128 -> fp16 (1024 + u) by the 0x64 magic -> (1024 + u) / 16 - 72 = w / 16 (exact)
                    const u32x4_v rec = rc[r][mm];
                    const bool hh = sh != 0;
                    const uint32_t wa = (hh ? rec[1] : rec[0]) ^ 0x80808080u, wb = (hh ? rec[3] : rec[2]) ^ 0x80808080u;
                    const uint32_t p[4] = {f16x2_b02(wa), f16x2_b13(wa), f16x2_b02(wb), f16x2_b13(wb)};
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) a[q4] = f16x2_q8(p[q4]);
                } else if constexpr (FMT == kFmtQ8) {
                    // record of 32-k chunk mm: word 2 s + hh holds row g + 8 hh, the signed weights w at
                    // k0 + {0, 8, 1, 9}, k0 = 32 mm + 16 s + 2 t: bytes (0, 2) and (1, 3) of u = w + 128 are the B
                    // operand's pairs (k0, k0 + 1) and (k0 + 8, k0 + 9)
                    const u32x4_v rec = rc[r][mm];
                    const bool hh = sh != 0;
                    const uint32_t wa = (hh ? rec[1] : rec[0]) ^ 0x80808080u, wb = (hh ? rec[3] : rec[2]) ^ 0x80808080u;
                    auto pr = [](uint32_t u, int b0) {  // bf16 pair of bytes b0, b0 + 2 (exact)
                        const float f0 = static_cast<float>((u >> (8 * b0)) & 0xFFu);
                        const float f1 = static_cast<float>((u >> (8 * b0 + 16)) & 0xFFu);
                        return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0),
                                                     0x07060302u);
                    };
                    a = u32x4_v{pr(wa, 0), pr(wa, 1), pr(wb, 0), pr(wb, 1)};
                } else {
                    // record of slab mm: dword d holds bytes (g, k) (g, k + 1) (g + 8, k) (g + 8, k + 1) at
                    // k = 32 mm + 16 (d / 2) + 8 (d % 2) + 2 t, the B operand's k order; row i takes its byte pair,
                    // u = w + 128 as float (exact) and the high halves are the bf16 pair
                    const u32x4_v rec = rc[r][mm];
#pragma unroll
                    for (int dd = 0; dd < 4; dd++) {
                        const uint32_t u = (rec[dd] ^ 0x80808080u) >> (4 * sh);
                        const float f0 = static_cast<float>(u & 0xFFu), f1 = static_cast<float>((u >> 8) & 0xFFu);
                        a[dd] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0),
                                                      0x07060302u);
                    }
                }
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    if constexpr (H16) {
                        const bf16x8_v bn = bb[nb];
                        c[r][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_v, a),
                                                                          __builtin_bit_cast(f16x8_v, bn), c[r][nb], 0, 0, 0);
                    } else {
                        c[r][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, a), bb[nb], c[r][nb], 0, 0, 0);
                    }
                }
            }
            if constexpr (!H16) {
#pragma unroll
                for (int nb = 0; nb < NB; nb++) cb[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_bias, bb[nb], cb[nb], 0, 0, 0);
            }
            if constexpr (H16) {
                if (mm & 1) {  // end of a 64-k chunk: its partial in fp16, then into fp32 at the group scale x 16 (x 256)
#pragma unroll
                    for (int r = 0; r < RT; r++) {
                        const uint2 sv = *reinterpret_cast<const uint2*>(&sl16[(r * NGM + ii) * 16 + 4 * qg]);
                        constexpr float kF = FMT == kFmtQ8 ? 256.f : 16.f;
                        const float sc[4] = {scale_rt<SDT>((uint16_t)(sv.x & 0xffffu), sdt) * kF,
                                             scale_rt<SDT>((uint16_t)(sv.x >> 16), sdt) * kF,
                                             scale_rt<SDT>((uint16_t)(sv.y & 0xffffu), sdt) * kF,
                                             scale_rt<SDT>((uint16_t)(sv.y >> 16), sdt) * kF};
#pragma unroll
                        for (int nb = 0; nb < NB; nb++) {
#pragma unroll
                            for (int j = 0; j < 4; j++) acc[r][nb][j] = fmaf((float)(_Float16)c[r][nb][j], sc[j], acc[r][nb][j]);
                            c[r][nb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RT; r++) {
            if constexpr (H16) break;  // flushed per 64-k chunk above
            // rows 4 qg .. 4 qg + 3 of the group's scales
            const uint2 sv = *reinterpret_cast<const uint2*>(&sl16[(r * NGM + (FMT == kFmtW8C ? 0 : ii)) * 16 + 4 * qg]);
            const float s0 = scale_rt<SDT>((uint16_t)(sv.x & 0xffffu), sdt), s1 = scale_rt<SDT>((uint16_t)(sv.x >> 16), sdt);
            const float s2 = scale_rt<SDT>((uint16_t)(sv.y & 0xffffu), sdt), s3 = scale_rt<SDT>((uint16_t)(sv.y >> 16), sdt);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                acc[r][nb][0] = fmaf(s0, c[r][nb][0] + cb[nb][0], acc[r][nb][0]);
                acc[r][nb][1] = fmaf(s1, c[r][nb][1] + cb[nb][1], acc[r][nb][1]);
                acc[r][nb][2] = fmaf(s2, c[r][nb][2] + cb[nb][2], acc[r][nb][2]);
                acc[r][nb][3] = fmaf(s3, c[r][nb][3] + cb[nb][3], acc[r][nb][3]);
            }
        }
        if constexpr (!UPX) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
    }

    // 2. slices through LDS in a fixed order: wave w's sums over its own staging area (its last LDS reads come
    //    first: a wave's LDS operations complete in order), lane (qg, i) holds rows 4 qg .. + 3 of column i
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
            *reinterpret_cast<f32x4_v*>(&red[(size_t)w * WSZ + (r * MTR + 16 * nb + i) * 16 + 4 * qg]) = acc[r][nb];
    __syncthreads();
    // an output's S partials are read at once (slots past S read slot S - 1 and are not added) and summed in slice
    // order; the outputs are indexed over MT rows (index math by shifts), rows >= m are not stored
    constexpr int KW = NG > 0 ? kMaxWaves : kMaxWavesGeneric;
    auto rsum = [&](int r, int tok, int rr) {
        float p[KW];
#pragma unroll
        for (int ws = 0; ws < KW; ws++) p[ws] = red[(size_t)(ws < S ? ws : S - 1) * WSZ + (r * MTR + tok) * 16 + rr];
        float v = 0.f;
#pragma unroll
        for (int ws = 0; ws < KW; ws++) v = ws < S ? v + p[ws] : v;
        return v;
    };
    if (out == kOutGLU) {
        for (int idx = threadIdx.x; idx < RT * MT * 8; idx += blockDim.x) {
            const int r = idx / (MT * 8), tok = (idx >> 3) % MT, gg = idx & 7;
            if (tok >= m) continue;
            const int col = 8 * (tile0 + r) + gg;
            const float v = silu_f32(rsum(r, tok, gg)) * rsum(r, tok, gg + 8);
            reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + col] = f32_to_bf16(v);
            if (yh) yh[(size_t)tok * ldyh + xh_pos(col)] = to_xh(v);
        }
    } else {
        for (int idx = threadIdx.x; idx < RT * MT * 16; idx += blockDim.x) {
            const int r = idx / (MT * 16), tok = (idx >> 4) % MT, rr = idx & 15;
            if (tok >= m) continue;
            const float v = rsum(r, tok, rr);
            const int col = 16 * (tile0 + r) + rr;
            const size_t o = (size_t)tok * ldy + col;
            if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[o] = f32_to_bf16(v);
            else reinterpret_cast<float*>(y)[o] = v;
            if (yh) yh[(size_t)tok * ldyh + xh_pos(col)] = to_xh(v);
        }
    }
}

template <int FMT, int SDT, bool H16 = false, bool UA = false>
void launch(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
            int out, int sdt, hipStream_t st, uint16_t* yh = nullptr, int ldyh = 0) {
    // the K slices of the m = 1 matrix-core kernel where they divide K, else the generic uneven slices; they depend
    // on (n, k) only, so every m in 2..16 sums a row in the same order (the rows of a batch equal the rows alone)
    const int dg = decode_groups(n, k);
    const Slicing sc = dg > 0 ? Slicing{dg, (k >> 7) / dg} : gemv_slicing(n, k);
    const int mt = m == 1 ? 1 : m == 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : m <= 16 ? 16 : 32;
    CHECK(mt <= 16 || FMT == qe_gemv::kFmtW4, "skinny: %d rows per launch (32-row launches: INT4 only)", m);
    const dim3 block(64 * sc.S);
    // two tiles per wave (where n / 16 is even) at m >= 5, and for m <= 4 on grids of fewer than 16 waves per CU at
    // one tile per wave. Measured (K = 5120): RT = 2 is 3 % slower at m = 2, 4 on N = 17408 (8704 waves), 3 % faster
    // at m = 8, 13 % faster at m = 16 (two blocks per CU since the partial sums reuse the staging LDS), and 6 to 16 %
    // faster on N = 5120 (2560 waves). Not where the tiles fit one round of CUs: N = 4096 (256 tiles), m = 2 / 16:
    // 4.27 / 6.29 us at RT = 1 (one block per CU) against 5.24 / 7.58 us at RT = 2 (half the CUs idle)
    const bool rt2 = n % 32 == 0 && n / 16 > qe_num_cus() && (mt >= 8 || (long)(n / 16) * sc.S < 16L * qe_num_cus());
#define QE_SK_K(MT_, NG_)                                                                                           \
    do {                                                                                                            \
        constexpr int RT_ = skinny_rt<MT_, NG_, FMT>();                                                             \
        if (RT_ == 2 && rt2)                                                                                        \
            skinny_kernel<MT_, SDT, NG_, RT_, FMT, H16, UA><<<dim3((unsigned)(n / (16 * RT_))), block,                  \
                                         (size_t)sc.S * skinny_wsz<MT_, NG_, RT_>() * 4, st>>>(                    \
                q, s, n, k, x, ldx, y, ldy, m, out, sdt, yh, ldyh);                                                 \
        else                                                                                                        \
            skinny_kernel<MT_, SDT, NG_, 1, FMT, H16, UA><<<dim3((unsigned)(n / 16)), block,                            \
                                              (size_t)sc.S * skinny_wsz<MT_, NG_, 1>() * 4, st>>>(                 \
                    q, s, n, k, x, ldx, y, ldy, m, out, sdt, yh, ldyh);                                             \
    } while (0)
#define QE_SK_NG(MT_)                             \
    do {                                          \
        if (sc.ng == 10) QE_SK_K(MT_, 10);        \
        else if (sc.ng == 8) QE_SK_K(MT_, 8);     \
        else if (sc.ng == 5) QE_SK_K(MT_, 5);     \
        else if (sc.ng == 4) QE_SK_K(MT_, 4);     \
        else if (sc.ng == 2) QE_SK_K(MT_, 2);     \
        else if (sc.ng == 0) QE_SK_K(MT_, 0);     \
        else CHECK(false, "skinny: slice of %d groups", sc.ng); \
    } while (0)
    if (mt == 1) QE_SK_NG(1);
    else if (mt == 2) QE_SK_NG(2);
    else if (mt == 4) QE_SK_NG(4);
    else if (mt == 8) QE_SK_NG(8);
    else if (mt == 16) QE_SK_NG(16);
    else if constexpr (FMT == qe_gemv::kFmtW4 && !UA) {
        // 32 rows: even slices only (the uneven-slice variant's 16 waves x 32 staged rows exceed the LDS); else two
        // launches of 16 and m - 16 rows (the same sums per row)
        if (sc.ng == 0) {
            const size_t esz = out == qe_gemv::kOutF32 ? 4 : 2;
            launch<FMT, SDT, H16>(q, s, n, k, x, ldx, y, ldy, 16, out, sdt, st, yh, ldyh);
            launch<FMT, SDT, H16>(q, s, n, k, x + (size_t)16 * ldx, ldx, reinterpret_cast<char*>(y) + (size_t)16 * ldy * esz,
                                  ldy, m - 16, out, sdt, st, yh ? yh + (size_t)16 * ldyh : nullptr, ldyh);
            return;
        }
        if (sc.ng == 10) QE_SK_K(32, 10);
        else if (sc.ng == 8) QE_SK_K(32, 8);
        else if (sc.ng == 5) QE_SK_K(32, 5);
        else if (sc.ng == 4) QE_SK_K(32, 4);
        else if (sc.ng == 2) QE_SK_K(32, 2);
        else CHECK(false, "skinny: slice of %d groups", sc.ng);
    }
#undef QE_SK_NG
#undef QE_SK_K
    HIP_CHECK(hipGetLastError());
}

}  // namespace qe_skinny

void skinny_w4_mfma(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, int out, hipStream_t st) {
    using qe_gemv::kFmtW4;
    if (((uintptr_t)x & 15) != 0 || ldx % 8 != 0) {  // rows 4-byte aligned only (the caller checked that much)
        CHECK(m <= kMaxGemvRows, "skinny: unaligned activations take up to 16 rows per launch (m = %d)", m);
        if (w.sdt == kScaleF16) qe_skinny::launch<kFmtW4, kScaleF16, false, true>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
        else qe_skinny::launch<kFmtW4, kScaleBF16, false, true>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
        return;
    }
    if (w.sdt == kScaleF16) qe_skinny::launch<kFmtW4, kScaleF16>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else qe_skinny::launch<kFmtW4, kScaleBF16>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
}

// whether skinny_w4_wide runs its rows as one launch: 16-byte aligned rows and an even K slicing (the uneven-slice
// variant's 16 waves x 32 staged rows exceed the LDS, so those shapes take two 16-row launches)
bool skinny_w4_wide_fits(const W4& w, const uint16_t* x, int ldx) {
    return ((uintptr_t)x & 15) == 0 && ldx % 8 == 0 && qe_gemv::decode_groups(w.n, w.k) > 0;
}

// 17..32 activation rows in one pass over the weights (two 16-row B blocks per MFMA A operand)
void skinny_w4_wide(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    CHECK(w.n > 0 && w.k > 0 && w.n % 16 == 0 && w.k % 128 == 0 && m > kMaxGemvRows && m <= kWideRows,
          "skinny_w4_wide %d %d %d", w.n, w.k, m);
    CHECK(((uintptr_t)x & 15) == 0 && ldx % 8 == 0 && ldx >= w.k, "skinny_w4_wide: x 16-byte aligned, ldx %d", ldx);
    CHECK(ldy >= (w.glu ? w.n / 2 : w.n), "skinny_w4_wide ldy %d", ldy);
    skinny_w4_mfma(w, x, ldx, y, ldy, m, w.glu ? qe_gemv::kOutGLU : out_bf16 ? qe_gemv::kOutBF16 : qe_gemv::kOutF32, st);
}

// bf16 activations -> the XH layout (one thread per value)
__global__ void xh_pack_kernel(const uint16_t* __restrict__ x, int ldx, int K, int m, uint16_t* __restrict__ xh,
                               int ldxh) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)m * K) return;
    const int r = (int)(idx / K), k = (int)(idx % K);
    xh[(size_t)r * ldxh + qe_gemv::xh_pos(k)] = qe_gemv::to_xh(bf16_to_f32(x[(size_t)r * ldx + k]));
}

void xh_pack(const uint16_t* x, int ldx, int k, int m, uint16_t* xh, int ldxh, hipStream_t st) {
    CHECK(k % 64 == 0 && m >= 1 && ldx >= k && ldxh >= k && ldxh % 64 == 0, "xh_pack k %d m %d ldxh %d", k, m, ldxh);
    const size_t nthreads = (size_t)m * k;
    xh_pack_kernel<<<dim3((unsigned)((nthreads + 255) / 256)), dim3(256), 0, st>>>(x, ldx, k, m, xh, ldxh);
    HIP_CHECK(hipGetLastError());
}

// H16 numerics (XH activations, see skinny_kernel): W4 and Q8; yh (optional): the outputs again as XH
void skinny_h16(const uint4* q, const uint16_t* s, int n, int k, int sdt, bool q8, const uint16_t* xh, int ldx, void* y,
                int ldy, int m, int out, uint16_t* yh, int ldyh, hipStream_t st) {
    using namespace qe_gemv;
    if (q8) qe_skinny::launch<kFmtQ8, -1, true>(reinterpret_cast<const uint4*>(q), s, n, k, xh, ldx, y, ldy, m, out, sdt, st, yh, ldyh);
    else if (sdt == kScaleF16) qe_skinny::launch<kFmtW4, kScaleF16, true>(q, s, n, k, xh, ldx, y, ldy, m, out, sdt, st, yh, ldyh);
    else qe_skinny::launch<kFmtW4, kScaleBF16, true>(q, s, n, k, xh, ldx, y, ldy, m, out, sdt, st, yh, ldyh);
}

// INT8 (W8 layout with per-channel or group scales, or the Q8 layout; the scale dtype a run-time value)
void skinny_w8_mfma(const W8& w, const uint16_t* x, int ldx, void* y, int ldy, int m, int out, hipStream_t st) {
    if (((uintptr_t)x & 15) != 0 || ldx % 8 != 0) {  // rows 4-byte aligned only
        CHECK(m <= kMaxGemvRows, "skinny: unaligned activations take up to 16 rows per launch (m = %d)", m);
        if (w.q8) qe_skinny::launch<qe_gemv::kFmtQ8, -1, false, true>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
        else if (w.per_channel) qe_skinny::launch<qe_gemv::kFmtW8C, -1, false, true>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
        else qe_skinny::launch<qe_gemv::kFmtW8G, -1, false, true>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
        return;
    }
    if (w.q8) qe_skinny::launch<qe_gemv::kFmtQ8, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else if (w.per_channel) qe_skinny::launch<qe_gemv::kFmtW8C, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else qe_skinny::launch<qe_gemv::kFmtW8G, -1>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
}
