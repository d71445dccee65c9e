// W4A8 prefill GEMM, the reference's default prefill numerics (reference gemm_w4_i8: x_to_i8_kernel +
// gemm_i8*_kernel, src/kernels/gemm.cu:463-594,4513-4518): C[t][n] = sum_k X[t][k] W[n][k] where
//   * the activations are quantized per (token, group of G k), G in {32, 64, 128}: sx = amax / 127 with the two
//     lowest mantissa bits cleared (1 for a zero group), q = rn(x * fp32(1 / sx)) as int8 (x_to_i8_kernel,
//     gemm.cu:540-594);
//   * the weights enter as the exact signed int8 u - 8;
//   * each G-group's integer dot product (exact, int32) is converted to fp32, multiplied by sx and added at sw
//     (the 128-k weight group scale) into fp32 accumulators: acc = fma(rn(sum * sx), sw, acc), with the int32 sums
//     started at the bit pattern of 1.5 * 2^23 so that the first two steps are one fma.
// The same kernel runs the W8A8 products of INT8 matrices (Q8 and W8 layouts, below).
// The reference flushes per G-group into a per-128-k partial and scales that by sw; both are within fp32 rounding
// of the float64 product of the dequantized int8 operands (the reference's gate, tests/test_gemm_i8.py:125-135:
// relative rms below 1e-5 against that emulation).
//
// v_mfma_i32_32x32x32_i8 (gfx950) with W as A and X as B, so a lane of the 32 x 32 result holds one token (column
// l % 32): one activation scale per lane and tile per G-group, the weight scales of its 16 rows from LDS (4 rows per
// 8-byte read). Block: 512 threads = 8 waves in 2 (tokens) x 4 (weight rows), tile BM = 128 tokens x BN = 256 rows,
// one 128-k weight group per step (128 B per LDS row, the bf16 kernels' swizzled tile). Pipeline as in the bf16
// prefill GEMM: X (int8, from the pre-pass) by LDS DMA one step ahead, the two raw W4 chunks of a step by DMA two
// steps ahead, the next step's int8 W tile unpacked between the MFMA rows (order pinned), the weight and activation
// scales by DMA into small double buffers. Within each 16-k block the weight bytes come out of a W4 word in the
// order k0, k0 + 8, k0 + 1, k0 + 9 (k0 = 2 t, words t = 0..3); the pre-pass stores the activations in that same
// order, so the dot products pair matching k (the same permutation as the reference's pre-pass, forced by the
// W4 layout).
#include "mfma_tile.hpp"

#include <mutex>
#include <type_traits>
#include <vector>

namespace {

using namespace qe_tile;

typedef int i32x4_v __attribute__((ext_vector_type(4)));
typedef int i32x16_v __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 256, BK = 128, NTH = 512, WMT = 2, WNT = 2;
constexpr int kStage = (BM + BN) * BK;       // X [BM][128] and W [BN][128] int8
constexpr int kRaw = BN * 64;                // two 64-k W4 chunks of BN / 16 tiles x 512 B
constexpr int kSc = BN * 2;                  // [BN / 16][16] weight scales of one group
constexpr int kSx = BM * 4 * 4;              // [BM][128 / G] activation scales, G >= 32
constexpr int kLds = 2 * kStage + 2 * kRaw + 2 * kSc + 2 * kSx;
enum Out : int { kOutF32 = 0, kOutBF16 = 1, kOutGLU = 2 };
constexpr int kColGroup = 4;  // weight-column tiles per group of the tile order

// byte p of a 16-k block holds k offset kPerm(p) = 2 (p / 4) + {0, 8, 1, 9}[p % 4]
__device__ __forceinline__ int k_perm(int p) { return 2 * (p >> 2) + ((p & 1) ? 8 : 0) + ((p >> 1) & 1); }

// thread = one 16-k block of one token (the flattened (token, block) index; reference x_to_i8_kernel,
// gemm.cu:540-594): the amax of its G-group over the G / 16 consecutive lanes that share it, sx = bits(amax / 127) &
// ~3 (1 for a zero group), inv = fp32(1 / sx) (0 for a zero group), q = rn(x * inv); bytes stored in the W4 word
// order of the block. VEC: x rows 16-byte aligned (two 16-byte loads per thread)
template <int G, bool VEC>
__global__ void __launch_bounds__(256) x_to_i8_kernel(const uint16_t* __restrict__ x, int ldx, int K, int T,
                                                      int8_t* __restrict__ xq, float* __restrict__ sx) {
    constexpr int L = G / 16;
    const int jpr = K / 16;  // blocks per row, a multiple of L: a group never straddles two tokens
    const long id = (long)blockIdx.x * 256 + threadIdx.x;
    const bool live = id < (long)T * jpr;
    const int t = live ? (int)(id / jpr) : 0, j = live ? (int)(id % jpr) : 0;
    const uint16_t* r = x + (size_t)t * ldx + 16 * j;
    float v[16];
    if constexpr (VEC) {
        const u32x4_v a = live ? *reinterpret_cast<const u32x4_v*>(r) : u32x4_v{0u, 0u, 0u, 0u};
        const u32x4_v b = live ? *reinterpret_cast<const u32x4_v*>(r + 8) : u32x4_v{0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wa = a[i], wb = b[i];
            v[2 * i] = __builtin_bit_cast(float, wa << 16);
            v[2 * i + 1] = __builtin_bit_cast(float, wa & 0xFFFF0000u);
            v[8 + 2 * i] = __builtin_bit_cast(float, wb << 16);
            v[8 + 2 * i + 1] = __builtin_bit_cast(float, wb & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = live ? bf16_to_f32(r[i]) : 0.f;
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
    for (int o = 1; o < L; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));  // the G / 16 lanes of a group
    if (!live) return;
    const float sc = mx > 0.f ? __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mx / 127.f) & ~3u) : 1.f;
    const float inv = mx > 0.f ? 1.f / sc : 0.f;
    uint32_t o[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        uint32_t wv = 0;
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            const float qf = fminf(fmaxf(__builtin_rintf(v[k_perm(4 * u + bb)] * inv), -127.f), 127.f);
            wv |= ((uint32_t)(int)qf & 0xFFu) << (8 * bb);
        }
        o[u] = wv;
    }
    *reinterpret_cast<u32x4_v*>(xq + (size_t)t * K + 16 * j) = u32x4_v{o[0], o[1], o[2], o[3]};
    if (j % L == 0) sx[(size_t)t * (K / G) + (16 * j) / G] = sc;
}

// W8A8 pre-pass (reference k_x_to_r8, src/flash/flash_pfq.cuh:473-518, the activations of the row GEMM k_rows_qt):
// thread = one 32-k block of one token; the same per-(token, 128-k group) scale and rounding as x_to_i8_kernel (the
// 4 lanes of a group share the amax). Byte p of the block holds k = k_perm8(p): a W8 record lane holds a row's bytes
// as pairs (k, k + 1) at k = 16 kb + 8 half + 2 t (record dword 2 kb + half, record lane 4 g + t), and the GEMM
// takes two consecutive record lanes per 16-byte operand, so both operands pair matching k
__device__ __forceinline__ int k_perm8(int p) { return 16 * ((p >> 2) & 1) + 8 * ((p >> 1) & 1) + 2 * (p >> 3) + (p & 1); }

template <bool VEC>
__global__ void __launch_bounds__(256) x_to_r8_kernel(const uint16_t* __restrict__ x, int ldx, int K, int T,
                                                      int8_t* __restrict__ xq, float* __restrict__ sx) {
    const int jpr = K / 32;  // blocks per row, a multiple of 4: a group never straddles two tokens
    const long id = (long)blockIdx.x * 256 + threadIdx.x;
    const bool live = id < (long)T * jpr;
    const int t = live ? (int)(id / jpr) : 0, j = live ? (int)(id % jpr) : 0;
    const uint16_t* r = x + (size_t)t * ldx + 32 * j;
    float v[32];
    if constexpr (VEC) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const u32x4_v a = live ? *reinterpret_cast<const u32x4_v*>(r + 8 * h) : u32x4_v{0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t wa = a[i];
                v[8 * h + 2 * i] = __builtin_bit_cast(float, wa << 16);
                v[8 * h + 2 * i + 1] = __builtin_bit_cast(float, wa & 0xFFFF0000u);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = live ? bf16_to_f32(r[i]) : 0.f;
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    if (!live) return;
    const float sc = mx > 0.f ? __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mx / 127.f) & ~3u) : 1.f;
    const float inv = mx > 0.f ? 1.f / sc : 0.f;
    uint32_t o[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        uint32_t wv = 0;
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            const float qf = fminf(fmaxf(__builtin_rintf(v[k_perm8(4 * u + bb)] * inv), -127.f), 127.f);
            wv |= ((uint32_t)(int)qf & 0xFFu) << (8 * bb);
        }
        o[u] = wv;
    }
    u32x4_v* dst = reinterpret_cast<u32x4_v*>(xq + (size_t)t * K + 32 * j);
    dst[0] = u32x4_v{o[0], o[1], o[2], o[3]};
    dst[1] = u32x4_v{o[4], o[5], o[6], o[7]};
    if ((j & 3) == 0) sx[(size_t)t * (K / 128) + (j >> 2)] = sc;
}

// 4 nibbles u (one per byte) -> 4 signed bytes u - 8
__device__ __forceinline__ uint32_t nib_s8(uint32_t u) { return ((u | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }

// Weight formats (WF):
// kW4: W4 records, raw chunks by DMA two steps ahead, unpacked to signed int8 between the MFMA rows.
// kQ8: the weights are the Q8 layout's signed bytes (W8A8 of an INT8 matrix, reference gemm_q8_dispatch,
//   gemm.cu:4516): a row's 16-k block is word 2 s + h of the 4 records (lanes 4 g + t, t = 0..3) of its 32-k slab, in
//   the same byte order as a W4 word, so the W tile is gathered straight into LDS by 4-byte DMAs (one dword of a
//   record per lane, no unpack) one step ahead, like the activations.
// kW8: the W8 layout's signed bytes (the reference's W8A8 row GEMM k_rows_qt, src/flash/flash_pfq.cuh:520-651, with
//   group-128 or per-channel (PC) weight scales). Every record dword holds two k of row g and the same two of row
//   g + 8, so the tile is stored as pair lines (rows g and g + 8 of a 16-row tile: the 4 consecutive records 4 g + t of
//   each 32-k block, 256 B per step) by 16-byte DMAs one step ahead, and the A operands of both rows come out of one
//   line read by 4 byte permutes each: the wave's two 32-row MFMA tiles are the rows g and the rows g + 8 of its four
//   16-row tiles. The activations arrive in the matching order (x_to_r8_kernel). G = 128, so every step flushes once:
//   acc = fma(rn(float(sum) sx), sw, acc), the reference's per-stage arithmetic (its magic-number accumulator gives
//   the same rn(sum sx)), so the result is fixed to the bit.
enum Wf : int { kW4 = 0, kQ8 = 1, kW8 = 2 };

// Every group's int32 sums start at the bit pattern of M = 1.5 * 2^23: |sum| < 2^22 (at most 128 * 127 * 127), so the
// accumulator read as fp32 is M + sum exactly, and fma(M + sum, sx, -M sx) = rn(sum * sx) (M sx is exact, sx having 22
// significant bits): the flush costs 2 VALU per output instead of convert, multiply and fma
constexpr float kMagicF = 12582912.f;
constexpr int kMagicI = 0x4B400000;
constexpr i32x16_v kMagic16 = {kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI,
                               kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI, kMagicI};

template <int G, int SDT, int OUT, int WF, bool PC>
__global__ void __launch_bounds__(NTH) gemm_i8_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s,
                                                      int N, int K, const int8_t* __restrict__ xq,
                                                      const float* __restrict__ sxg, int T, void* __restrict__ c,
                                                      int ldc, int nbn, int ntiles) {
    constexpr int NGS = BK / G;   // activation groups per step
    constexpr int KPG = G / 32;   // k32 MFMA steps per activation group
    static_assert(WF != kW8 || G == 128, "W8A8: activation groups of 128");
    static_assert(!PC || WF == kW8, "per-channel scales: W8 only");
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned lds32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);
    const int per = (ntiles + 7) >> 3, b = blockIdx.x;
    const int tile = (b & 7) * per + (b >> 3);
    if (tile >= ntiles) return;
    // tile order: groups of kColGroup weight-column tiles, token blocks outer and columns inner within a group; each
    // XCD takes a contiguous run of it (blocks b, b + 8, .. run on XCD b % 8), so its 32 resident tiles are 8 token
    // blocks x 4 columns: per step 8 X slices (16 KB) and 4 W slices (32 KB) through its L2 instead of 1 X slice and
    // 32 W slices (4x the HBM fetch: each W tile re-read per token block)
    int tb, cb;
    {
        const int nbt = ntiles / nbn, full = nbn / kColGroup, cg = tile / (nbt * kColGroup);
        const int w = cg < full ? kColGroup : nbn - full * kColGroup, r = tile - cg * nbt * kColGroup;
        tb = r / w;
        cb = cg * kColGroup + r % w;
    }
    const int n0 = cb * BN, t0 = tb * BM;
    const int G128 = K >> 7, KT = K / BK;
    const int ntile_last = (N >> 4) - 1;

    auto dma_x = [&](int kt, unsigned xt) {  // 8 rows of 128 B per wave instruction
#pragma unroll
        for (int i = 0; i < BM / 64; i++) {
            const int r0 = (wave * (BM / 64) + i) * 8, row = r0 + (lane >> 3);
            const int ch = (lane & 7) ^ swz_f(row);
            const int tok = t0 + row < T ? t0 + row : T - 1;
            dma16(xq + (size_t)tok * K + kt * BK + ch * 16, __builtin_amdgcn_readfirstlane(lds32 + xt + r0 * 128));
        }
    };
    // the step's two raw 64-k W4 chunks: lane i of wave w < 8 loads record (tile 2 w + (i / 8) % 2, g = i % 8,
    // t = i / 16) of chunk 2 kt (waves 0..7) and 2 kt + 1 (waves 8..15 = the same waves again)
    auto dma_w4 = [&](int kt, unsigned raw) {
        if (wave < BN / 32) {
            const int tl = min((n0 >> 4) + 2 * wave + ((lane >> 3) & 1), ntile_last);
            const uint4* src = q + ((size_t)tl * (K >> 6) + 2 * kt) * 32 + 4 * (lane & 7) + (lane >> 4);
            dma16(src, __builtin_amdgcn_readfirstlane(lds32 + raw + wave * 1024));
            dma16(src + 32, __builtin_amdgcn_readfirstlane(lds32 + raw + BN * 32 + wave * 1024));
        }
    };
    // Q8 W tile of step kt: 128 wave instructions of 256 B (two 128-B rows), 16 per wave; lane l fills dword l % 4 of
    // chunk position (l / 4) % 8 of row 2 u + l / 32: logical chunk c = position ^ swz_f(row) = 16-k block c % 2 of
    // 32-k slab c / 2; the dword is word 2 (c % 2) + h of record lane 4 g + (l % 4) (g = row % 8, h = (row % 16) / 8)
    auto dma_wq8 = [&](int kt, unsigned wtile) {
        const uint32_t* q32 = reinterpret_cast<const uint32_t*>(q);
#pragma unroll
        for (int i = 0; i < BN / 16; i++) {
            const int u = wave * (BN / 16) + i, row = 2 * u + (lane >> 5);
            const int cl = ((lane >> 2) & 7) ^ swz_f(row);
            const int tl = min((n0 + row) >> 4, ntile_last), g = row & 7, h = (row >> 3) & 1;
            const size_t rec = ((size_t)tl * (K >> 5) + kt * 4 + (cl >> 1)) * 32 + g * 4 + (lane & 3);
            dma4(q32 + rec * 4 + 2 * (cl & 1) + h, __builtin_amdgcn_readfirstlane(lds32 + wtile + u * 256));
        }
    };
    // W8 tile of step kt as BN / 2 pair lines (line 8 (local tile) + g: rows g and g + 8), 256 B each: the records
    // (32-k block kk, lane 4 g + t) of the step, logical chunk 4 kk + t stored at chunk position (4 kk + t) ^ g (the
    // eight lines g of one read hit distinct banks); four 1-KB wave instructions (four lines each) per wave
    auto dma_w8 = [&](int kt, unsigned wtile) {
#pragma unroll
        for (int i = 0; i < BN / 64; i++) {
            const int u = wave * (BN / 64) + i, line = 4 * u + (lane >> 4), g = line & 7;
            const int cl = (lane & 15) ^ g;
            const int tl = min((n0 >> 4) + (line >> 3), ntile_last);
            dma16(q + ((size_t)tl * (K >> 5) + kt * 4 + (cl >> 2)) * 32 + 4 * g + (cl & 3),
                  __builtin_amdgcn_readfirstlane(lds32 + wtile + u * 1024));
        }
    };
    auto dma_sc = [&](int grp, unsigned sc) {
        if (wave < BN / 128) {
            const int tl = min((n0 >> 4) + 8 * wave + (lane >> 3), ntile_last);
            const unsigned dst = __builtin_amdgcn_readfirstlane(lds32 + sc + wave * 256);
            if constexpr (PC) dma4(s + (size_t)tl * 16 + 2 * (lane & 7), dst);
            else dma4(s + ((size_t)tl * G128 + grp) * 16 + 2 * (lane & 7), dst);
        }
    };
    // activation scales of the step: [BM tokens][NGS] floats, 4 bytes per lane
    auto dma_sx = [&](int kt, unsigned sxo) {
        constexpr int NW = BM * NGS / 64;  // wave instructions
        if (wave < NW) {
            const int i = wave * 64 + lane, row = i / NGS, gi = i % NGS;
            const int tok = t0 + row < T ? t0 + row : T - 1;
            dma4(sxg + (size_t)tok * (K / G) + kt * NGS + gi, __builtin_amdgcn_readfirstlane(lds32 + sxo + wave * 256));
        }
    };
    const int jj = tid & 3, jg = (tid >> 2) & 7, jtr = tid >> 5;
    static_assert(BN * 2 == NTH, "one unpack job per thread");

    // two stages of X, W and the scales in LDS (a third, the DMA two steps ahead, measured slower for kW8)
    constexpr unsigned kRawOff = 2 * kStage, kScOff = kRawOff + 2 * kRaw, kSxOff = kScOff + 2 * kSc;
    auto dma_step = [&](int kk, int slot) {  // X, the Q8 / W8 tile and the scales of step kk into stage slot
        dma_x(kk, slot * kStage);
        if constexpr (WF == kQ8) dma_wq8(kk, slot * kStage + BM * BK);
        if constexpr (WF == kW8) dma_w8(kk, slot * kStage + BM * BK);
        dma_sc(kk, kScOff + slot * kSc);
        dma_sx(kk, kSxOff + slot * kSx);
    };
    const int wm = wave >> 2, wn = wave & 3;
    // first of the 4 consecutive weight rows (block-local) of register quad rq of MFMA tile bb, lanes l < 32 (+4 for
    // l >= 32): kW8 tiles bb hold the rows g + 8 bb of the wave's four 16-row tiles, the others 32 consecutive rows
    static_assert(WNT == 2, "kW8: the two row halves of four 16-row tiles");
    auto wrow = [&](int bb, int rq) { return WF == kW8 ? (4 * wn + rq) * 16 + 8 * bb : wn * 32 * WNT + bb * 32 + 8 * rq; };
    f32x16_v acc[WMT][WNT];
    i32x16_v dsum[WMT][WNT];
#pragma unroll
    for (int a = 0; a < WMT; a++)
#pragma unroll
        for (int bb = 0; bb < WNT; bb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][bb][r] = 0.f;
    // kW8: byte offset of record e of k32 step ks in the lane's pair line = w8b[e][ks & 1] + 64 ks: chunk
    // (4 ks + 2 h + e) ^ g = 4 (ks ^ (g >> 2)) + ((2 h + e) ^ (g & 3)), and ks ^ (g >> 2) = ks + (g >> 2) for even ks,
    // ks - (g >> 2) for odd ks (so the four reads of a record take immediate offsets from two bases)
    float swf_pc[PC ? WNT : 1][16];  // per-channel weight scales: the same every step, read once
    int w8b[2][2];
    {
        const int g = lane & 7, hb = 2 * (lane >> 5), line = (wave & 3) * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int base = line * 256 + (((hb + e) ^ (g & 3)) << 4);
            w8b[e][0] = base + ((g >> 2) << 6);
            w8b[e][1] = base - ((g >> 2) << 6);
        }
    }
    int lane_off[BK / 32];  // k32 step ks: 16 bytes at chunk 2 ks + l / 32 of row l % 32
#pragma unroll
    for (int ks = 0; ks < BK / 32; ks++) lane_off[ks] = swz(lane & 31, 2 * ks + (lane >> 5));

    // unpack unit (ch, h, t): word t of raw chunk ch, row half h -> 4 signed bytes; after t = 3 the 16-byte chunk
    // (row jtr * 16 + jg + 8 h, 16-k block 4 ch + jj) is stored
    uint32_t wd[2][4], ob[4];
    auto unit = [&](char* wtile, int ch, int h, int t) {
        const uint32_t u = (h ? wd[ch][t] >> 4 : wd[ch][t]) & nib_mask();
        ob[t] = nib_s8(u);
        if (t == 3) {
            const int row = jtr * 16 + jg + 8 * h;
            *reinterpret_cast<u32x4_v*>(wtile + swz(row, 4 * ch + jj)) = u32x4_v{ob[0], ob[1], ob[2], ob[3]};
        }
    };
    auto read_words = [&](const char* rawb) {
#pragma unroll
        for (int ch = 0; ch < 2; ch++) {
            const uint32_t* rw = reinterpret_cast<const uint32_t*>(rawb + ch * BN * 32 + (jtr >> 1) * 1024) +
                                 (8 * (jtr & 1) + jg) * 4 + jj;
#pragma unroll
            for (int t = 0; t < 4; t++) wd[ch][t] = rw[64 * t];
        }
    };

    dma_step(0, 0);
    if constexpr (WF == kW4) {
        dma_w4(0, kRawOff);
        if (KT > 1) dma_w4(1, kRawOff + kRaw);
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if constexpr (WF == kW4) {
        read_words(lds + kRawOff);
#pragma unroll
        for (int ch = 0; ch < 2; ch++)
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 4; t++) unit(lds + BM * BK, ch, h, t);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }

    // step kt: DMA X (kt + 1), the raw W, weight scales and activation scales of kt + 1 / kt + 2; MFMAs of step kt
    // with the unpack of step kt + 1 (two units after each MFMA row); each activation group's sums flushed after its
    // last k32 step: acc += float(sum) * sx * sw
    auto kstep = [&](int kt, auto more) {
        constexpr bool MORE = decltype(more)::value;
        char* wnext = lds + ((kt + 1) & 1) * kStage + BM * BK;
        const int cur = kt & 1;
        if (MORE) dma_step(kt + 1, (kt + 1) & 1);
        if constexpr (WF == kW4) {
            if (kt + 2 < KT) dma_w4(kt + 2, kRawOff + (kt & 1) * kRaw);
        }
        const char* xt = lds + cur * kStage;
        const char* wt = xt + BM * BK;
        i32x4_v af[2][WMT], bfr[2][WNT];  // af: X (B operand), bfr: W (A operand)
        i32x4_v wraw[2][2];                // kW8: the two records (t = 2 h, 2 h + 1) of the lane's pair line
        auto read_frags = [&](int ks, int buf) {
#pragma unroll
            for (int a = 0; a < WMT; a++)
                af[buf][a] = *reinterpret_cast<const i32x4_v*>(xt + lane_off[ks] + (wm * 32 * WMT + a * 32) * 128);
            if constexpr (WF == kW8) {
                // pair line wn * 32 + l % 32 (tile l % 32 / 8 of the wave's four, g = l % 8), records 2 h, 2 h + 1
#pragma unroll
                for (int e = 0; e < 2; e++)
                    wraw[buf][e] = *reinterpret_cast<const i32x4_v*>(wt + w8b[e][ks & 1] + 64 * ks);
            } else {
#pragma unroll
                for (int bb = 0; bb < WNT; bb++)
                    bfr[buf][bb] = *reinterpret_cast<const i32x4_v*>(wt + lane_off[ks] + (wn * 32 * WNT + bb * 32) * 128);
            }
        };
        // kW8: record dwords 2 kb + half hold (row g: k, k + 1; row g + 8: k, k + 1); operand dword 2 e + kb of the
        // rows g (bb = 0) / g + 8 (bb = 1) = the low / high byte pairs of dwords 2 kb and 2 kb + 1 of record e
        auto split_rows = [&](int buf) {
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int kb = 0; kb < 2; kb++) {
                    const uint32_t d0 = (uint32_t)wraw[buf][e][2 * kb], d1 = (uint32_t)wraw[buf][e][2 * kb + 1];
                    bfr[buf][0][2 * e + kb] = (int)__builtin_amdgcn_perm(d1, d0, 0x05040100u);
                    bfr[buf][1][2 * e + kb] = (int)__builtin_amdgcn_perm(d1, d0, 0x07060302u);
                }
        };
        read_frags(0, 0);
        if constexpr (WF == kW8) split_rows(0);
        if constexpr (MORE && WF == kW4) read_words(lds + kRawOff + ((kt + 1) & 1) * kRaw);
        // weight scales of this lane's rows (4 consecutive rows per register quad, one 8-byte read) for the step
        const uint16_t* scb = reinterpret_cast<const uint16_t*>(lds + kScOff + cur * kSc);
        const float* sxb = reinterpret_cast<const float*>(lds + kSxOff + cur * kSx);
        float swf[WNT][16];
        auto load_sw = [&](float (&dst)[WNT][16]) {
#pragma unroll
            for (int bb = 0; bb < WNT; bb++)
#pragma unroll
                for (int rq = 0; rq < 4; rq++) {
                    const uint2 sp = *reinterpret_cast<const uint2*>(scb + wrow(bb, rq) + 4 * (lane >> 5));
                    dst[bb][4 * rq] = scale_to_f32<SDT>((uint16_t)(sp.x & 0xFFFFu));
                    dst[bb][4 * rq + 1] = scale_to_f32<SDT>((uint16_t)(sp.x >> 16));
                    dst[bb][4 * rq + 2] = scale_to_f32<SDT>((uint16_t)(sp.y & 0xFFFFu));
                    dst[bb][4 * rq + 3] = scale_to_f32<SDT>((uint16_t)(sp.y >> 16));
                }
        };
        if constexpr (PC) {
            if (kt == 0) load_sw(swf_pc);
#pragma unroll
            for (int bb = 0; bb < WNT; bb++)
#pragma unroll
                for (int r = 0; r < 16; r++) swf[bb][r] = swf_pc[bb][r];
        } else {
            load_sw(swf);
        }
        __builtin_amdgcn_sched_barrier(0);
        int slot = 0;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            if (ks + 1 < BK / 32) read_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
            for (int a = 0; a < WMT; a++) {
#pragma unroll
                for (int bb = 0; bb < WNT; bb++) {
                    const i32x16_v cin = ks % KPG == 0 ? kMagic16 : dsum[a][bb];
                    dsum[a][bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bfr[ks & 1][bb], af[ks & 1][a], cin, 0, 0, 0);
                }
                if constexpr (MORE && WF == kW4) {
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int un = 2 * slot + e;  // 16 units over 8 rows
                        unit(wnext, un >> 3, (un >> 2) & 1, un & 3);
                    }
                }
                if constexpr (WF == kW8) {
                    if (a == 0 && ks + 1 < BK / 32) split_rows((ks + 1) & 1);
                }
                slot++;
                __builtin_amdgcn_sched_barrier(0);
            }
            if (ks % KPG == KPG - 1) {  // flush activation group ks / KPG: acc += (float(sum) * sx) * sw
                const int gi = ks / KPG;
#pragma unroll
                for (int a = 0; a < WMT; a++) {
                    const float sxa = sxb[(wm * 32 * WMT + a * 32 + (lane & 31)) * NGS + gi];
                    const float msx = -kMagicF * sxa;  // exact: sx has 22 significant bits
#pragma unroll
                    for (int bb = 0; bb < WNT; bb++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            // copied to a scalar first: hipcc lowers a bit_cast of an ext_vector element as element 0
                            const int d = dsum[a][bb][r];
                            acc[a][bb][r] = fmaf(fmaf(__builtin_bit_cast(float, d), sxa, msx), swf[bb][r], acc[a][bb][r]);
                        }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    static_assert((BK / 32) * WMT * 2 == 16, "16 unpack units per step, two per MFMA row");
    for (int kt = 0; kt + 1 < KT; kt++) kstep(kt, std::true_type{});
    kstep(KT - 1, std::false_type{});

    // epilogue: lane = token l % 32, register r = weight row 8 (r / 4) + 4 (l / 32) + r % 4 of its tile
    const int cj = lane & 31, ci = 4 * (lane >> 5);
    const bool vec = ((ldc & 3) == 0 && ((uintptr_t)c & (OUT == kOutF32 ? 15u : 7u)) == 0);
#pragma unroll
    for (int a = 0; a < WMT; a++)
#pragma unroll
        for (int bb = 0; bb < WNT; bb++) {
            const int tok = t0 + wm * 32 * WMT + a * 32 + cj;
            if (tok >= T) continue;
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const int n = n0 + wrow(bb, rb) + ci;  // first of 4 consecutive rows
                if (n >= N) continue;
                const f32x16_v& v = acc[a][bb];
                if constexpr (OUT == kOutGLU) {
                    if (rb & 1) continue;  // rows 8 (rb + 1) + ..: the up rows of this gate block
                    uint16_t* p = reinterpret_cast<uint16_t*>(c) + (size_t)tok * ldc + (n >> 4) * 8 + (n & 7);
                    float g[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) g[j] = silu_f32(v[4 * rb + j]) * v[4 * rb + 4 + j];
                    if (vec) {
                        *reinterpret_cast<uint2*>(p) = uint2{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3])};
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j++) p[j] = f32_to_bf16(g[j]);
                    }
                } else if constexpr (OUT == kOutBF16) {
                    uint16_t* p = reinterpret_cast<uint16_t*>(c) + (size_t)tok * ldc + n;
                    if (vec) {
                        *reinterpret_cast<uint2*>(p) =
                            uint2{pack_bf16x2(v[4 * rb], v[4 * rb + 1]), pack_bf16x2(v[4 * rb + 2], v[4 * rb + 3])};
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j++) p[j] = f32_to_bf16(v[4 * rb + j]);
                    }
                } else {
                    float* p = reinterpret_cast<float*>(c) + (size_t)tok * ldc + n;
                    if (vec) {
                        *reinterpret_cast<f32x4_v*>(p) = f32x4_v{v[4 * rb], v[4 * rb + 1], v[4 * rb + 2], v[4 * rb + 3]};
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j++) p[j] = v[4 * rb + j];
                    }
                }
            }
        }
}

// the pre-pass buffer (xq [t][k] int8, sx [t][k / G] fp32) of (device, stream): a capture that needs more than an
// eager call or gemm_i8_reserve on its stream sized aborts with a message
void* i8_ws(size_t bytes, hipStream_t st) {
    void* p = stream_ws(kWsI8, bytes, st);
    CHECK(p != nullptr,
          "gemm_w4_i8: the pre-pass buffer (%zu bytes) must be sized by an eager call or qe_gemm_i8_reserve(_s) on "
          "this stream before capture",
          bytes);
    return p;
}

size_t xq_bytes(int k, int t) { return ((size_t)t * k + 255) / 256 * 256; }
size_t i8_ws_bytes(int k, int t) { return xq_bytes(k, t) + (size_t)t * (k / 32) * 4; }  // sx sized for G = 32

template <int G, int WF>
void run_i8(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, int out, hipStream_t st) {
    char* ws = static_cast<char*>(i8_ws(i8_ws_bytes(w.k, t), st));
    int8_t* xq = reinterpret_cast<int8_t*>(ws);
    float* sx = reinterpret_cast<float*>(ws + xq_bytes(w.k, t));
    const unsigned pb = (unsigned)(((long)t * (w.k / 16) + 255) / 256);
    if (((uintptr_t)x & 15) == 0 && ldx % 8 == 0) x_to_i8_kernel<G, true><<<dim3(pb), dim3(256), 0, st>>>(x, ldx, w.k, t, xq, sx);
    else x_to_i8_kernel<G, false><<<dim3(pb), dim3(256), 0, st>>>(x, ldx, w.k, t, xq, sx);
    HIP_CHECK(hipGetLastError());
    const int nbn = (w.n + BN - 1) / BN, nbt = (t + BM - 1) / BM, ntiles = nbn * nbt;
    const unsigned blocks = (unsigned)(8 * ((ntiles + 7) / 8));
#define QE_GI(SDT_, OUT_)                                                                                            \
    gemm_i8_kernel<G, SDT_, OUT_, WF, false><<<dim3(blocks), dim3(NTH), kLds, st>>>(w.q, w.s, w.n, w.k, xq, sx, t, c, ldc, nbn, \
                                                                          ntiles)
    if (w.sdt == kScaleF16) {
        if (out == kOutGLU) QE_GI(kScaleF16, kOutGLU);
        else if (out == kOutBF16) QE_GI(kScaleF16, kOutBF16);
        else QE_GI(kScaleF16, kOutF32);
    } else {
        if (out == kOutGLU) QE_GI(kScaleBF16, kOutGLU);
        else if (out == kOutBF16) QE_GI(kScaleBF16, kOutBF16);
        else QE_GI(kScaleBF16, kOutF32);
    }
#undef QE_GI
    HIP_CHECK(hipGetLastError());
}

template <int SDT, bool PC>
void run_w8a8(const W8& w, const int8_t* xq, const float* sx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    const int nbn = (w.n + BN - 1) / BN, nbt = (t + BM - 1) / BM, ntiles = nbn * nbt;
    const unsigned blocks = (unsigned)(8 * ((ntiles + 7) / 8));
    if (out_bf16)
        gemm_i8_kernel<128, SDT, kOutBF16, kW8, PC><<<dim3(blocks), dim3(NTH), kLds, st>>>(w.q, w.s, w.n, w.k, xq, sx, t,
                                                                                        c, ldc, nbn, ntiles);
    else
        gemm_i8_kernel<128, SDT, kOutF32, kW8, PC><<<dim3(blocks), dim3(NTH), kLds, st>>>(w.q, w.s, w.n, w.k, xq, sx, t,
                                                                                       c, ldc, nbn, ntiles);
}

}  // namespace

void gemm_w8a8(const W8& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    CHECK(!w.q8 && !w.glu, "gemm_w8a8: W8 layout matrices only");
    CHECK(w.n > 0 && w.n % 16 == 0 && w.k >= 128 && w.k % 128 == 0, "gemm_w8a8: n = %d, k = %d", w.n, w.k);
    CHECK(t > 0, "gemm_w8a8: t = %d", t);
    CHECK(ldx >= w.k && ((uintptr_t)x & 1) == 0, "gemm_w8a8: ldx = %d < k", ldx);
    CHECK(ldc >= w.n, "gemm_w8a8: ldc = %d < n", ldc);
    char* ws = static_cast<char*>(i8_ws(i8_ws_bytes(w.k, t), st));
    int8_t* xq = reinterpret_cast<int8_t*>(ws);
    float* sx = reinterpret_cast<float*>(ws + xq_bytes(w.k, t));
    const unsigned pb = (unsigned)(((long)t * (w.k / 32) + 255) / 256);
    if (((uintptr_t)x & 15) == 0 && ldx % 8 == 0) x_to_r8_kernel<true><<<dim3(pb), dim3(256), 0, st>>>(x, ldx, w.k, t, xq, sx);
    else x_to_r8_kernel<false><<<dim3(pb), dim3(256), 0, st>>>(x, ldx, w.k, t, xq, sx);
    HIP_CHECK(hipGetLastError());
    if (w.sdt == kScaleF16) {
        if (w.per_channel) run_w8a8<kScaleF16, true>(w, xq, sx, c, ldc, t, out_bf16, st);
        else run_w8a8<kScaleF16, false>(w, xq, sx, c, ldc, t, out_bf16, st);
    } else {
        if (w.per_channel) run_w8a8<kScaleBF16, true>(w, xq, sx, c, ldc, t, out_bf16, st);
        else run_w8a8<kScaleBF16, false>(w, xq, sx, c, ldc, t, out_bf16, st);
    }
    HIP_CHECK(hipGetLastError());
}

void gemm_i8_reserve(int k, int t, hipStream_t st) {
    if (k > 0 && t > 0) stream_ws_reserve(kWsI8, i8_ws_bytes(k, t), st);
}

void gemm_w4_i8(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, int G, bool out_bf16,
                hipStream_t st, bool q8) {
    CHECK(w.n > 0 && w.n % 16 == 0 && w.k >= 128 && w.k % 128 == 0, "gemm_w4_i8: n = %d, k = %d", w.n, w.k);
    CHECK(G == 32 || G == 64 || G == 128, "gemm_w4_i8: activation group G = %d (32, 64 or 128)", G);
    CHECK(t > 0, "gemm_w4_i8: t = %d", t);
    CHECK(ldx >= w.k && ((uintptr_t)x & 1) == 0, "gemm_w4_i8: ldx = %d < k", ldx);
    CHECK(ldc >= (w.glu ? w.n / 2 : w.n), "gemm_w4_i8: ldc = %d", ldc);
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    if (q8) {
        if (G == 32) run_i8<32, kQ8>(w, x, ldx, c, ldc, t, out, st);
        else if (G == 64) run_i8<64, kQ8>(w, x, ldx, c, ldc, t, out, st);
        else run_i8<128, kQ8>(w, x, ldx, c, ldc, t, out, st);
    } else {
        if (G == 32) run_i8<32, kW4>(w, x, ldx, c, ldc, t, out, st);
        else if (G == 64) run_i8<64, kW4>(w, x, ldx, c, ldc, t, out, st);
        else run_i8<128, kW4>(w, x, ldx, c, ldc, t, out, st);
    }
}
