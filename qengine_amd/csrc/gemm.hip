// Prefill GEMM on the W4 / W8 layouts for gfx950: C[t][n] = sum_k X[t][k] * W[n][k], bf16 MFMA, fp32 accumulate.
//
// The weights are dequantized once per block tile, in registers, to the reference's bf16 operand
// (bf16_rn((u - 8) * s) for INT4, bf16_rn(w * s) for INT8; reference gemm.cu:68-77) and staged in LDS next to the
// activation tile; v_mfma_f32_32x32x16_bf16 consumes both from LDS.
//   block: 512 threads = 8 waves in 2 (tokens) x 4 (weight rows); wave tile WMT x WNT MFMA tiles of 32 x 32;
//          block tile BM = 64 WMT tokens x BN = 128 WNT rows, BK = 64 (one W4 chunk)
//   LDS: two stages of X [BM][64] and W [BN][64] bf16, rows of 128 B with the 16-byte chunks XOR-swizzled by
//        (row % 8) so the MFMA fragment reads (32 rows x 16 B per half-wave) spread over the banks
//   pipeline, per k step: the MFMAs of step k read stage k % 2 while the same waves dequantize step k + 1 into the
//        other stage; the activations of step k + 1 arrive there by LDS DMA issued at the top of step k. INT4: the
//        raw records of step k + 2 are DMA'd to LDS at the top of step k and dequantized from LDS a step later.
//        INT8: the records go through two register sets, loaded at the top of step k for step k + 2. Every step
//        ends with vmcnt(0), lgkmcnt(0) and one barrier: each load gets a step of MFMA time to arrive, and the VALU
//        dequantization overlaps the matrix pipe.
//   grid: one block per output tile, tiles ordered so that the 8 XCDs (blockIdx % 8) each sweep a contiguous band
//        of tiles (their L2 keeps the shared X / W tiles).
#include "mfma_tile.hpp"
#include "gemm_tune.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

namespace {

using namespace qe_tile;
constexpr int BK = 64, NTH = 512;

enum Fmt : int { kFmtW4 = 0, kFmtW8G = 1, kFmtW8C = 2, kFmtQ8 = 3 };
enum Out : int { kOutF32 = 0, kOutBF16 = 1, kOutGLU = 2 };

template <int WMT, int WNT>
struct Cfg {
    static constexpr int BM = 64 * WMT, BN = 128 * WNT;
    static constexpr int kStage = (BM + BN) * BK * 2;
    static constexpr int XDMA = BM / 64;         // 1 KB X DMA loads per wave and step (INT4 path)
    // INT4 path: raw W records of one k step (BN / 16 tiles x 512 B) and the scales of one group (BN / 16 x 32 B),
    // both double-buffered after the two stages
    static constexpr int kRaw = BN * 32, kSc = BN * 2;
    static constexpr int kLdsW4 = 2 * kStage + 2 * kRaw + 2 * kSc;
};

// Split tiles: the tiles from `ndirect` on run as `ks` K ranges each (stream-K of the last, partly filled
// round); their fp32 partials go to part [(tile - ndirect) * ks + split][BM][BN] and splitk_reduce_kernel adds them
struct SplitArgs {
    int ndirect = 1 << 30;
    int ks = 1;
    float* part = nullptr;
};

template <int FMT, int SDT, int WMT, int WNT>
__global__ void __launch_bounds__(NTH) gemm_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s,
                                                   int N, int K, const uint16_t* __restrict__ x, int ldx, int T,
                                                   void* __restrict__ c, int ldc, int out, int sdt, int nbn, int nbt,
                                                   SplitArgs sp) {
    using C = Cfg<WMT, WNT>;
    constexpr int BM = C::BM, BN = C::BN;
    constexpr bool W4 = FMT == kFmtW4;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned lds32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);  // LDS byte address of lds[]
    // XCD-aware tile order: block b runs on XCD b % 8; XCD j takes tiles [j * per, (j + 1) * per) of the
    // n-major tile sequence (consecutive tiles share the X tile, a band of them shares W tiles)
    int n0, t0;
    int kt0 = 0, KTL = K / BK;  // this block's k steps [kt0, kt0 + KTL)
    int split_slot = -1;        // >= 0: a split tile's part, stored raw to sp.part
    // tiles [0, sp.ndirect): whole K, XCD bands; tiles [sp.ndirect, ntiles): split into sp.ks K ranges whose
    // fp32 partials splitk_reduce_kernel sums (the blocks of the otherwise partly idle last round)
    const int ntiles = nbn * nbt, per = (sp.ndirect + 7) >> 3;
    const int b = blockIdx.x;
    int tile;
    if (b < 8 * per) {
        tile = (b & 7) * per + (b >> 3);
        if (tile >= sp.ndirect) return;
    } else {
        const int j = b - 8 * per;
        tile = sp.ndirect + j / sp.ks;
        if (tile >= ntiles) return;
        KTL = K / BK / sp.ks;
        kt0 = (j % sp.ks) * KTL;
        split_slot = j;
    }
    n0 = (tile % nbn) * BN;
    t0 = (tile / nbn) * BM;
    const int G = K >> 7;

    // ---- X (every format): LDS DMA (global_load_lds_dwordx4), 1 KB = 8 rows per wave instruction. Lane i lands at
    //      LDS slot i of the 8-row block, so it loads the chunk that the swizzle puts there. Rows past T re-read
    //      row T - 1 (their outputs are not stored).
    auto dma_x = [&](int kt, unsigned xt) {  // xt: LDS offset of the X tile from lds[]
#pragma unroll
        for (int i = 0; i < C::XDMA; i++) {
            const int r0 = (wave * C::XDMA + i) * 8, row = r0 + (lane >> 3);
            const int ch = (lane & 7) ^ swz_f(row);
            const int tok = t0 + row < T ? t0 + row : T - 1;
            dma16(x + (size_t)tok * ldx + kt * BK + ch * 8, lds32 + xt + r0 * 128);
        }
    };
    // ---- W, INT4 path. Raw records go to LDS by DMA: a 1 KB wave load covers two 16-row tiles; lane i holds record
    //      (tile 2 u + (i / 8) % 2, g = i % 8, t = i / 16), so that a job's reads below hit 64 distinct banks. A job =
    //      k step j (16 k) of the row pair (g, g + 8) of a tile: word j of the tile's 4 records (g, t = 0..3) ->
    //      4 full 16-byte chunks of the bf16 tile (rows g and g + 8, chunks 2 j and 2 j + 1).
    constexpr int NJOB = BN * 2;
    const bool jactive = tid < NJOB;
    const int jj = tid & 3, jg = (tid >> 2) & 7, jtr = tid >> 5;
    const int ntile_last = (N >> 4) - 1;
    // record (tile tl, 64-k step kt) and scales (tile tl, group grp)
    auto w_rec = [&](int tl, int kt) -> const uint4* { return q + ((size_t)tl * (K >> 6) + kt) * 32; };
    auto w_sc = [&](int tl, int grp) -> const uint16_t* { return s + ((size_t)tl * G + grp) * 16; };
    auto dma_w4 = [&](int kt, unsigned raw) {  // raw: LDS offset of the raw record buffer
        if (wave < BN / 32) {
            const int tl = min((n0 >> 4) + 2 * wave + ((lane >> 3) & 1), ntile_last);
            dma16(w_rec(tl, kt) + 4 * (lane & 7) + (lane >> 4), lds32 + raw + wave * 1024);
        }
    };
    auto dma_sc = [&](int grp, unsigned sc) {  // [BN / 16 tiles][16] scales of group grp; lane i: dword i % 8 of tile i / 8
        if (wave < BN / 128) {
            const int tl = min((n0 >> 4) + 8 * wave + (lane >> 3), ntile_last);
            dma4(w_sc(tl, grp) + 2 * (lane & 7), lds32 + sc + wave * 256);
        }
    };
    // dequantize half h (0: row g, 1: row g + 8) of this thread's job from the raw records into the W tile
    auto store_w4 = [&](char* wtile, const char* raw, const char* sc, int h) {
        if constexpr (NJOB < NTH) {
            if (!jactive) return;
        }
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(raw + (jtr >> 1) * 1024) + (8 * (jtr & 1) + jg) * 4 + jj;
        const float scl = scale_rt<SDT>(reinterpret_cast<const uint16_t*>(sc)[jtr * 16 + jg + 8 * h], sdt);
        // h = 1 keeps its nibbles high (v = 16 u): qe_tile::dq_pair's s / 16, -72 s
        const float sv = h ? scl * 0.0625f : scl, bv = h ? -72.f * scl : -1032.f * scl;
        const uint32_t msk = h ? 0xF0F0F0F0u : nib_mask();
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t u = rw[64 * t] & msk;  // bytes: k0, k0+8, k0+1, k0+9
            lo[t] = dq_pair(magic_f16<kSel02>(u), sv, bv);
            hi[t] = dq_pair(magic_f16<kSel13>(u), sv, bv);
        }
        const int row = jtr * 16 + jg + 8 * h;
        *reinterpret_cast<u32x4_v*>(wtile + swz(row, 2 * jj)) = u32x4_v{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<u32x4_v*>(wtile + swz(row, 2 * jj + 1)) = u32x4_v{hi[0], hi[1], hi[2], hi[3]};
    };

    // ---- W, INT8 path: two 16-byte records (slabs of 32 k) per (16-row tile, lane), WREC per thread
    constexpr int NREC = (BN / 16) * 64;
    constexpr int WREC = NREC >= NTH ? NREC / NTH : 1;
    const bool wactive = tid < NREC;
    struct WSet {
        u32x4_v wr[W4 ? 1 : WREC];
        uint16_t sr_lo[W4 ? 1 : WREC], sr_hi[W4 ? 1 : WREC];
    };
    WSet wsA, wsB;
    auto rec_of = [&](int e, int& tr, int& slab, int& wl) {
        const int r = tid + e * NTH;
        tr = r >> 6, slab = (r >> 5) & 1, wl = r & 31;
    };
    auto load_w8 = [&](WSet& ws, int kt) {
#pragma unroll
        for (int e = 0; e < WREC; e++) {
            int tr, slab, wl;
            rec_of(e, tr, slab, wl);
            const size_t tl = (size_t)(n0 >> 4) + tr;
            const bool v = wactive && n0 + tr * 16 < N;
            const uint4* p = q + (tl * (K >> 5) + 2 * kt + slab) * 32 + wl;
            ws.wr[e] = v ? __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p)) : u32x4_v{0u, 0u, 0u, 0u};
            const int wg = wl >> 2;
            if (FMT == kFmtW8C) {
                ws.sr_lo[e] = v ? s[n0 + tr * 16 + wg] : 0;
                ws.sr_hi[e] = v ? s[n0 + tr * 16 + wg + 8] : 0;
            } else {
                const uint16_t* sp = s + (tl * G + (kt >> 1)) * 16;
                ws.sr_lo[e] = v ? sp[wg] : 0;
                ws.sr_hi[e] = v ? sp[wg + 8] : 0;
            }
        }
    };
    // Lanes t = 0..3 of a quad hold the records (g, t) of one 32-k slab. W8: dword d = the k pair 8 d + 2 t of rows
    // g / g + 8; Q8: word d = row g + 8 (d % 2), bytes at k0 + {0, 8, 1, 9}, k0 = 16 (d / 2) + 2 t. A 4 x 4 transpose
    // across the quad (two rounds of DPP exchanges with lanes t ^ 2, then t ^ 1) gives lane t dword / word t of all
    // four, i.e. whole 8-k chunks, stored as 16-byte chunks (instead of eight 4-byte stores). Record e is dequantized
    // at step ks = e.
    auto xpose4 = [&](u32x4_v v) {
        const int t = lane & 3;
        const bool b = (t & 2) != 0, c = (t & 1) != 0;
        int r0 = __builtin_amdgcn_mov_dpp((int)(b ? v[0] : v[2]), 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
        int r1 = __builtin_amdgcn_mov_dpp((int)(b ? v[1] : v[3]), 0x4E, 0xF, 0xF, false);
        v = u32x4_v{b ? (uint32_t)r0 : v[0], b ? (uint32_t)r1 : v[1], b ? v[2] : (uint32_t)r0, b ? v[3] : (uint32_t)r1};
        r0 = __builtin_amdgcn_mov_dpp((int)(c ? v[0] : v[1]), 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
        r1 = __builtin_amdgcn_mov_dpp((int)(c ? v[2] : v[3]), 0xB1, 0xF, 0xF, false);
        return u32x4_v{c ? (uint32_t)r0 : v[0], c ? v[1] : (uint32_t)r0, c ? (uint32_t)r1 : v[2], c ? v[3] : (uint32_t)r1};
    };
    auto store_w8x = [&](const WSet& ws, char* wtile, int e) {
        if (!wactive || e >= WREC) return;
        int tr, slab, wl;
        rec_of(e, tr, slab, wl);
        const int row = tr * 16 + (wl >> 2);
        const float s_lo = scale_rt<SDT>(ws.sr_lo[e], sdt), s_hi = scale_rt<SDT>(ws.sr_hi[e], sdt);
        const float b_lo = -1152.f * s_lo, b_hi = -1152.f * s_hi;  // qe_tile::dq_pair's W8 bias
        const u32x4_v tv = xpose4(ws.wr[e]);  // tv[t'] = dword (lane t) of record (g, t')
        if constexpr (FMT == kFmtQ8) {
            // Q8 word 2 s + h: row g + 8 h, bytes at k0 + {0, 8, 1, 9}, k0 = 32 slab + 16 s + 2 t: lane t now holds
            // word t of the quad, i.e. row g + 8 (t % 2) at chunks 4 slab + 2 (t / 2) (bytes 0, 2) and + 1 (bytes 1, 3)
            const int t = wl & 3;
            const float sc = (t & 1) ? s_hi : s_lo, bs = -1152.f * sc;
            uint32_t a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t x = tv[u] ^ 0x80808080u;  // w + 128
                a[u] = dq_pair(magic_f16<kSel02>(x), sc, bs);
                b[u] = dq_pair(magic_f16<kSel13>(x), sc, bs);
            }
            const int qrow = row + 8 * (t & 1), ch = 4 * slab + 2 * (t >> 1);
            *reinterpret_cast<u32x4_v*>(wtile + swz(qrow, ch)) = u32x4_v{a[0], a[1], a[2], a[3]};
            *reinterpret_cast<u32x4_v*>(wtile + swz(qrow, ch + 1)) = u32x4_v{b[0], b[1], b[2], b[3]};
            return;
        }
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t x = tv[u] ^ 0x80808080u;  // w + 128
            lo[u] = dq_pair(magic_f16<kSel01>(x), s_lo, b_lo);
            hi[u] = dq_pair(magic_f16<kSel23>(x), s_hi, b_hi);
        }
        const int ch = 4 * slab + (wl & 3);
        *reinterpret_cast<u32x4_v*>(wtile + swz(row, ch)) = u32x4_v{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<u32x4_v*>(wtile + swz(row + 8, ch)) = u32x4_v{hi[0], hi[1], hi[2], hi[3]};
    };

    // ---- MFMA tiles: wave (wm, wn) owns tokens wm * 32 WMT .. , rows wn * 32 WNT ..
    const int wm = wave >> 2, wn = wave & 3;
    f32x16_v acc[WMT][WNT];
#pragma unroll
    for (int a = 0; a < WMT; a++)
#pragma unroll
        for (int bb = 0; bb < WNT; bb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][bb][r] = 0.f;

    // one k step: MFMAs on stage kt % 2 while the next step's tiles go into the other stage
    int lane_off[BK / 16];  // swz(l % 32, 2 ks + l / 32) of this lane
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) lane_off[ks] = swz(lane & 31, 2 * ks + (lane >> 5));
    // pre() runs after the first fragment reads, between(slot) after each row of WNT MFMAs (slot = ks * WMT + row).
    // pin: nothing is scheduled across those calls, so the work placed in them keeps its place among the MFMAs
    // (the INT4 dequantization: left to the scheduler it clusters into one VALU block per k16 step, during which
    // the wave issues no MFMA).
    auto mfma_step = [&](int kt, auto&& pre, auto&& between, auto pin) {
        const char* xt = lds + (kt & 1) * C::kStage;
        const char* wt = xt + BM * BK * 2;
        // fragments of lane l: row l % 32, k = 16 ks + 8 (l / 32) .. + 8 -> chunk 2 ks + l / 32; the reads of k16
        // step ks + 1 are issued before the MFMAs of step ks
        // (every fragment row block is 32-aligned, so the swizzled offset is a per-lane part + a constant)
        bf16x8_v af[2][WMT], bfr[2][WNT];
        auto read_frags = [&](int ks, int buf) {
            const char* xl = xt + lane_off[ks];
            const char* wl = wt + lane_off[ks];
#pragma unroll
            for (int a = 0; a < WMT; a++)
                af[buf][a] = *reinterpret_cast<const bf16x8_v*>(xl + (wm * 32 * WMT + a * 32) * 128);
#pragma unroll
            for (int bb = 0; bb < WNT; bb++)
                bfr[buf][bb] = *reinterpret_cast<const bf16x8_v*>(wl + (wn * 32 * WNT + bb * 32) * 128);
        };
        auto fence = [&] {
            if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
        };
        read_frags(0, 0);
        pre();
        fence();
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            if (ks + 1 < BK / 16) read_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
            for (int a = 0; a < WMT; a++) {
#pragma unroll
                for (int bb = 0; bb < WNT; bb++)
                    acc[a][bb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ks & 1][bb], af[ks & 1][a], acc[a][bb], 0, 0, 0);
                between(ks * WMT + a);
                fence();
            }
        }
    };

    if constexpr (W4) {
        // Every global load is an LDS DMA issued at the top of a step, so the compiler tracks none of them and
        // inserts no waits inside the step; each step ends with vmcnt(0) (its DMAs landed), lgkmcnt(0) and the
        // barrier that publishes them. Step kt: DMA X of step kt + 1 into the other stage and the raw W of step
        // kt + 2 (plus the scales of its group when it starts one), then the MFMAs of step kt with the dequantization
        // of step kt + 1 (raw records published by the previous step) into the other stage: this thread's 4 raw
        // words and 2 scales are read at the top, and its 8 (row half, word) units run one after every
        // NSLOT / 8-th MFMA row, each half's two 16-byte stores after its last unit. The last step, which has no
        // next step to dequantize, is a separate instance, so the steps before it are one basic block (measured on
        // C2: 41-42 % -> 44-46 % of the bf16 peak against the dequantization left to the scheduler after a branch;
        // matrix pipes busy 51 % -> 61 % of the busy cycles).
        constexpr unsigned kRawOff = 2 * C::kStage, kScOff = kRawOff + 2 * C::kRaw;
        char* raw = lds + kRawOff;
        char* scb = lds + kScOff;
        // buffers by the local step kt, addresses by the global step kt0 + kt (kt0 is even: group aligned)
        dma_x(kt0, 0);
        dma_w4(kt0, kRawOff);
        dma_w4(kt0 + 1, kRawOff + C::kRaw);
        dma_sc(kt0 >> 1, kScOff);
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        store_w4(lds + BM * BK * 2, raw, scb, 0);
        store_w4(lds + BM * BK * 2, raw, scb, 1);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        constexpr int NSLOT = (BK / 16) * WMT, STRIDE = NSLOT >= 8 ? NSLOT / 8 : 1;
        static_assert(NSLOT >= 8, "eight dequantization units per k step");
        auto kstep = [&](int kt, auto more) {
            constexpr bool MORE = decltype(more)::value;
            char* wnext = lds + ((kt + 1) & 1) * C::kStage + BM * BK * 2;
            if (MORE) dma_x(kt0 + kt + 1, ((kt + 1) & 1) * C::kStage);
            if (kt + 2 < KTL) {
                dma_w4(kt0 + kt + 2, kRawOff + (kt & 1) * C::kRaw);
                if (((kt + 2) & 1) == 0) dma_sc((kt0 + kt + 2) >> 1, kScOff + (((kt + 2) >> 1) & 1) * C::kSc);
            }
            const char* rnext = raw + ((kt + 1) & 1) * C::kRaw;
            const uint16_t* snext = reinterpret_cast<const uint16_t*>(scb + (((kt + 1) >> 1) & 1) * C::kSc);
            const uint32_t* rw = reinterpret_cast<const uint32_t*>(rnext + (jtr >> 1) * 1024) + (8 * (jtr & 1) + jg) * 4 + jj;
            uint32_t wd[4], lo[2][4], hi[2][4];
            float scl[2];
            mfma_step(kt, [&] {
                if constexpr (MORE) {
#pragma unroll
                    for (int t = 0; t < 4; t++) wd[t] = rw[64 * t];
#pragma unroll
                    for (int h = 0; h < 2; h++) scl[h] = scale_rt<SDT>(snext[jtr * 16 + jg + 8 * h], sdt);
                }
            }, [&](int slot) {
                if constexpr (MORE) {
                    if (slot % STRIDE != STRIDE - 1 || slot / STRIDE >= 8) return;
                    // unit (h, t): word t, nibbles of row g + 8 h -> bf16 pairs at k0 (lo) and k0 + 8 (hi)
                    const int un = slot / STRIDE, h = un >> 2, t = un & 3;
                    // h = 1 keeps its nibbles high (v = 16 u): qe_tile::dq_pair's s / 16, -72 s
                    const float sv = h ? scl[h] * 0.0625f : scl[h], bv = h ? -72.f * scl[h] : -1032.f * scl[h];
                    const uint32_t u = wd[t] & (h ? 0xF0F0F0F0u : nib_mask());  // bytes: k0, k0+8, k0+1, k0+9
                    lo[h][t] = dq_pair(magic_f16<kSel02>(u), sv, bv);
                    hi[h][t] = dq_pair(magic_f16<kSel13>(u), sv, bv);
                    if (t == 3 && (NJOB >= NTH || jactive)) {
                        const int row = jtr * 16 + jg + 8 * h;
                        *reinterpret_cast<u32x4_v*>(wnext + swz(row, 2 * jj)) = u32x4_v{lo[h][0], lo[h][1], lo[h][2], lo[h][3]};
                        *reinterpret_cast<u32x4_v*>(wnext + swz(row, 2 * jj + 1)) = u32x4_v{hi[h][0], hi[h][1], hi[h][2], hi[h][3]};
                    }
                }
            }, std::true_type{});
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };
        for (int kt = 0; kt + 1 < KTL; kt++) kstep(kt, std::true_type{});
        kstep(KTL - 1, std::false_type{});
    } else {
        // X by LDS DMA (as the INT4 path), INT8 records through two register sets: step kt issues the DMA of X
        // (kt + 1) and the record loads of kt + 2 at its top, dequantizes the records of kt + 1 (loaded one step
        // earlier) into the other stage during its MFMAs, and ends with vmcnt(0) + the barrier.
        dma_x(kt0, 0);
        load_w8(wsA, kt0);
        if (KTL > 1) load_w8(wsB, kt0 + 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int d = 0; d < 4; d++) store_w8x(wsA, lds + BM * BK * 2, d);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        auto step = [&](int kt, const WSet& cur, WSet& nxt_regs) {
            char* nxt = lds + ((kt + 1) & 1) * C::kStage;
            if (kt + 1 < KTL) dma_x(kt0 + kt + 1, ((kt + 1) & 1) * C::kStage);
            const bool more = kt + 1 < KTL;
            mfma_step(kt, [] {}, [&](int slot) {
                if (slot % WMT != WMT - 1) return;  // after the last MFMA row of k16 step ks
                const int ks = slot / WMT;
                if (more) store_w8x(cur, nxt + BM * BK * 2, ks);
                if (ks == 0 && kt + 2 < KTL) load_w8(nxt_regs, kt0 + kt + 2);  // after the first stores free no registers
            }, std::false_type{});
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };
        for (int kt = 0; kt < KTL; kt += 2) {
            step(kt, wsB, wsA);
            if (kt + 1 < KTL) step(kt + 1, wsA, wsB);
        }
    }

    // ---- epilogue. The MFMAs take the W fragments as A and the X fragments as B, so each 32 x 32 tile holds C^T:
    //      lane l holds token l % 32 and weight rows (output columns) 8 (r / 4) + 4 (l / 32) + r % 4, i.e. 4
    //      consecutive output columns per r / 4 -> one 8-byte (bf16) or 16-byte (fp32) store, or scalar stores where
    //      ldc / c are not aligned for them. GLU: gate row g and up row g + 8 of a 16-row tile are registers r and
    //      r + 4 of the same lane.
    const int cj = lane & 31, ci = 4 * (lane >> 5);
    if (split_slot >= 0) {
        // raw fp32 partial of the whole BM x BN tile, [token][row] (rows past N / tokens past T included)
        float* pp = sp.part + (size_t)split_slot * BM * BN;
#pragma unroll
        for (int a = 0; a < WMT; a++)
#pragma unroll
            for (int bb = 0; bb < WNT; bb++)
#pragma unroll
                for (int rb = 0; rb < 4; rb++) {
                    const int tl = wm * 32 * WMT + a * 32 + cj, nl = wn * 32 * WNT + bb * 32 + 8 * rb + ci;
                    const f32x16_v& v = acc[a][bb];
                    *reinterpret_cast<f32x4_v*>(pp + (size_t)tl * BN + nl) =
                        f32x4_v{v[4 * rb], v[4 * rb + 1], v[4 * rb + 2], v[4 * rb + 3]};
                }
        return;
    }
    const bool vec = (ldc & 3) == 0 && ((uintptr_t)c & (out == kOutF32 ? 15u : 7u)) == 0;
    auto st4 = [&](uint16_t* p, float v0, float v1, float v2, float v3) {  // 4 consecutive bf16
        if (vec) {
            *reinterpret_cast<uint2*>(p) = uint2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
        } else {
            p[0] = f32_to_bf16(v0);
            p[1] = f32_to_bf16(v1);
            p[2] = f32_to_bf16(v2);
            p[3] = f32_to_bf16(v3);
        }
    };
#pragma unroll
    for (int a = 0; a < WMT; a++)
#pragma unroll
        for (int bb = 0; bb < WNT; bb++) {
            const int tok = t0 + wm * 32 * WMT + a * 32 + cj;
            if (tok >= T) continue;
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const int n = n0 + wn * 32 * WNT + bb * 32 + 8 * rb + ci;  // first of the 4 columns
                const f32x16_v& v = acc[a][bb];
                if (out == kOutGLU) {
                    if (rb & 1) continue;  // rows 8 (rb + 1) + ..: the up rows of this gate block
                    float g[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) g[j] = silu_f32(v[4 * rb + j]) * v[4 * rb + 4 + j];
                    if (n < N)
                        st4(reinterpret_cast<uint16_t*>(c) + (size_t)tok * ldc + (n >> 4) * 8 + (n & 7), g[0], g[1],
                            g[2], g[3]);
                } else if (n < N) {
                    if (out == kOutBF16) {
                        st4(reinterpret_cast<uint16_t*>(c) + (size_t)tok * ldc + n, v[4 * rb], v[4 * rb + 1],
                            v[4 * rb + 2], v[4 * rb + 3]);
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
}

// Split tiles' partials -> outputs: one thread per (split tile, token row, 16 output columns); the ks partials are
// added in split order (fixed order: the result does not depend on timing), then the epilogue of the GEMM
template <int BM, int BN>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ part, int ks, int ndirect,
                                                            int nsplit, int nbn, int T, int N, void* __restrict__ c,
                                                            int ldc, int out) {
    constexpr int CB = BN / 16;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)nsplit * BM * CB) return;
    const int st = (int)(idx / ((size_t)BM * CB)), r = (int)((idx / CB) % BM), cb = (int)(idx % CB);
    const int tile = ndirect + st;
    const int tok = (tile / nbn) * BM + r, n = (tile % nbn) * BN + 16 * cb;
    if (tok >= T || n >= N) return;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = 0.f;
    for (int z = 0; z < ks; z++) {
        const f32x4_v* p = reinterpret_cast<const f32x4_v*>(part + (((size_t)st * ks + z) * BM + r) * BN + 16 * cb);
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const f32x4_v a = p[q4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[4 * q4 + j] += a[j];
        }
    }
    if (out == kOutGLU) {
        uint16_t* o = reinterpret_cast<uint16_t*>(c) + (size_t)tok * ldc + (n >> 4) * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = f32_to_bf16(silu_f32(v[j]) * v[j + 8]);
    } else if (out == kOutBF16) {
        uint16_t* o = reinterpret_cast<uint16_t*>(c) + (size_t)tok * ldc + n;
#pragma unroll
        for (int j = 0; j < 16; j++) o[j] = f32_to_bf16(v[j]);
    } else {
        float* o = reinterpret_cast<float*>(c) + (size_t)tok * ldc + n;
#pragma unroll
        for (int j = 0; j < 16; j++) o[j] = v[j];
    }
}

// tile configurations: 0 = 256 tokens x 256 rows (WMT 4, WNT 2), 1 = 256 x 128 (4, 1)
constexpr int kNumCfg = 2;
template <int CFG>
struct CfgOf;
template <>
struct CfgOf<0> {
    static constexpr int WMT = 4, WNT = 2;
};
template <>
struct CfgOf<1> {
    static constexpr int WMT = 4, WNT = 1;
};

struct GemmGeom {
    int nbn, nbt, ntiles, ndirect, nsplit, ks;
    size_t ws_bytes;
};
// tiles of configuration cfg and, for ks > 1, the split of the last partial round (stream-K): whole rounds of
// tiles run directly, the remaining tiles as ks K ranges; false when that split does not apply (no partial round,
// K steps not divisible into even ranges)
bool gemm_geom(int cfg, int n, int k, int t, int ks, GemmGeom& g) {
    const int BM = 256, BN = cfg == 0 ? 256 : 128;
    g.nbn = (n + BN - 1) / BN;
    g.nbt = (t + BM - 1) / BM;
    g.ntiles = g.nbn * g.nbt;
    g.ks = ks;
    g.ndirect = g.ntiles;
    g.nsplit = 0;
    g.ws_bytes = 0;
    if (ks == 1) return true;
    const int cus = qe_num_cus(), KT = k / BK;
    if (KT % (2 * ks) != 0) return false;
    const int tail = g.ntiles % cus;
    if (tail == 0 || tail * ks > cus) return false;
    g.ndirect = g.ntiles - tail;
    g.nsplit = tail;
    g.ws_bytes = (size_t)tail * ks * BM * BN * 4;
    return true;
}

}  // namespace

void gemm_reserve(size_t bytes, hipStream_t st) {
    stream_ws_reserve(kWsSplit, bytes, st);
}

namespace {

template <int FMT, int SDT, int CFG>
void launch_cfg(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, int t, void* c, int ldc,
                int out, int sdt, const GemmGeom& g, float* part, hipStream_t st) {
    constexpr int WMT = CfgOf<CFG>::WMT, WNT = CfgOf<CFG>::WNT;
    using C = Cfg<WMT, WNT>;
    SplitArgs sp;
    sp.ndirect = g.ndirect;
    sp.ks = g.ks;
    sp.part = part;
    const int per = (g.ndirect + 7) / 8;
    const unsigned blocks = (unsigned)(8 * per + g.nsplit * g.ks);
    gemm_kernel<FMT, SDT, WMT, WNT><<<dim3(blocks), dim3(NTH), FMT == kFmtW4 ? C::kLdsW4 : 2 * C::kStage, st>>>(
        q, s, n, k, x, ldx, t, c, ldc, out, sdt, g.nbn, g.nbt, sp);
    HIP_CHECK(hipGetLastError());
    if (g.nsplit > 0) {
        const size_t threads = (size_t)g.nsplit * C::BM * (C::BN / 16);
        splitk_reduce_kernel<C::BM, C::BN><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st>>>(
            part, g.ks, g.ndirect, g.nsplit, g.nbn, t, n, c, ldc, out);
        HIP_CHECK(hipGetLastError());
    }
}

template <int FMT, int SDT>
void run_choice(int cfg, int ks, const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, int t,
                void* c, int ldc, int out, int sdt, hipStream_t st) {
    GemmGeom g;
    float* part = nullptr;
    if (ks > 1) {
        if (!gemm_geom(cfg, n, k, t, ks, g) || (part = static_cast<float*>(stream_ws(kWsSplit, g.ws_bytes, st))) == nullptr) ks = 1;
    }
    if (ks == 1) gemm_geom(cfg, n, k, t, 1, g);
    if (cfg == 0) launch_cfg<FMT, SDT, 0>(q, s, n, k, x, ldx, t, c, ldc, out, sdt, g, part, st);
    else launch_cfg<FMT, SDT, 1>(q, s, n, k, x, ldx, t, c, ldc, out, sdt, g, part, st);
}

// untuned choice (cost model): 256 x 256 tiles when they fill the CUs at least once (else 256 x 128), with the last
// partial round split in two K ranges when it is at most half full
GemmChoice gemm_model_choice(int n, int k, int t) {
    const int cus = qe_num_cus();
    const long tiles_big = (long)((n + 255) / 256) * ((t + 255) / 256);
    GemmChoice ch{tiles_big >= cus ? 0 : 1, 1};
    GemmGeom g;
    if (ch.cfg == 0 && gemm_geom(0, n, k, t, 2, g)) ch.ks = 2;
    else if (ch.cfg == 0) {
        const long rounds = (tiles_big + cus - 1) / cus;
        if ((double)tiles_big / (rounds * cus) < 0.9) ch.cfg = 1;
    }
    return ch;
}

// timed choice: every (configuration, split) candidate once untimed, then 5 rounds in rotating order, the median;
// outside graph capture only (during capture: the cost model)
template <int FMT, int SDT>
GemmChoice gemm_tune_choice(int n, int k, const uint16_t* x, int ldx, int t, void* c, int ldc, int out, int sdt,
                            const uint4* q, const uint16_t* s, hipStream_t st) {
    std::vector<GemmChoice> cl;
    for (int cfg = 0; cfg < kNumCfg; cfg++)
        for (int ks : {1, 2, 4}) {
            GemmGeom g;
            if (gemm_geom(cfg, n, k, t, ks, g)) cl.push_back(GemmChoice{cfg, ks});
        }
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    auto time1 = [&](const GemmChoice& ch) {
        HIP_CHECK(hipEventRecord(e0, st));
        run_choice<FMT, SDT>(ch.cfg, ch.ks, q, s, n, k, x, ldx, t, c, ldc, out, sdt, st);
        HIP_CHECK(hipEventRecord(e1, st));
        HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0.f;
        HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        return ms;
    };
    for (const auto& ch : cl) time1(ch);
    constexpr int kReps = 5;
    std::vector<std::vector<float>> ts(cl.size());
    for (int r = 0; r < kReps; r++)
        for (size_t j = 0; j < cl.size(); j++) {
            const size_t i = (j + r) % cl.size();
            ts[i].push_back(time1(cl[i]));
        }
    size_t best = 0;
    float best_ms = 1e30f;
    for (size_t j = 0; j < cl.size(); j++) {
        std::sort(ts[j].begin(), ts[j].end());
        if (ts[j][kReps / 2] < best_ms) {
            best_ms = ts[j][kReps / 2];
            best = j;
        }
    }
    HIP_CHECK(hipEventDestroy(e0));
    HIP_CHECK(hipEventDestroy(e1));
    return cl[best];
}

// the largest split <= ks that qe_gemm_set_sk_maxparts allows (splits are 1, 2 or 4)
int capped_split(int ks) {
    const int cap = gemm_sk_maxparts();
    while (cap > 0 && ks > cap) ks /= 2;
    return ks < 1 ? 1 : ks;
}

template <int FMT, int SDT>
void launch_gemm(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, int t, void* c, int ldc,
                 int out, int sdt, bool tuned, hipStream_t st) {
    GemmChoice ch;
    const GemmKey key{FMT, n, k, gemm_bucket(t), out == kOutGLU ? 1 : 0};
    if (!gemm_table_find(key, ch)) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIP_CHECK(hipStreamIsCapturing(st, &cs));
        if ((tuned || qe_config().gemm_tune) && cs == hipStreamCaptureStatusNone) {
            ch = gemm_tune_choice<FMT, SDT>(n, k, x, ldx, t, c, ldc, out, sdt, q, s, st);
            gemm_table_add(key, ch);
        } else {
            ch = gemm_model_choice(n, k, t);
        }
    }
    run_choice<FMT, SDT>(ch.cfg, capped_split(ch.ks), q, s, n, k, x, ldx, t, c, ldc, out, sdt, st);
}

void gemm_check(int n, int k, const void* x, int ldx, int ldc, int t, bool glu) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && t >= 1, "gemm %d %d %d", n, k, t);
    CHECK(ldx >= k && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0, "gemm ldx %d (multiple of 8, x 16-byte aligned)", ldx);
    CHECK(ldc >= (glu ? n / 2 : n), "gemm ldc %d", ldc);
    CHECK((long)((n + 127) / 128) * ((t + 255) / 256) < (1L << 31) / 8, "gemm t %d n %d", t, n);
}

}  // namespace

void gemm_w4(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st,
             bool tuned) {
    gemm_check(w.n, w.k, x, ldx, ldc, t, w.glu);
    if (qe_config().gemm_h16) {  // the reference's fp16-accumulate numerics (its QE_GEMM_H16 with W4A8 off)
        gemm_w4h(w, x, ldx, c, ldc, t, out_bf16, st);
        return;
    }
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    if (w.sdt == kScaleF16) launch_gemm<kFmtW4, kScaleF16>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, tuned, st);
    else launch_gemm<kFmtW4, kScaleBF16>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, tuned, st);
}

void gemm_w4_choice(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, int cfg, int ks,
                    hipStream_t st) {
    gemm_check(w.n, w.k, x, ldx, ldc, t, w.glu);
    CHECK(cfg >= 0 && cfg < kNumCfg && (ks == 1 || ks == 2 || ks == 4), "gemm choice cfg %d ks %d", cfg, ks);
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    if (w.sdt == kScaleF16) run_choice<kFmtW4, kScaleF16>(cfg, ks, w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, st);
    else run_choice<kFmtW4, kScaleBF16>(cfg, ks, w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, st);
}

bool gemm_split_applies(int cfg, int n, int k, int t, int ks) {
    GemmGeom g;
    return gemm_geom(cfg, n, k, t, ks, g) && g.nsplit > 0;
}

void gemm_w8(const W8& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st,
             bool tuned) {
    gemm_check(w.n, w.k, x, ldx, ldc, t, w.glu);
    CHECK(!w.glu || w.q8, "gemm_w8: GLU is for Q8 matrices");
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
    if (w.q8) launch_gemm<kFmtQ8, -1>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, tuned, st);
    else if (w.per_channel) launch_gemm<kFmtW8C, -1>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, tuned, st);
    else launch_gemm<kFmtW8G, -1>(w.q, w.s, w.n, w.k, x, ldx, t, c, ldc, out, w.sdt, tuned, st);
}

void matmul_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    if (m > kMatmulGemvRows) {
        gemm_w4(w, x, ldx, y, ldy, m, out_bf16, st);
        return;
    }
    // 17..64 rows: one pass over the weights (wdec.hip) where the shape fits it and it is the faster choice, unless
    // every row must keep the bits it has alone (batch_invariant)
    if (m > kMaxGemvRows && !qe_config().batch_invariant && wdec_w4_pick(w, x, ldx, m)) {
        wdec_w4(w, x, ldx, y, ldy, m, out_bf16, st);
        return;
    }
    // row blocks: 32 rows per launch (the skinny kernel's wide variant) while more than 16 remain and the rows are
    // 16-byte aligned, else 16; a row's bits do not depend on the block it falls in
    const size_t esz = (w.glu || out_bf16) ? 2 : 4;
    const bool aligned = ((uintptr_t)x & 15) == 0 && ldx % 8 == 0;
    for (int r0 = 0; r0 < m;) {
        const int left = m - r0;
        char* yr = reinterpret_cast<char*>(y) + (size_t)r0 * ldy * esz;
        if (aligned && left > kMaxGemvRows) {
            const int mm = left < kWideRows ? left : kWideRows;
            skinny_w4_wide(w, x + (size_t)r0 * ldx, ldx, yr, ldy, mm, out_bf16, st);
            r0 += mm;
        } else {
            const int mm = left < kMaxGemvRows ? left : kMaxGemvRows;
            gemv_w4(w, x + (size_t)r0 * ldx, ldx, yr, ldy, mm, out_bf16, st);
            r0 += mm;
        }
    }
}
