// MoE grouped prefill GEMMs (gate_up with the GLU epilogue, down into the slot rows) with the expert weights
// dequantized in registers.
//
// The dense prefill GEMM dequantizes a 256-row W tile into LDS once per k step and every wave reads its fragments
// back; with ~80 rows per expert (C4, T = 4096) each dequantized weight feeds only ~80 tokens, so the
// dequantization costs as much issue as the MFMAs it feeds and the step time is their sum. Here each wave owns 64
// weight rows (four 16-row tiles) of a 512-row block and turns its own W4 records straight into MFMA A operands,
// placed between the MFMAs of the previous k16 step so that the vector ALU and the matrix cores work at the same
// time; LDS carries only the job's gathered activation rows (B operands of all eight waves), each wave's raw records
// and scales.
//
// Operand layout (v_mfma_f32_32x32x16_bf16, A = weights, B = activations): lane l = 32 kh + m is A row m = 8 q + g
// (tile q of the wave, row pair g / g + 8), k half kh. A W4 record (g, t) holds rows g (low nibbles) and g + 8 (high
// nibbles) at k = 16 j + 2 t + {0, 8, 1, 9} in bytes 0..3 of word j (64-k steps, records of 512 B per tile), so
// bytes (h, h + 2) of word j of the four records t = 0..3 are the 8 consecutive k of 16-byte chunk 2 j + h. The
// MFMAs take the chunks of a step in the order c(ks, kh) = 2 (2 (ks % 2) + kh) + ks / 2 (k16 step ks, k half kh): a
// lane needs only words kh and 2 + kh of its row pair's four records, every lane of a k16 step the same byte pair
// (h = ks / 2), and the B operand is chunk c of the token's row, one ds_read_b128 of the swizzled activation tile.
// Low nibbles = A of row g (operand 0), high nibbles = A of row g + 8 (operand 1). gate_up (MODE 1): weights
// bf16_rn((u - 8) s) (the high nibbles are converted as 16 u and multiplied by s / 16: the same fma) on bf16
// activations, the dense kernel's arithmetic (only the order of the k inside the step differs); down (MODE 2): weights
// fp16_rn((u - 8) s) on the fp16 activation (act / 16) on the f16 matrix cores (v_mfma_f32_32x32x16_f16, the same
// operand layout). Products accumulated in fp32 by the MFMAs. The activation and the slot rows are fp16 of the
// value / 16 (the reference's fp16 intermediates).
//
// Output: D row i = 8 (r / 4) + 4 (l / 32) + r % 4 of lane l register r is A row m = i: tile r / 4 of the wave, row
// pair g = 4 (l / 32) + r % 4; operand 0 holds row g (gate), operand 1 row g + 8 (up) of the same register, so the
// GLU epilogue pairs acc[a][0][r] with acc[a][1][r], and registers r = 4 q .. 4 q + 3 are 4 consecutive outputs.
#include "mfma_tile.hpp"
#include <type_traits>

namespace qe_moe_rw {
using namespace qe_tile;

constexpr int NTH = 512, BM = 128, BN = 512, BK = 64, NBUF = 4;
constexpr int kXStage = BM * BK * 2;         // gathered activation rows of one k step: [128][64] bf16, swizzled
constexpr int kRawWave = 2048;               // one wave's two 1 KB record loads of one k step
constexpr int kScWave = 256;                 // one wave's scales of one k step: [4 tiles][16 rows] fp16 (+ a copy)
constexpr int kRawOff = NBUF * kXStage, kScOff = kRawOff + NBUF * 8 * kRawWave;
constexpr int kLds = kScOff + NBUF * 8 * kScWave;  // 136 KB: every buffer four deep (steps kt .. kt + 3)

// MODE 1: gate_up, N = 2 I GLU rows (records of 256 rows x K = H), epilogue act[slot][I] = silu(gate) up w_slot.
// MODE 2: down, N = H rows, K = I over the expert's records (128 k each), epilogue slot_out[slot][H].
// NA: 32-row token tiles holding a row of the job (the others are not computed). SHORT: K = 128 (two k steps).
template <int MODE, int NA, bool SHORT>
__device__ __forceinline__ void rw_body(const MoePfArgs& ma, char* lds, int nt, int e, int slot0, int T) {
    constexpr int NS = 2 * NA;  // MFMAs per k16 step
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned lds32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);
    const int N = MODE == 1 ? 2 * ma.I : ma.H, K = MODE == 1 ? ma.H : ma.I;
    const int KT = K / BK, G = K >> 7;
    const int wrow = nt * BN + 64 * wave;  // first weight row of this wave
    const bool wact = wrow < N;            // wave-uniform: N is a multiple of 64
    const int drow = wact ? wrow : N - 64;  // rows whose records a wave loads (waves past N: loaded, not used)
    const int m = lane & 31, kh = lane >> 5, g = m & 7;
    const int tl = (wrow >> 4) + (m >> 3);  // the lane's 16-row tile among the expert's N rows

    // records of 64-k step kt: DMA d, lane i fetches record (g = i % 8, t = 2 d + i / 32) of wave tile (i / 8) % 4 into
    // LDS slot 64 d + i = 32 t + m (m = i % 32: the row pair of A row m)
    const int dt = (lane >> 3) & 3;  // wave tile of this lane's DMA record
    auto w_at = [&](int kt) -> const uint4* {
        const int t2 = (drow >> 4) + dt;
        if constexpr (MODE == 1) {
            const char* rp = ma.recs + ((size_t)e * ma.ngrp + (drow >> 8)) * ma.rec;
            return reinterpret_cast<const uint4*>(rp) + ((size_t)(t2 & 15) * (K >> 6) + kt) * 32 + 4 * g + kh;
        } else {
            const char* rp = ma.recs + ((size_t)e * ma.ngrp + (kt >> 1)) * ma.rec + ma.gg_q + ma.gg_s;
            return reinterpret_cast<const uint4*>(rp) + ((size_t)t2 * 2 + (kt & 1)) * 32 + 4 * g + kh;
        }
    };
    // scale dword (rows 2 d, 2 d + 1) of wave tile q for group grp; DMA lane l fetches q = (l / 8) % 4, d = l % 8
    const int sq = (lane >> 3) & 3, sd = lane & 7;
    auto s_at = [&](int grp) -> const uint16_t* {
        const int t = (drow >> 4) + sq;
        if constexpr (MODE == 1) {
            const char* rp = ma.recs + ((size_t)e * ma.ngrp + (drow >> 8)) * ma.rec + ma.gg_q;
            return reinterpret_cast<const uint16_t*>(rp) + ((size_t)(t & 15) * G + grp) * 16 + 2 * sd;
        } else {
            const char* rp = ma.recs + ((size_t)e * ma.ngrp + grp) * ma.rec + ma.gg_q + ma.gg_s + ma.gd_q;
            return reinterpret_cast<const uint16_t*>(rp) + (size_t)t * 16 + 2 * sd;
        }
    };
    // gathered activation rows: wave w stages rows 16 w .. 16 w + 15 (two 1 KB DMAs of 8 rows; lane i lands at slot i
    // of its 8-row block, so it loads the chunk the swizzle puts there); rows past T re-read row T - 1 (their outputs
    // are not stored)
    const uint16_t* xrow[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int row = wave * 16 + i * 8 + (lane >> 3);
        const int sl = slot0 + (row < T ? row : T - 1);
        xrow[i] = ma.a + (MODE == 1 ? (size_t)ma.slot_tok[sl] * ma.H : (size_t)sl * ma.I) + ((lane & 7) ^ swz_f(row)) * 8;
    }
    // step kt's 5 DMAs per wave into buffer kt % 4: the activation rows (2), the wave's records (2) and scales (1).
    // Every wave issues the same 5, so a wait for all but the last `after` steps is vmcnt(5 after).
    auto dma_step = [&](int kt) {
        const int buf = kt % NBUF;
#pragma unroll
        for (int i = 0; i < 2; i++) dma16(xrow[i] + kt * BK, lds32 + buf * kXStage + (wave * 16 + i * 8) * 128);
        const uint4* p = w_at(kt);
        const unsigned dst = lds32 + kRawOff + (buf * 8 + wave) * kRawWave;
        dma16(p, dst);             // t = 0, 1
        dma16(p + 2, dst + 1024);  // t = 2, 3
        dma4(s_at(kt >> 1), lds32 + kScOff + (buf * 8 + wave) * kScWave);
    };
    auto wait_dma = [&](auto after) {
        constexpr int A = decltype(after)::value;
        if constexpr (A == 2) asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
        else if constexpr (A == 1) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };

    f32x16_v acc[NA][2];
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][h][r] = 0.f;
    // B operand of k16 step ks: chunk c(ks, kh) of row m of a 32-row block (swz_f depends on the row mod 32 only)
    int xo[BK / 16];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) xo[ks] = m * 128 + (((4 * (ks & 1) + 2 * kh + (ks >> 1)) ^ swz_f(m)) << 4);

    // operand state, two sets (by step parity): the masked words of a step (low / high nibbles of words kh and 2 + kh
    // of records t = 0..3) and its scales; the next A operands by k16 parity (0: row g, 1: row g + 8)
    uint32_t mw[2][2][4][2];  // [set][nibble half][record t][word: kh, 2 + kh]
    float sl[2], sh16[2], bl[2], bh[2];
    u32x4_v an[2][2];  // [k16 parity][operand]
    auto load_step = [&](int kt, auto set) {  // this wave's records and scales of step kt (its own DMAs, landed)
        constexpr int S = decltype(set)::value;
        const int buf = kt % NBUF;
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(lds + kRawOff + (buf * 8 + wave) * kRawWave) + m * 4 + kh;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const uint32_t v = rw[t * 128 + 2 * w];  // record slot 32 t + m, word kh + 2 w
                mw[S][0][t][w] = v & nib_mask();
                mw[S][1][t][w] = v & nib_mask_hi();  // 16 u: times s / 16
            }
        const uint16_t* sc = reinterpret_cast<const uint16_t*>(lds + kScOff + (buf * 8 + wave) * kScWave) + (m >> 3) * 16 + g;
        sl[S] = scale_to_f32<kScaleF16>(sc[0]);
        const float s_hi = scale_to_f32<kScaleF16>(sc[8]);
        sh16[S] = s_hi * 0.0625f;
        bl[S] = -1032.f * sl[S];  // qe_tile::dq_pair: v = u (low), v = 16 u (high, s / 16)
        bh[S] = -72.f * s_hi;
    };
    // unit u of the dequantization of k16 step j from set S: operand u / 4, pair t = u % 4 (record t, bytes
    // (h, h + 2) of word 2 (j % 2) + kh, h = j / 2)
    auto unit = [&](int u, int j, auto set) {
        constexpr int S = decltype(set)::value;
        const int bb = u >> 2, t = u & 3;
        const uint32_t v = mw[S][bb][t][j & 1];
        const float s = bb ? sh16[S] : sl[S], bias = bb ? bh[S] : bl[S];
        an[j & 1][bb][t] = (j >> 1) ? dq_pair<MODE == 2>(magic_f16<kSel13>(v), s, bias)
                                    : dq_pair<MODE == 2>(magic_f16<kSel02>(v), s, bias);
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using PM1 = std::integral_constant<int, -1>;
    // prologue: DMAs of steps 0, 1, 2 (0, 1 if SHORT), wait for step 0, its first operands
    dma_step(0);
    dma_step(1);
    if constexpr (SHORT) {
        wait_dma(P1{});
    } else {
        dma_step(2);
        wait_dma(P2{});
    }
    __builtin_amdgcn_s_barrier();
    if (wact) {
        load_step(0, P0{});
#pragma unroll
        for (int u = 0; u < 8; u++) unit(u, 0, P0{});
    }

    bf16x8_v xf[2][NA];
    auto read_x = [&](const char* xt, int ks, int buf) {
#pragma unroll
        for (int a = 0; a < NA; a++) xf[buf][a] = *reinterpret_cast<const bf16x8_v*>(xt + xo[ks] + a * 32 * 128);
    };

    // step kt (set = kt % 2): DMAs of kt + 3 (DMA); per k16 step ks the 2 NA MFMAs on the current operands, each
    // followed by its share of the 8 units that build the next operands (ks + 1 from this step's set, or step kt + 1's
    // first from the other set: its records are read at ks = 2, after the wait for its DMAs; AFTER: steps issued
    // after kt + 1). Nothing is scheduled across the fences, so the units keep their place.
    auto kstep = [&](int kt, auto more, auto set, auto dma, auto after) {
        constexpr bool MORE = decltype(more)::value;
        constexpr int S = decltype(set)::value;
        using SN = std::integral_constant<int, S ^ 1>;
        if constexpr (decltype(dma)::value) dma_step(kt + 3);
        if (wact) {
            const char* xt = lds + (kt % NBUF) * kXStage;
            read_x(xt, 0, 0);
#pragma unroll
            for (int ks = 0; ks < BK / 16; ks++) {
                const u32x4_v a0 = an[ks & 1][0], a1 = an[ks & 1][1];
                const bf16x8_v A0 = __builtin_bit_cast(bf16x8_v, a0);
                const bf16x8_v A1 = __builtin_bit_cast(bf16x8_v, a1);
                if (ks + 1 < BK / 16) read_x(xt, ks + 1, (ks + 1) & 1);
                if (ks == 2 && MORE) {
                    wait_dma(after);
                    load_step(kt + 1, SN{});
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < NS; i++) {
                    const int a = i >> 1;
                    if constexpr (MODE == 2) {
                        const bf16x8_v xb = xf[ks & 1][a];  // bit casts take a scalar temporary
                        const f16x8_v B = __builtin_bit_cast(f16x8_v, xb);
                        if (i & 1) acc[a][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_v, a1), B, acc[a][1], 0, 0, 0);
                        else acc[a][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_v, a0), B, acc[a][0], 0, 0, 0);
                    } else {
                        if (i & 1) acc[a][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A1, xf[ks & 1][a], acc[a][1], 0, 0, 0);
                        else acc[a][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A0, xf[ks & 1][a], acc[a][0], 0, 0, 0);
                    }
                    if (ks + 1 < BK / 16) {
#pragma unroll
                        for (int u = 0; u < 8; u++)
                            if ((u * NS) / 8 == i) unit(u, ks + 1, set);
                    } else if (MORE) {
#pragma unroll
                        for (int u = 0; u < 8; u++)
                            if ((u * NS) / 8 == i) unit(u, 0, SN{});
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        wait_dma(after);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    // KT even, >= 4: pairs of steps with DMAs three ahead, then the last four (DMA of the last step, none); SHORT:
    // the two steps
    using T_ = std::true_type;
    using F_ = std::false_type;
    if constexpr (SHORT) {
        kstep(0, T_{}, P0{}, F_{}, P0{});
        kstep(1, F_{}, P1{}, F_{}, PM1{});
    } else {
        for (int kt = 0; kt + 4 < KT; kt += 2) {
            kstep(kt, T_{}, P0{}, T_{}, P2{});
            kstep(kt + 1, T_{}, P1{}, T_{}, P2{});
        }
        kstep(KT - 4, T_{}, P0{}, T_{}, P2{});
        kstep(KT - 3, T_{}, P1{}, F_{}, P1{});
        kstep(KT - 2, T_{}, P0{}, F_{}, P0{});
        kstep(KT - 1, F_{}, P1{}, F_{}, PM1{});
    }

    if (!wact) return;
    // epilogue: lane l holds token a * 32 + l % 32; register r = 4 q + j is row pair g = 4 (l / 32) + j of tile q
#pragma unroll
    for (int a = 0; a < NA; a++) {
        const int tok = a * 32 + m;
        if (tok >= T) continue;
        const int slot = slot0 + tok;
        if constexpr (MODE == 1) {
            const float sw = ma.slot_w[slot];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    v[j] = silu_f32(acc[a][0][4 * q + j]) * acc[a][1][4 * q + j] * sw * kMoeF16Scale;
                const int col = ((wrow >> 4) + q) * 8 + 4 * kh;
                *reinterpret_cast<uint2*>(ma.out + (size_t)slot * ma.I + col) =
                    uint2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = wrow + 16 * q + 4 * kh;
                uint16_t* o = ma.out + (size_t)slot * ma.H + n;
                const f32x16_v& lo = acc[a][0];
                const f32x16_v& hi = acc[a][1];
                // the activation is act / 16, so the sums are the slot / 16: stored as is (fp16)
                *reinterpret_cast<uint2*>(o) =
                    uint2{pack_f16x2(lo[4 * q], lo[4 * q + 1]), pack_f16x2(lo[4 * q + 2], lo[4 * q + 3])};
                *reinterpret_cast<uint2*>(o + 8) =
                    uint2{pack_f16x2(hi[4 * q], hi[4 * q + 1]), pack_f16x2(hi[4 * q + 2], hi[4 * q + 3])};
            }
        }
    }
}

// Block b: XCD b % 8, n tile (b / 8) % nbn, job (b / 8 / nbn) * 8 + b % 8 (the n tiles of a job share its gathered
// rows in that XCD's L2)
template <int MODE>
__global__ void __launch_bounds__(NTH) moe_rw_kernel(MoePfArgs ma, int nbn) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int b = blockIdx.x, r8 = b >> 3;
    const int nt = r8 % nbn;
    const int job = (r8 / nbn) * 8 + (b & 7);
    if (job >= *ma.njobs) return;
    const int e = ma.jobs[2 * job];
    const int slot0 = ma.off[e] + ma.jobs[2 * job + 1];
    const int T = min(BM, ma.off[e + 1] - slot0);  // rows of the job, >= 1
    const int na = __builtin_amdgcn_readfirstlane((T + 31) >> 5);
    if ((MODE == 1 ? ma.H : ma.I) == 128) {
        if constexpr (MODE == 2) {  // (gate_up: K = H, a multiple of 512)
            if (na >= 4) rw_body<MODE, 4, true>(ma, lds, nt, e, slot0, T);
            else if (na == 3) rw_body<MODE, 3, true>(ma, lds, nt, e, slot0, T);
            else if (na == 2) rw_body<MODE, 2, true>(ma, lds, nt, e, slot0, T);
            else rw_body<MODE, 1, true>(ma, lds, nt, e, slot0, T);
        }
        return;
    }
    if (na >= 4) rw_body<MODE, 4, false>(ma, lds, nt, e, slot0, T);
    else if (na == 3) rw_body<MODE, 3, false>(ma, lds, nt, e, slot0, T);
    else if (na == 2) rw_body<MODE, 2, false>(ma, lds, nt, e, slot0, T);
    else rw_body<MODE, 1, false>(ma, lds, nt, e, slot0, T);
}

}  // namespace qe_moe_rw

// grid = 8 XCD lanes x ceil(max_jobs / 8) job groups x n tiles of 512 rows (blocks past the job count exit)
void moe_pf_gemm(int mode, const MoePfArgs& a, hipStream_t st) {
    using namespace qe_moe_rw;
    const int N = mode == 1 ? 2 * a.I : a.H, K = mode == 1 ? a.H : a.I;
    // K = 128 runs the two-step variant; the others need an even number of 64-k steps, at least 4
    CHECK(N % 64 == 0 && K % 128 == 0 && (mode == 2 || K >= 512) && a.max_jobs >= 1, "moe_pf mode %d N %d K %d", mode,
          N, K);
    const int nbn = (N + BN - 1) / BN;
    const unsigned grid = 8u * (unsigned)((a.max_jobs + 7) / 8) * (unsigned)nbn;
    if (mode == 1) moe_rw_kernel<1><<<grid, NTH, kLds, st>>>(a, nbn);
    else moe_rw_kernel<2><<<grid, NTH, kLds, st>>>(a, nbn);
    HIP_CHECK(hipGetLastError());
}
