// Decode GEMV for one activation row (m = 1) on the W4 layout, with the multiply-adds on the matrix cores.
//
// The VALU GEMV (gemv_impl.hpp) spends one v_dot2 per weight pair next to the unpack, and at m = 1 its VALU
// work, not HBM, sets the time. Here each lane keeps the W4 record it loads (one coalesced 1 KB wave-load per
// 128-k group, the layout unchanged) and v_mfma_f32_16x16x32_bf16 does the products:
//   * lane L = 16 q + c holds W4 lane L % 32 of chunk L / 32: rows g = 4 (q & 1) + c / 4 (low nibbles) and
//     g + 8 (high nibbles), k = 64 h + 16 j + 2 t + {0, 1, 8, 9}, h = q / 2, t = c % 4, j = 0..3. As an MFMA A
//     operand, lane (q, c) is A row c with k slots 8 q .. 8 q + 7; its eight values of one row for words j, j + 1
//     are one operand: ((w >> sh) & 0x000F000F) | 0x43004300 is the bf16 pair 128 + u of k, k + 1 (sh = 0 / 8
//     for row g, 4 / 12 for row g + 8).
//   * Lanes of one A row c hold different k sets (t = c % 4 and h differ), so B is block diagonal: column
//     4 q + t of k block q holds the activations of class (h = q / 2, t), every other entry is 0. Output entry
//     D[c][4 q + (c % 4)] is then exactly lane (q, c)'s own dot product; lane L of D holds it in register c % 4
//     (D rows 4 q' .. 4 q' + 3 of column c'), for row g = 4 ((c' / 4) & 1) + q' of class (h = c' / 8, t = c' % 4).
//     The activations are staged class-major in LDS, so a B operand is one ds_read_b128; lanes off the diagonal
//     read a zeroed block.
//   * The bias (u = w + 8 over the 128 of the magic) enters as the MFMA's initial C: -136 times the class sum
//     of the activations, computed once per group at staging. D = sum (u - 8) x exactly (products exact in fp32).
//   * Per group: acc += s * D (the group scale of the lane's row), the other three registers are carried along
//     unused. At the end the lane keeps register c % 4, the quad (t) and the two chunk halves (h) are added by
//     DPP, and the K slices (waves) through LDS in a fixed order: deterministic.
// Per lane and group that is 28 VALU for the unpack and 8 for the scales, against about 60 for the VALU GEMV.
#include "gemv_impl.hpp"
#include "mfma_tile.hpp"

namespace qe_gemv1 {
using namespace qe_gemv;

// register r of a (r = 2 b2 + b1): selects (v_cndmask_b32), no branch
__device__ __forceinline__ float pick4(f32x4_v a, bool b1, bool b2) {
    const float lo = b1 ? a[1] : a[0], hi = b1 ? a[3] : a[2];
    return b2 ? hi : lo;
}

// Staging works on 8-dword pieces of the wave's activation slice, 64 pieces (one per lane) per round; the arrays
// are padded to whole rounds so every lane stages unconditionally (lanes past the slice write duplicates into the
// padding): a staging branch would let the compiler sink the early activation loads into it, behind the weight
// loads, and vmcnt retires in order.
template <int NG>
constexpr int stage_groups() {
    return (NG * 8 + 63) / 64 * 8;
}
// LDS per wave (dwords): xl [GP][kGStride] activations class-major (64 dwords of a group, kGStride apart: with 64
// the 8 groups a staging store covers hit the same banks, an 8-way conflict; with 68 they are 4 banks apart),
// zero [GP][8] (the B operand of lanes off the diagonal), xsum [GP][8] (-136 x class sums), scales [GP][8] pairs
// (s[g], s[g + 8]) of 16-bit values, GP = stage_groups; then red [S][16] floats for the block
constexpr int kGStride = 68;
template <int NG>
constexpr int wave_dwords() {
    return stage_groups<NG>() * (kGStride + 8 + 8 + 8);
}

// NG groups per wave (K slice), D weight records in flight per lane (D < NG: a sliding window, the load of group
// i + D is issued once group i has been unpacked, so a wave receives its weights spread over the stream instead
// of in one burst and the compute left after its last bytes arrive is one group, not a whole slice).
template <int NG, int D, int SDT>
__global__ void __launch_bounds__(64 * kMaxWaves) __attribute__((amdgpu_waves_per_eu(7)))
gemv1_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s, int N, int K,
             const uint16_t* __restrict__ x, void* __restrict__ y, int out) {
    constexpr int WSZ = wave_dwords<NG>();
    constexpr int NP = NG * 8;              // 8-dword activation pieces (and scale dwords, class sums) of a slice
    constexpr int NR = (NP + 63) / 64;      // pieces per lane
    constexpr int GP = stage_groups<NG>();  // staged groups including the padding
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    const int tile = blockIdx.x, G = K >> 7, gb = w * NG;
    uint32_t* xl = lds + (size_t)w * WSZ;                          // [GP][kGStride]
    uint32_t* zr = xl + GP * kGStride;                               // [GP][8] zeros
    float* xsum = reinterpret_cast<float*>(zr + GP * 8);             // [GP][8]
    uint16_t* sl16 = reinterpret_cast<uint16_t*>(xsum + GP * 8);     // [GP][8][2]: (s[g], s[g + 8])
    float* red = reinterpret_cast<float*>(lds + (size_t)S * WSZ);  // [S][16]

    // 1. loads, no wait between them: the activation pieces of the slice (piece p = L + 64 r: dwords 8 p .. 8 p + 7,
    //    group p / 8), the slice's scales (dword p), then the first D groups of weight records.
    //    Addresses are clamped rather than branched on, so nothing waits before the weight stream starts.
    const uint32_t* xs0 = reinterpret_cast<const uint32_t*>(x) + (size_t)gb * 64;
    const uint32_t* ss0 = reinterpret_cast<const uint32_t*>(s + ((size_t)tile * G + gb) * 16);
    u32x4_v xv[NR][2];
    uint32_t sraw[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int p = L + 64 * r < NP ? L + 64 * r : NP - 1;
        xv[r][0] = reinterpret_cast<const u32x4_v*>(xs0)[2 * p];
        xv[r][1] = reinterpret_cast<const u32x4_v*>(xs0)[2 * p + 1];
        sraw[r] = ss0[p];
    }
    const uint4* qp = q + ((size_t)tile * (K >> 6) + 2 * gb) * 32 + L;
    u32x4_v wv[D];
#pragma unroll
    for (int i = 0; i < D; i++) wv[i] = ld_stream(qp + (size_t)i * 64);
    __builtin_amdgcn_sched_barrier(0);

    // 2. staging (every lane, whole rounds): scales as (s[g], s[g + 8]) pairs, activations class-major (x_slot),
    //    then the class sums times -136. Scale dword p holds rows 2 (p % 8) and 2 (p % 8) + 1 of group p / 8.
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int p = L + 64 * r;
        const int gi = p >> 3, l8 = p & 7;
        zr[p] = 0u;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int row = 2 * l8 + e;
            sl16[(gi * 8 + (row & 7)) * 2 + (row >> 3)] = (uint16_t)(sraw[r] >> (16 * e));
        }
#pragma unroll
        for (int e = 0; e < 8; e++) xl[gi * kGStride + x_slot<kFmtW4>(8 * l8 + e)] = e < 4 ? xv[r][0][e] : xv[r][1][e - 4];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int p = L + 64 * r;
        const u32x4_v* cl = reinterpret_cast<const u32x4_v*>(&xl[(p >> 3) * kGStride + (p & 7) * 8]);
        const u32x4_v a0 = cl[0], a1 = cl[1];
        float sm = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) sm = dot2_bf16(a0[e], 0x3F803F80u, sm);  // x_lo + x_hi (bf16 (1, 1))
#pragma unroll
        for (int e = 0; e < 4; e++) sm = dot2_bf16(a1[e], 0x3F803F80u, sm);
        xsum[p] = -136.f * sm;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 3. per group: 4 MFMAs (rows g / g + 8 x words 0-1 / 2-3), acc += s * D
    const int qb = L >> 4, c = L & 15;
    const bool diag = (c >> 2) == qb;
    // B operand: class 4 (q / 2) + c % 4 of the staged activations on the diagonal, else 8 zeros; group i is
    // kGStride dwords further for the diagonal lanes, 8 for the others (no branch in the loop: a branch per group would
    // let the compiler sink every group's FMAs to the end and keep all D results live)
    const uint32_t* bb = diag ? &xl[(4 * (qb >> 1) + (c & 3)) * 8] : zr;
    const int bstep = diag ? kGStride : 8;
    const float* cb = &xsum[4 * (c >> 3)];  // class sums of classes 4 (c / 8) .. + 3 (register r <-> t = r)
    const int grow = 4 * ((c >> 2) & 1) + qb;  // row (low nibbles) of the lane's useful D entry
    f32x4_v acc_lo = {0.f, 0.f, 0.f, 0.f}, acc_hi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const u32x4_v b01 = *reinterpret_cast<const u32x4_v*>(bb + i * bstep);
        const u32x4_v b23 = *reinterpret_cast<const u32x4_v*>(bb + i * bstep + 4);
        const f32x4_v c0 = *reinterpret_cast<const f32x4_v*>(cb + i * 8);
        const bf16x8_v B01 = __builtin_bit_cast(bf16x8_v, b01), B23 = __builtin_bit_cast(bf16x8_v, b23);
        const uint32_t sp = reinterpret_cast<const uint32_t*>(sl16)[i * 8 + grow];
        const float s_lo = scale_to_f32<SDT>((uint16_t)(sp & 0xffffu));
        const float s_hi = scale_to_f32<SDT>((uint16_t)(sp >> 16));
        const u32x4_v r = wv[i % D];
        // the eight values of row g (t0: low nibbles) or g + 8 (t1: high nibbles) in words j, j + 1
        u32x4_v t0, t1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            t0[j] = r[j] & kNib;
            t1[j] = (r[j] >> 4) & kNib;
        }
        auto opnd = [&](const u32x4_v& t, int j) {
            const u32x4_v a = {bf16x2_b02(t[j]), bf16x2_b13(t[j]), bf16x2_b02(t[j + 1]), bf16x2_b13(t[j + 1])};
            return __builtin_bit_cast(bf16x8_v, a);
        };
        const bf16x8_v A0 = opnd(t0, 0), A1 = opnd(t1, 0), A2 = opnd(t0, 2), A3 = opnd(t1, 2);
        // the window: group i's record is unpacked, its registers take group i + D
        if (i + D < NG) wv[i % D] = ld_stream(qp + (size_t)(i + D) * 64);
        f32x4_v dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B01, c0, 0, 0, 0);
        f32x4_v dh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B01, c0, 0, 0, 0);
        dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A2, B23, dl, 0, 0, 0);
        dh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A3, B23, dh, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            acc_lo[e] = fmaf(s_lo, dl[e], acc_lo[e]);
            acc_hi[e] = fmaf(s_hi, dh[e], acc_hi[e]);
        }
    }

    // 4. the lane's entry is register c % 4 (selected without branches: a branchy select lets the compiler sink
    //    every group's FMAs into the branches and keep all D results live); add the quad (t) and the two chunks
    //    (h, lanes c and c + 8)
    constexpr int kDppRowRor8 = 0x128;  // row_ror:8 (lane c <- lane (c + 8) % 16 of the row)
    float vlo = pick4(acc_lo, (c & 1) != 0, (c & 2) != 0), vhi = pick4(acc_hi, (c & 1) != 0, (c & 2) != 0);
    vlo = dpp_add<kDppXor1>(vlo);
    vhi = dpp_add<kDppXor1>(vhi);
    vlo = dpp_add<kDppXor2>(vlo);
    vhi = dpp_add<kDppXor2>(vhi);
    vlo = dpp_add<kDppRowRor8>(vlo);
    vhi = dpp_add<kDppRowRor8>(vhi);
    if ((c & 11) == 0) {  // c = 0: rows q, q + 8; c = 4: rows 4 + q, 12 + q
        red[w * 16 + grow] = vlo;
        red[w * 16 + grow + 8] = vhi;
    }
    __syncthreads();
    const int row0 = 16 * tile;
    if (out == kOutGLU) {
        if (threadIdx.x < 8) {
            const int gg = threadIdx.x;
            float a = 0.f, b = 0.f;
            for (int ws = 0; ws < S; ws++) {
                a += red[ws * 16 + gg];
                b += red[ws * 16 + gg + 8];
            }
            reinterpret_cast<uint16_t*>(y)[row0 / 2 + gg] = f32_to_bf16(silu_f32(a) * b);
        }
    } else if (threadIdx.x < 16) {
        const int rw = threadIdx.x;
        float v = 0.f;
        for (int ws = 0; ws < S; ws++) v += red[ws * 16 + rw];
        if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[row0 + rw] = f32_to_bf16(v);
        else reinterpret_cast<float*>(y)[row0 + rw] = v;
    }
}


// ---- the streaming variant (long K slices): per wave a K slice of NG groups streamed through a window of D records,
// the slice's activations and scales staged into LDS by DMA in their natural order (no VALU), each B operand gathered
// by two ds_read2_b32 (dwords 32 h + t + {0, 4, 8, 12} of a group: the class (h, t) of words 0 / 1, and + 16 for words
// 2 / 3), the bias -136 x (class sum) by two MFMAs on the same B operands (A = -136). Measured on the C0 shape
// (N = 17408, K = 5120) against the kernel above in the same processes: 8-14 % faster on the boxes whose GEMV runs
// slowest (10.1-11.8 us -> 9.4-10.4 us), within 1 % (slower) on the fastest ones (9.1-9.3 us); longer slices with a
// small window do best (a deeper window leaves each wave a backlog of arrived groups to compute after the stream
// ends), and fewer waves carry less per-wave set-up.
template <int NG>
constexpr int st_xbytes() { return (NG * 256 + 1023) / 1024 * 1024; }
template <int NG>
constexpr int st_wbytes() { return st_xbytes<NG>() + 1024 + 256; }  // x, scales (NG x 32 B <= 1 KB), zeros

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 1 && N <= 5, "vm_wait");
    if constexpr (N == 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
    else if constexpr (N == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else if constexpr (N == 3) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
}

// Quarter tiles. A grid of whole tiles leaves the CUs that receive one more tile than the others (C0: 1088 tiles, 64
// CUs with a fifth) streaming after the rest have finished. The tiles past the last whole round of CUs therefore run
// as four quarter blocks each, at the end of the grid: rows {2a, 2a + 1} (low nibbles) and {2a + 8, 2a + 9} (high
// nibbles) of a tile are W4 lanes 8a .. 8a + 7 of every record, 128 contiguous bytes per 64-k step, and no sum
// crosses blocks. A wave-load covers 8 steps of the wave's K slice: lane L = 8 st + 4 gq + t holds W4 lane
// 4 (2a + gq) + t of step st, i.e. k = 64 st + 16 j + 2 t + {0, 1, 8, 9} of rows 2a + gq and 2a + gq + 8; the
// products run on v_dot2 against the staged activations (dwords 32 st + t + 4 i), chained from -136 x their sum, and
// are scaled per lane. Lanes past the slice (NG not a multiple of 4) load the slice's last step and add nothing.
// Measured (m = 1, K = 5120): N = 17408 9.25 -> 8.83 us, N = 5120 5.48 -> 4.85 us; N = 14336, K = 4096 (two
// quarters on half the CUs) 7.09 -> 6.74 us.
template <int NG, int SDT>
__device__ __forceinline__ void gemv1s_quarter(const uint4* __restrict__ q, const uint16_t* __restrict__ s, int K,
                                               const uint16_t* __restrict__ x, void* __restrict__ y, int out,
                                               int tile, int a, char* lds8, int gb, int ng) {
    constexpr int XB = st_xbytes<NG>(), WB = st_wbytes<NG>();
    constexpr int NL = (2 * NG + 7) / 8;  // wave-loads of 8 steps for the longest slice (ng <= NG groups)
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    const int G = K >> 7, NS = 2 * ng;  // the wave's 64-k steps
    char* wl = lds8 + (size_t)w * WB;
    const unsigned wl32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)wl);
    float* red = reinterpret_cast<float*>(lds8 + (size_t)S * WB);  // [S][16]
    // the slice's activations and scales by DMA, as for a whole tile, then every weight load of the slice
    const char* xs0 = reinterpret_cast<const char*>(x) + (size_t)gb * 256;
#pragma unroll
    for (int r = 0; r < XB / 1024; r++) {
        const int p = 64 * r + L < ng * 16 ? 64 * r + L : ng * 16 - 1;
        qe_tile::dma16(xs0 + 16 * p, wl32 + 1024 * r);
    }
    {
        const int p = L < ng * 2 ? L : ng * 2 - 1;
        qe_tile::dma16(reinterpret_cast<const char*>(s + ((size_t)tile * G + gb) * 16) + 16 * p, wl32 + XB);
    }
    const int st = L >> 3, gq = (L >> 2) & 1, t = L & 3, g = 2 * a + gq;
    const uint4* qp = q + ((size_t)tile * (K >> 6) + 2 * gb) * 32 + 4 * g + t;
    u32x4_v wv[NL];
#pragma unroll
    for (int ld = 0; ld < NL; ld++) {
        const int si = 8 * ld + st < NS ? 8 * ld + st : NS - 1;
        wv[ld] = ld_stream(qp + (size_t)si * 32);
    }
    vm_wait<NL>();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const uint32_t* xl = reinterpret_cast<const uint32_t*>(wl);
    const uint16_t* sl = reinterpret_cast<const uint16_t*>(wl + XB);
    constexpr uint32_t kBias = 0xC308C308u;  // bf16 (-136, -136)
    float acc_lo = 0.f, acc_hi = 0.f;
#pragma unroll
    for (int ld = 0; ld < NL; ld++) {
        const bool valid = 8 * ld + st < NS;
        const int si = valid ? 8 * ld + st : NS - 1;
        const uint32_t* xb = xl + si * 32 + t;
        uint32_t xd[8];  // x pairs (k, k + 1) of word j at 2 j, (k + 8, k + 9) at 2 j + 1
#pragma unroll
        for (int i = 0; i < 8; i++) xd[i] = xb[4 * i];
        float cb = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) cb = dot2_bf16(kBias, xd[i], cb);
        const u32x4_v r = wv[ld];
        float lo = cb, hi = cb;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t t0 = r[j] & kNib, t1 = (r[j] >> 4) & kNib;
            lo = dot2_bf16(bf16x2_b02(t0), xd[2 * j], lo);
            lo = dot2_bf16(bf16x2_b13(t0), xd[2 * j + 1], lo);
            hi = dot2_bf16(bf16x2_b02(t1), xd[2 * j], hi);
            hi = dot2_bf16(bf16x2_b13(t1), xd[2 * j + 1], hi);
        }
        const int grp = si >> 1;
        const float s_lo = scale_to_f32<SDT>(sl[grp * 16 + g]), s_hi = scale_to_f32<SDT>(sl[grp * 16 + g + 8]);
        const float nlo = fmaf(s_lo, lo, acc_lo), nhi = fmaf(s_hi, hi, acc_hi);
        acc_lo = valid ? nlo : acc_lo;
        acc_hi = valid ? nhi : acc_hi;
    }
    // t by DPP, the two steps of a 16-lane row by row_ror 8: lanes 16 r + 4 gq hold (row 2a + gq, row 2a + gq + 8)
    // of steps 2 r, 2 r + 1; the four 16-lane rows and the S slices are added through LDS in a fixed order
    constexpr int kDppRowRor8 = 0x128;
    acc_lo = dpp_add<kDppXor1>(acc_lo);
    acc_hi = dpp_add<kDppXor1>(acc_hi);
    acc_lo = dpp_add<kDppXor2>(acc_lo);
    acc_hi = dpp_add<kDppXor2>(acc_hi);
    acc_lo = dpp_add<kDppRowRor8>(acc_lo);
    acc_hi = dpp_add<kDppRowRor8>(acc_hi);
    if ((L & 11) == 0) {
        red[w * 16 + 4 * (L >> 4) + 2 * gq] = acc_lo;
        red[w * 16 + 4 * (L >> 4) + 2 * gq + 1] = acc_hi;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        const int e = threadIdx.x;  // row 2a + e / 2 (+ 8 for odd e)
        float v = 0.f;
        for (int ws = 0; ws < S; ws++)
            for (int rr = 0; rr < 4; rr++) v += red[ws * 16 + 4 * rr + e];
        if (out == kOutGLU) {
            const float up = __shfl_xor(v, 1, 64);  // lanes e, e ^ 1: gate and up of GLU output 2a + e / 2
            if ((e & 1) == 0) reinterpret_cast<uint16_t*>(y)[8 * tile + 2 * a + (e >> 1)] = f32_to_bf16(silu_f32(v) * up);
        } else {
            const int row = 16 * tile + 2 * a + (e >> 1) + 8 * (e & 1);
            if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[row] = f32_to_bf16(v);
            else reinterpret_cast<float*>(y)[row] = v;
        }
    }
}

// QT: blocks tq.. are quarter blocks (b = blockIdx.x - tq: quarter b % 4 of tile tq + b / 4); the kernel without them
// is a separate instance, whose code is then exactly the whole-tile kernel's (the branch alone, taken by no block,
// cost up to 5 % on some shapes)
template <int NG, int D, int SDT, bool QT, bool EXACT = true>
__global__ void __launch_bounds__(64 * (EXACT ? kMaxWaves : 2 * kMaxWaves)) __attribute__((amdgpu_waves_per_eu(7)))
gemv1s_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s, int N, int K,
              const uint16_t* __restrict__ x, void* __restrict__ y, int out, int tq) {
    static_assert(NG * 32 <= 1024 && D >= 1 && D <= 4 && D < NG, "gemv1s slice");
    constexpr int XB = st_xbytes<NG>(), WB = st_wbytes<NG>();
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    // EXACT: every wave a slice of NG groups; else wave w takes groups w G / S .. (w + 1) G / S - 1 (ng <= NG, > D)
    const int G = K >> 7, gb = EXACT ? w * NG : w * G / S;
    const int ng = EXACT ? NG : (w + 1) * G / S - gb;
    if constexpr (QT) {
        if (__builtin_expect((int)blockIdx.x >= tq, 0)) {
            const int b = blockIdx.x - tq;
            gemv1s_quarter<NG, SDT>(q, s, K, x, y, out, tq + (b >> 2), b & 3, lds8, gb, ng);
            return;
        }
    }
    const int tile = blockIdx.x;
    char* wl = lds8 + (size_t)w * WB;
    const unsigned wl32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)wl);
    float* red = reinterpret_cast<float*>(lds8 + (size_t)S * WB);  // [S][16]

    // 1. DMAs of the slice's activations (1 KB per instruction; lanes past the slice re-read its last 16 bytes into
    //    the padding) and scales (NG x 32 B), then the first D weight records; the zero area for the lanes off the
    //    diagonal. The DMAs are the oldest loads, so once at most D are outstanding they have landed.
    const char* xs0 = reinterpret_cast<const char*>(x) + (size_t)gb * 256;
#pragma unroll
    for (int r = 0; r < XB / 1024; r++) {
        const int p = 64 * r + L < ng * 16 ? 64 * r + L : ng * 16 - 1;
        qe_tile::dma16(xs0 + 16 * p, wl32 + 1024 * r);
    }
    {
        const int p = L < ng * 2 ? L : ng * 2 - 1;
        qe_tile::dma16(reinterpret_cast<const char*>(s + ((size_t)tile * G + gb) * 16) + 16 * p, wl32 + XB);
    }
    const uint4* qp = q + ((size_t)tile * (K >> 6) + 2 * gb) * 32 + L;
    u32x4_v wv[D];
#pragma unroll
    for (int i = 0; i < D; i++) wv[i] = ld_stream(qp + (size_t)i * 64);
    reinterpret_cast<uint32_t*>(wl + XB + 1024)[L] = 0u;
    vm_wait<D>();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 2. per group: B operands (diagonal lanes: class (h = qb / 2, t = c % 4); others: zeros), the bias MFMAs, the 4
    //    weight MFMAs, acc += s * D (the lane's register c % 4 is the useful one, as in gemv1_kernel)
    const int qb = L >> 4, c = L & 15;
    const bool diag = (c >> 2) == qb;
    const uint32_t* bb = diag ? reinterpret_cast<const uint32_t*>(wl) + 32 * (qb >> 1) + (c & 3)
                              : reinterpret_cast<const uint32_t*>(wl + XB + 1024);
    const int bstep = diag ? 64 : 0;
    const int grow = 4 * ((c >> 2) & 1) + qb;
    const uint16_t* sl = reinterpret_cast<const uint16_t*>(wl + XB);
    constexpr uint32_t kBias = 0xC308C308u;  // bf16 (-136, -136)
    const bf16x8_v a_bias = __builtin_bit_cast(bf16x8_v, u32x4_v{kBias, kBias, kBias, kBias});
    f32x4_v acc_lo = {0.f, 0.f, 0.f, 0.f}, acc_hi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NG; i++) {
        // the first D groups unconditionally (ng > D): with a branch before group 0 the compiler sank the D record
        // loads below vm_wait<D> into it, and the wait then no longer covered the activation and scale DMAs
        if (!EXACT && i >= D && i >= ng) break;
        const uint32_t* b = bb + i * bstep;
        const u32x4_v b01 = {b[0], b[4], b[8], b[12]}, b23 = {b[16], b[20], b[24], b[28]};
        const bf16x8_v B01 = __builtin_bit_cast(bf16x8_v, b01), B23 = __builtin_bit_cast(bf16x8_v, b23);
        const float s_lo = scale_to_f32<SDT>(sl[i * 16 + grow]);
        const float s_hi = scale_to_f32<SDT>(sl[i * 16 + grow + 8]);
        const u32x4_v r = wv[i % D];
        u32x4_v t0, t1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            t0[j] = r[j] & kNib;
            t1[j] = (r[j] >> 4) & kNib;
        }
        auto opnd = [&](const u32x4_v& t, int j) {
            const u32x4_v a = {bf16x2_b02(t[j]), bf16x2_b13(t[j]), bf16x2_b02(t[j + 1]), bf16x2_b13(t[j + 1])};
            return __builtin_bit_cast(bf16x8_v, a);
        };
        const bf16x8_v A0 = opnd(t0, 0), A1 = opnd(t1, 0), A2 = opnd(t0, 2), A3 = opnd(t1, 2);
        if (i + D < ng) wv[i % D] = ld_stream(qp + (size_t)(i + D) * 64);
        f32x4_v cb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_bias, B01, f32x4_v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        cb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_bias, B23, cb, 0, 0, 0);
        f32x4_v dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B01, cb, 0, 0, 0);
        f32x4_v dh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B01, cb, 0, 0, 0);
        dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A2, B23, dl, 0, 0, 0);
        dh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A3, B23, dh, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            acc_lo[e] = fmaf(s_lo, dl[e], acc_lo[e]);
            acc_hi[e] = fmaf(s_hi, dh[e], acc_hi[e]);
        }
    }

    // 3. the lane's register, the quad and chunk halves by DPP, the slices through LDS in order (as gemv1_kernel)
    constexpr int kDppRowRor8 = 0x128;
    float vlo = pick4(acc_lo, (c & 1) != 0, (c & 2) != 0), vhi = pick4(acc_hi, (c & 1) != 0, (c & 2) != 0);
    vlo = dpp_add<kDppXor1>(vlo);
    vhi = dpp_add<kDppXor1>(vhi);
    vlo = dpp_add<kDppXor2>(vlo);
    vhi = dpp_add<kDppXor2>(vhi);
    vlo = dpp_add<kDppRowRor8>(vlo);
    vhi = dpp_add<kDppRowRor8>(vhi);
    if ((c & 11) == 0) {
        red[w * 16 + grow] = vlo;
        red[w * 16 + grow + 8] = vhi;
    }
    __syncthreads();
    const int row0 = 16 * tile;
    if (out == kOutGLU) {
        if (threadIdx.x < 8) {
            const int gg = threadIdx.x;
            float a = 0.f, b = 0.f;
            for (int ws = 0; ws < S; ws++) {
                a += red[ws * 16 + gg];
                b += red[ws * 16 + gg + 8];
            }
            reinterpret_cast<uint16_t*>(y)[row0 / 2 + gg] = f32_to_bf16(silu_f32(a) * b);
        }
    } else if (threadIdx.x < 16) {
        const int rw = threadIdx.x;
        float v = 0.f;
        for (int ws = 0; ws < S; ws++) v += red[ws * 16 + rw];
        if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[row0 + rw] = f32_to_bf16(v);
        else reinterpret_cast<float*>(y)[row0 + rw] = v;
    }
}

// slices of the streaming variant: the fewest waves per tile (S in {2, 4, 8}, S dividing K / 128, NG = K / 128 / S
// in {5, 8, 10, 16, 20}) whose grid still has >= 8 waves per CU; 0 when none fits (the caller takes gemv1_kernel)
int stream_groups(int n, int k) {
    const int tiles = n / 16, G = k / 128;
    for (int S : {2, 4, 8}) {
        if (G % S) continue;
        const int ng = G / S;
        if (ng != 5 && ng != 8 && ng != 10 && ng != 16 && ng != 20) continue;
        if ((long)tiles * S >= 8L * qe_num_cus()) return ng;
    }
    return 0;
}
}  // namespace qe_gemv1

// m = 1 on the matrix cores (x 16-byte aligned): the streaming kernel where stream_groups finds a slicing; its
// run-time slices (8 or 16 per tile, quarter blocks past the last whole round of CUs or for every tile of a grid
// filling at most half the CUs) where K / 128 has no even slicing or few tiles meet a long K; else gemv1_kernel when
// K / 128 splits evenly into slices of 10, 8, 5, 4 or 2 groups; returns false otherwise (the caller takes the VALU
// GEMV)
bool gemv1_w4(const W4& w, const uint16_t* x, void* y, int out, hipStream_t st) {
    using namespace qe_gemv1;
    if (((uintptr_t)x & 15) != 0) return false;
    const int sng = stream_groups(w.n, w.k);
    if (sng > 0) {
        const int S = w.k / 128 / sng;
        // the tiles past the last whole round of CUs as quarter blocks at the end of the grid
        const int tiles = w.n / 16, ncu = qe_num_cus(), rem = tiles > ncu ? tiles % ncu : 0;
        const int tq = tiles - rem;
        const dim3 grid((unsigned)(tq + 4 * rem)), block(64 * S);
#define QE_GEMV1S(NG_, SDT_)                                                                                  \
    do {                                                                                                      \
        const size_t lb = (size_t)S * st_wbytes<NG_>() + (size_t)S * 64;                                      \
        if (rem) gemv1s_kernel<NG_, 3, SDT_, true><<<grid, block, lb, st>>>(w.q, w.s, w.n, w.k, x, y, out, tq); \
        else gemv1s_kernel<NG_, 3, SDT_, false><<<grid, block, lb, st>>>(w.q, w.s, w.n, w.k, x, y, out, tq);   \
    } while (0)
#define QE_GEMV1S_NG(SDT_)                          \
    do {                                            \
        if (sng == 20) QE_GEMV1S(20, SDT_);         \
        else if (sng == 16) QE_GEMV1S(16, SDT_);    \
        else if (sng == 10) QE_GEMV1S(10, SDT_);    \
        else if (sng == 8) QE_GEMV1S(8, SDT_);      \
        else QE_GEMV1S(5, SDT_);                    \
    } while (0)
        if (w.sdt == kScaleF16) QE_GEMV1S_NG(kScaleF16);
        else QE_GEMV1S_NG(kScaleBF16);
#undef QE_GEMV1S_NG
#undef QE_GEMV1S
        HIP_CHECK(hipGetLastError());
        return true;
    }
    const int ng = decode_groups(w.n, w.k);
    // even K too where the tiles fill at most half the CUs and K >= 6144: the quarter blocks below (N = 1024, K = 8192
    // 4.24 -> 3.54 us, N = 1536, K = 6144 4.33 -> 3.96 us; at K = 4096 / 5120 the whole-tile kernel stays ahead)
    const int G0 = w.k / 128;
    if (ng == 0 || (2 * (w.n / 16) <= qe_num_cus() && G0 >= 48 && (G0 + 2 * kMaxWaves - 1) / (2 * kMaxWaves) <= 20)) {
        // no even slicing (K = 17408: 136 groups): the streaming kernel with 8 slices of floor / ceil (G / 8) groups,
        // each longer than the load window, or 16 where the grid holds at most one tile per CU (long K: one 8-wave
        // block per CU keeps too few bytes in flight) or where 8 slices would be too long for quarter blocks. Past one
        // tile per CU, 16 slices (100 KB of LDS per block) leave one block per CU, and the quarter blocks wait for the
        // whole tiles; with 8 (51 KB) they run beside them. Measured N = 5120, K = 17408: the VALU GEMV's uneven
        // slices 41.5 us; 16 slices 13.25 us, 8 slices 10.66 us (K = 13824: 9.94 -> 8.84 us); at N = 2048 .. 4096 16
        // slices stay ahead (7.5 vs 8.4 us). Where the tiles fill at most half the CUs, every tile runs as four quarter
        // blocks of 8 slices (16 where 8 would exceed 20 groups), so that every CU streams: N = 2048, K = 17408 7.50 ->
        // 6.59 us, N = 1024 7.23 -> 4.61 us (at one tile per CU, N = 4096, quarters lose: 7.5 -> 9.8 us)
        const int G = w.k / 128, tiles = w.n / 16, ncu = qe_num_cus();
        const bool aq = 2 * tiles <= ncu && (G + 2 * kMaxWaves - 1) / (2 * kMaxWaves) <= 20;
        const bool s16 = (G + kMaxWaves - 1) / kMaxWaves > 20 || (!aq && tiles <= ncu);
        const int S = s16 && G / (2 * kMaxWaves) > 3 ? 2 * kMaxWaves : kMaxWaves;
        const int ngmax = (G + S - 1) / S;
        if (G / S <= 3 || ngmax > 32) return false;
        // quarter blocks for the tiles past the last whole round of CUs, or for all of them (slices of up to 20
        // groups: the quarter path keeps all of a slice's wave-loads in flight)
        const int rem = aq ? tiles : tiles > ncu && ngmax <= 20 ? tiles % ncu : 0, tq = tiles - rem;
        const dim3 grid((unsigned)(tq + 4 * rem)), block(64 * S);
#define QE_GEMV1U(NG_, QT_, SDT_)                                                                             \
    gemv1s_kernel<NG_, 3, SDT_, QT_, false><<<grid, block, (size_t)S * st_wbytes<NG_>() + (size_t)S * 64, st>>>( \
        w.q, w.s, w.n, w.k, x, y, out, tq)
#define QE_GEMV1U_S(SDT_)                                  \
    do {                                                   \
        if (ngmax > 20) QE_GEMV1U(32, false, SDT_);        \
        else if (ngmax > 8 && rem) QE_GEMV1U(20, true, SDT_); \
        else if (ngmax > 8) QE_GEMV1U(20, false, SDT_);    \
        else if (rem) QE_GEMV1U(8, true, SDT_);            \
        else QE_GEMV1U(8, false, SDT_);                    \
    } while (0)
        if (w.sdt == kScaleF16) QE_GEMV1U_S(kScaleF16);
        else QE_GEMV1U_S(kScaleBF16);
#undef QE_GEMV1U_S
#undef QE_GEMV1U
        HIP_CHECK(hipGetLastError());
        return true;
    }
    const int S = w.k / 128 / ng;
    const dim3 grid((unsigned)(w.n / 16)), block(64 * S);
    // all of a slice's records in flight for slices of up to 5 groups, else a window of 3
#define QE_GEMV1(NG_, SDT_)                                                                                   \
    gemv1_kernel<NG_, (NG_ <= 5 ? NG_ : 3), SDT_><<<grid, block, ((size_t)S * wave_dwords<NG_>() + (size_t)S * 16) * 4, \
                                                     st>>>(w.q, w.s, w.n, w.k, x, y, out)
#define QE_GEMV1_NG(SDT_)                        \
    do {                                         \
        if (ng == 10) QE_GEMV1(10, SDT_);        \
        else if (ng == 8) QE_GEMV1(8, SDT_);     \
        else if (ng == 5) QE_GEMV1(5, SDT_);     \
        else if (ng == 4) QE_GEMV1(4, SDT_);     \
        else QE_GEMV1(2, SDT_);                  \
    } while (0)
    if (w.sdt == kScaleF16) QE_GEMV1_NG(kScaleF16);
    else QE_GEMV1_NG(kScaleBF16);
#undef QE_GEMV1_NG
#undef QE_GEMV1
    HIP_CHECK(hipGetLastError());
    return true;
}

// ---- W8 per-channel records, m = 1, on the matrix cores. A W8 record (lane (g, t) of a 32-k slab) holds in dword d
// the bytes (g, k) (g, k + 1) (g + 8, k) (g + 8, k + 1), k = 8 d + 2 t: one row's 8 values of the record are exactly one
// v_mfma_f32_16x16x32_bf16 A operand (u = w + 128 as floats, whose high halves are the exact bf16 pair), and the
// activations they meet are dwords 16 s + t + {0, 4, 8, 12} of the slab pair, the class-major B operand of
// gemv1s_kernel with 32-k slabs in place of 64-k chunks. A wave-load is 64 lanes x 16 B = two slabs (lane L = 16 q + c:
// W8 lane L % 32 of slab L / 32), B is block diagonal as there, and with one scale per row no per-group scaling is
// needed: three MFMA chains (rows g, rows g + 8, and -128 x the class sums) run over the whole slice, and the row
// scale multiplies the slice sums once. Per 1 KB wave-load 28 VALU for the conversion (xor, 4 byte conversions and
// 2 permutes per dword) and 3 MFMAs.
namespace qe_gemv1 {
template <int NWL>
constexpr int w8_xbytes() { return (NWL * 128 + 1023) / 1024 * 1024; }  // the slice's activations (64 k per wave-load)

template <int NWL, int D, int SDT>
__global__ void __launch_bounds__(64 * kMaxWaves) __attribute__((amdgpu_waves_per_eu(7)))
gemv1s_w8c_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s, int K, const uint16_t* __restrict__ x,
                  void* __restrict__ y, int out) {
    static_assert(NWL >= D && D >= 1 && D <= 4 && w8_xbytes<NWL>() <= 8192, "gemv1s_w8c slice");
    constexpr int XB = w8_xbytes<NWL>(), WB = XB + 256;
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    const int tile = blockIdx.x, kb = w * NWL;  // kb: the slice's first 64-k unit
    char* wl = lds8 + (size_t)w * WB;
    const unsigned wl32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)wl);
    float* red = reinterpret_cast<float*>(lds8 + (size_t)S * WB);  // [S][16]

    // 1. the row scale of lane L % 16 (used after the reduction: loaded first, so the block's end does not wait a
    //    memory latency for it), the slice's activations by DMA (lanes past the slice re-read its last 16 bytes into
    //    the padding), the first D wave-loads of records, the zero block for the lanes off the diagonal
    const uint16_t sraw = s[16 * tile + (L & 15)];
    const char* xs0 = reinterpret_cast<const char*>(x) + (size_t)kb * 128;
#pragma unroll
    for (int r = 0; r < XB / 1024; r++) {
        const int p = 64 * r + L < NWL * 8 ? 64 * r + L : NWL * 8 - 1;
        qe_tile::dma16(xs0 + 16 * p, wl32 + 1024 * r);
    }
    const uint4* qp = q + ((size_t)tile * (K >> 5) + 2 * kb) * 32 + L;
    u32x4_v wv[D];
#pragma unroll
    for (int i = 0; i < D; i++) wv[i] = ld_stream(qp + (size_t)i * 64);
    reinterpret_cast<uint32_t*>(wl + XB)[L] = 0u;
    vm_wait<D>();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 2. per wave-load: B (diagonal lanes: class (slab qb / 2, t = c % 4); others: zeros), the rows' A operands, the
    //    three MFMA chains
    const int qb = L >> 4, c = L & 15;
    const bool diag = (c >> 2) == qb;
    const uint32_t* bb = diag ? reinterpret_cast<const uint32_t*>(wl) + 16 * (qb >> 1) + (c & 3)
                              : reinterpret_cast<const uint32_t*>(wl + XB);
    const int bstep = diag ? 32 : 0;
    constexpr uint32_t kBias = 0xC300C300u;  // bf16 (-128, -128)
    const bf16x8_v a_bias = __builtin_bit_cast(bf16x8_v, u32x4_v{kBias, kBias, kBias, kBias});
    auto pair = [](uint32_t u, int b0) {  // bf16 pair of bytes b0, b0 + 1 of u (exact: u <= 255)
        const float f0 = static_cast<float>((u >> (8 * b0)) & 0xFFu), f1 = static_cast<float>((u >> (8 * b0 + 8)) & 0xFFu);
        return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
    };
    f32x4_v dl = {0.f, 0.f, 0.f, 0.f}, dh = {0.f, 0.f, 0.f, 0.f}, cb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NWL; i++) {
        const uint32_t* b = bb + i * bstep;
        const u32x4_v bv = {b[0], b[4], b[8], b[12]};
        const bf16x8_v B = __builtin_bit_cast(bf16x8_v, bv);
        const u32x4_v r = wv[i % D];
        u32x4_v alo, ahi;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t u = r[d] ^ 0x80808080u;
            alo[d] = pair(u, 0);
            ahi[d] = pair(u, 2);
        }
        if (i + D < NWL) wv[i % D] = ld_stream(qp + (size_t)(i + D) * 64);
        cb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_bias, B, cb, 0, 0, 0);
        dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, alo), B, dl, 0, 0, 0);
        dh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, ahi), B, dh, 0, 0, 0);
    }

    // 3. the lane's register (c % 4) with the bias, the quad and slab halves by DPP, the slices through LDS in order,
    //    then the row scale
    constexpr int kDppRowRor8 = 0x128;
    const bool b1 = (c & 1) != 0, b2 = (c & 2) != 0;
    float vlo = pick4(dl, b1, b2) + pick4(cb, b1, b2), vhi = pick4(dh, b1, b2) + pick4(cb, b1, b2);
    vlo = dpp_add<kDppXor1>(vlo);
    vhi = dpp_add<kDppXor1>(vhi);
    vlo = dpp_add<kDppXor2>(vlo);
    vhi = dpp_add<kDppXor2>(vhi);
    vlo = dpp_add<kDppRowRor8>(vlo);
    vhi = dpp_add<kDppRowRor8>(vhi);
    const int grow = 4 * ((c >> 2) & 1) + qb;
    if ((c & 11) == 0) {
        red[w * 16 + grow] = vlo;
        red[w * 16 + grow + 8] = vhi;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const int rw = threadIdx.x, row = 16 * tile + rw;
        float v = 0.f;
        for (int ws = 0; ws < S; ws++) v += red[ws * 16 + rw];
        v *= scale_to_f32<SDT>(sraw);
        if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[row] = f32_to_bf16(v);
        else reinterpret_cast<float*>(y)[row] = v;
    }
}

// K slices: the most waves per tile (S in {8, 4, 2}) with 4..40 wave-loads each and >= 16 waves per CU; 0: none.
// Measured (one process, window 3): S = 8 / 4 / 2 at N = 8192, K = 2048 (C3) 4.85 / 5.16 / 6.38 us; N = 17408,
// K = 5120 16.00 / 16.38 / 16.34 us; N = 16384, K = 4096 12.50 / 13.06 / 12.62 us (the VALU GEMV before: 5.2-5.3 us
// at C3, window 2 or 4 no better). One tile per CU (N = 4096, K = 5120, 8 waves per CU): 5.67 us against 5.53 for
// the skinny kernel, so those grids keep it
int w8c_slices(int n, int k) {
    const int tiles = n / 16, KU = k / 64;
    for (int S : {8, 4, 2}) {
        if (KU % S) continue;
        const int nwl = KU / S;
        if (nwl != 4 && nwl != 8 && nwl != 10 && nwl != 16 && nwl != 20 && nwl != 32 && nwl != 40) continue;
        if ((long)tiles * S >= 16L * qe_num_cus()) return S;
    }
    return 0;
}
}  // namespace qe_gemv1

// m = 1 on W8 per-channel records (x 16-byte aligned, out fp32 or bf16); false when no slicing fits (the caller takes
// its other kernels)
bool gemv1_w8c(const W8& w, const uint16_t* x, void* y, int out, hipStream_t st) {
    using namespace qe_gemv1;
    if (!w.per_channel || w.q8 || out == kOutGLU || ((uintptr_t)x & 15) != 0) return false;
    const int S = w8c_slices(w.n, w.k);
    if (S == 0) return false;
    const int nwl = w.k / 64 / S;
    const dim3 grid((unsigned)(w.n / 16)), block(64 * S);
    // all records in flight at 4 wave-loads per wave (C3: 4.80 -> 4.65 us), else a window of 3 (K = 5120: equal)
#define QE_W8C(NWL_, SDT_)                                                                                       \
    gemv1s_w8c_kernel<NWL_, (NWL_ == 4 ? 4 : 3), SDT_><<<grid, block, (size_t)S * (w8_xbytes<NWL_>() + 256) + (size_t)S * 64, st>>>( \
        w.q, w.s, w.k, x, y, out)
#define QE_W8C_N(SDT_)                          \
    do {                                        \
        if (nwl == 4) QE_W8C(4, SDT_);          \
        else if (nwl == 8) QE_W8C(8, SDT_);     \
        else if (nwl == 10) QE_W8C(10, SDT_);   \
        else if (nwl == 16) QE_W8C(16, SDT_);   \
        else if (nwl == 20) QE_W8C(20, SDT_);   \
        else if (nwl == 32) QE_W8C(32, SDT_);   \
        else QE_W8C(40, SDT_);                  \
    } while (0)
    if (w.sdt == kScaleF16) QE_W8C_N(kScaleF16);
    else QE_W8C_N(kScaleBF16);
#undef QE_W8C_N
#undef QE_W8C
    HIP_CHECK(hipGetLastError());
    return true;
}

// ---- the m = 1 GEMV's HBM read floor: the same blocks, waves and record loads, no arithmetic
namespace qe_gemv1 {
template <int NG>
__global__ void __launch_bounds__(64 * kMaxWaves) read_probe_kernel(const uint4* __restrict__ q, int K,
                                                                    uint32_t* __restrict__ sink) {
    const int w = threadIdx.x >> 6, L = threadIdx.x & 63;
    const uint4* qp = q + ((size_t)blockIdx.x * (K >> 6) + 2 * w * NG) * 32 + L;
    u32x4_v v[NG];
#pragma unroll
    for (int i = 0; i < NG; i++) v[i] = ld_stream(qp + (size_t)i * 64);
    u32x4_v a = v[0];
#pragma unroll
    for (int i = 1; i < NG; i++) a ^= v[i];
    const uint32_t r = a[0] ^ a[1] ^ a[2] ^ a[3];
    if (r == 0x9E3779B9u) sink[blockIdx.x] = r;
}
}  // namespace qe_gemv1

void read_probe_w4(const void* q, int n, int k, uint32_t* sink, hipStream_t st) {
    using namespace qe_gemv1;
    int ng = decode_groups(n, k);
    if (ng == 0) ng = (k / 128) % 4 == 0 && k / 128 / 4 <= kMaxWaves ? 4 : 0;
    CHECK(ng > 0, "read_probe: no even K slicing for k = %d", k);
    const dim3 grid((unsigned)(n / 16)), block(64 * (k / 128 / ng));
    const uint4* qq = reinterpret_cast<const uint4*>(q);
    if (ng == 10) read_probe_kernel<10><<<grid, block, 0, st>>>(qq, k, sink);
    else if (ng == 8) read_probe_kernel<8><<<grid, block, 0, st>>>(qq, k, sink);
    else if (ng == 5) read_probe_kernel<5><<<grid, block, 0, st>>>(qq, k, sink);
    else if (ng == 4) read_probe_kernel<4><<<grid, block, 0, st>>>(qq, k, sink);
    else read_probe_kernel<2><<<grid, block, 0, st>>>(qq, k, sink);
    HIP_CHECK(hipGetLastError());
}

// ---- the shader clock: one lane counts clock64() (shader clock cycles) over `ticks` of wall_clock64() (a constant
// rate), then stores both spans; the loop ends once the wall clock has advanced `ticks`, whatever the shader clock
namespace qe_gemv1 {
__global__ void __launch_bounds__(64) clock_probe_kernel(unsigned long long* __restrict__ out, long long ticks) {
    if (threadIdx.x != 0) return;
    const long long r0 = wall_clock64(), c0 = clock64();
    long long r = r0;
    while (r - r0 < ticks) r = wall_clock64();
    const long long c1 = clock64();
    out[0] = (unsigned long long)(r - r0);
    out[1] = (unsigned long long)(c1 - c0);
}
}  // namespace qe_gemv1

float clock_probe_mhz(hipStream_t st) {
    int dev = 0, rate_khz = 0;
    HIP_CHECK(hipGetDevice(&dev));
    HIP_CHECK(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev));
    CHECK(rate_khz > 0, "clock_probe: wall clock rate %d kHz", rate_khz);
    unsigned long long* d = nullptr;
    unsigned long long h[2] = {0, 0};
    HIP_CHECK(hipMalloc(&d, sizeof(h)));
    const long long ticks = (long long)rate_khz / 20;  // 50 us of wall clock
    qe_gemv1::clock_probe_kernel<<<1, 64, 0, st>>>(d, ticks);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, st));
    HIP_CHECK(hipStreamSynchronize(st));
    HIP_CHECK(hipFree(d));
    return h[0] ? (float)((double)h[1] / (double)h[0] * rate_khz / 1000.0) : 0.f;
}
