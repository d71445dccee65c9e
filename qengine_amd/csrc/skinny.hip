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
//   * The bias 136 (u = w + 8 over the 128 of the magic) is removed by one more MFMA per k step with A = -136:
//     C = sum (128 + u) x - 136 sum x = sum (u - 8) x, all products exact in fp32. The group scale is applied
//     once per group: acc += s * C.
//   * K slices per block are those of the m = 1 matrix-core kernel (decode_groups; gemv_slicing's uneven slices
//     where no even slicing fits) and the fixed-order LDS reduction makes the result deterministic; an activation
//     row's result does not depend on the other rows (MFMA columns are independent, the slicing depends on (n, k)
//     only).
#include "gemv_impl.hpp"

namespace qe_skinny {
using namespace qe_gemv;

// weight groups in flight per wave (with the activations of each group in the window for MT >= 8). Measured on the
// BASELINE shapes with 5-group slices: 3 for every MT but 8, where 2 keeps the kernel at 6 waves per SIMD (deeper
// windows cost more in occupancy than they gain in latency)
template <int MT, int NG>
constexpr int skinny_d() {
    constexpr int d = MT == 8 ? 2 : 3;
    return NG > 0 && NG < d ? NG : d;
}

// UPX (MT <= 4 with even slices): every group's activations are loaded before the weights and staged in LDS
// while the weights are in flight. Else the activations of a group are loaded with its weights (x_j before w_j,
// so waiting for x_j never waits for w_j) and staged one group ahead into a double buffer. Weight records stream
// through a window of D groups.
template <int MT, int NG>
constexpr bool skinny_upx() {
    return MT <= 4 && NG > 0;
}
// staged activation rows (one row = one activation row's 64 dwords of a group) are kXStride dwords apart: the B
// operand reads of 8 consecutive lanes (8 rows, same offset in the row) then hit 8 disjoint groups of 4 banks; with
// 64 they all hit the same banks (an 8-way conflict per read at MT >= 8)
constexpr int kXStride = 68;
template <int MT, int NG>
constexpr int skinny_wsz() {  // dwords of LDS per wave: xl [UPX ? NGM : 2][MT][kXStride], scales [NGM][16] half
    constexpr int NGM = NG > 0 ? NG : kGenericNG;
    return (skinny_upx<MT, NG>() ? NGM : 2) * MT * kXStride + NGM * 8;
}

template <int MT, int SDT, int NG, int D>
__global__ void __launch_bounds__(64 * (NG > 0 ? kMaxWaves : kMaxWavesGeneric))
__attribute__((amdgpu_waves_per_eu(MT <= 4 ? 6 : 1))) skinny_kernel(
    const uint4* __restrict__ q, const uint16_t* __restrict__ s, int N, int K, const uint16_t* __restrict__ x,
    int ldx, void* __restrict__ y, int ldy, int m, int out, int sdt) {
    constexpr int NGM = NG > 0 ? NG : kGenericNG;
    constexpr bool UPX = skinny_upx<MT, NG>();
    constexpr int WSZ = skinny_wsz<MT, NG>();
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    const int tile = blockIdx.x, G = K >> 7;
    const int gb = NG > 0 ? w * NG : w * G / S;
    const int ng = NG > 0 ? NG : (w + 1) * G / S - gb;
    uint32_t* xl = lds + (size_t)w * WSZ;
    uint16_t* sl16 = reinterpret_cast<uint16_t*>(xl + (WSZ - NGM * 8));
    float* red = reinterpret_cast<float*>(lds + (size_t)S * WSZ);  // [S][16 tok][16 rows]

    const int qg = L >> 4, i = L & 15;  // operand lane group, row / column within the tile
    const int g = i & 7, sh = 4 * (i >> 3);

    // Activation rows tok >= m (up to MT) load row m - 1 instead: no load sits under a branch, and those MFMA
    // columns are never stored (columns are independent).
    const size_t xs = (size_t)(ldx >> 1);  // dwords per activation row
    // !UPX: a group's activations are MT rows x 16 pieces of 16 bytes; lane L loads piece L % 16 of row xrow_of(e)
    // and stages its 4 dwords at their class-major positions (MT < 4: lanes of rows past MT load a duplicate and
    // stage nothing). A staging store covers 4 rows of 8 consecutive dwords (+32): MT >= 8 takes rows 2 apart
    // (2 x kXStride = 8 banks mod 64, so the 4 rows' spans are disjoint); rows 1 apart would overlap by 4 banks.
    constexpr int XP = MT >= 4 ? MT / 4 : 1;
    auto xrow_of = [&](int e) { return MT >= 8 ? (e & 1) + 2 * (L >> 4) + 8 * (e >> 1) : (L >> 4) + 4 * e; };
    const u32x4_v* xq[XP];
#pragma unroll
    for (int e = 0; e < XP; e++) {
        const int tp = xrow_of(e);
        xq[e] = reinterpret_cast<const u32x4_v*>(reinterpret_cast<const uint32_t*>(x) + (size_t)(tp < m ? tp : m - 1) * xs +
                                                 (size_t)gb * 64) + (L & 15);
    }
    auto ldxg = [&](u32x4_v* dst, int ii) {
#pragma unroll
        for (int e = 0; e < XP; e++) dst[e] = xq[e][ii * 16];
    };
    auto stxg = [&](const u32x4_v* src, int buf) {
#pragma unroll
        for (int e = 0; e < XP; e++)
            if (MT >= 4 || (L >> 4) < MT) {
#pragma unroll
                for (int c = 0; c < 4; c++)
                    xl[(buf * MT + xrow_of(e)) * kXStride + x_slot<kFmtW4>(4 * (L & 15) + c)] = src[e][c];
            }
    };

    // 1. loads in consumption order: the slice's scales (one dword per lane); UPX: every group's activations, then
    //    the first D groups of weight records; else (x_j, w_j) pairs for the first D groups
    {
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(s + ((size_t)tile * G + gb) * 16);
        if (L < ng * 8) reinterpret_cast<uint32_t*>(sl16)[L] = sp[L];
    }
    u32x4_v xr[UPX ? 1 : D][XP];  // activation register slots (per-group staging)
    const uint4* qp = q + ((size_t)tile * (K >> 6) + 2 * gb) * 32 + 4 * g + qg;
    u32x4_v wv[D][2];
    auto ldw = [&](int slot, int ii) {
        wv[slot][0] = ld_stream(qp + (size_t)ii * 64);
        wv[slot][1] = ld_stream(qp + (size_t)ii * 64 + 32);
    };
    if constexpr (UPX) {
        // lane L loads dwords [8 L, 8 L + 8) of each row's slice (16-byte pieces; x and ldx are 16-byte aligned)
        // and stores dword 8 (L % 8) + e of group L / 8 at its class-major position
        constexpr int XL = NGM * 8;
        u32x4_v xv[MT][2];
        const uint32_t* xs0 = reinterpret_cast<const uint32_t*>(x) + (size_t)gb * 64;
        const int lc = L < XL ? L : XL - 1;  // lanes past the slice reload its last piece (not staged)
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
            const u32x4_v* src = reinterpret_cast<const u32x4_v*>(xs0 + (tok < m ? tok : m - 1) * xs) + 2 * lc;
            xv[tok][0] = src[0];
            xv[tok][1] = src[1];
        }
#pragma unroll
        for (int ii = 0; ii < D; ii++)
            if (ii < ng) ldw(ii, ii);
        if (L < XL) {
#pragma unroll
            for (int tok = 0; tok < MT; tok++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    xl[((L >> 3) * MT + tok) * kXStride + x_slot<kFmtW4>(8 * (L & 7) + e)] = xv[tok][e >> 2][e & 3];
        }
    } else {
#pragma unroll
        for (int ii = 0; ii < D; ii++) {
            if (ii < ng) {
                ldxg(xr[ii], ii);
                ldw(ii, ii);
            }
        }
        stxg(xr[0], 0);  // group 0 -> buffer 0
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const bf16x8_v a_bias = __builtin_bit_cast(bf16x8_v, u32x4_v{0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u});
    f32x4_v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ii = 0; ii < NGM; ii++) {
        if (NG == 0 && ii >= ng) break;
        const int xrow = UPX ? ii * MT : (ii & 1) * MT;  // first staged row of this group
        if constexpr (!UPX) {
            // stage the next group's activations into the other buffer (read two groups ago, LDS operations of
            // a wave complete in order)
            if (ii + 1 < ng) stxg(xr[(ii + 1) % D], (ii + 1) & 1);
        }
        const u32x4_v r0 = wv[ii % D][0], r1 = wv[ii % D][1];
        // refill the window: group ii + D goes where group ii was
        if (ii + D < ng) {
            if constexpr (!UPX) ldxg(xr[ii % D], ii + D);
            ldw(ii % D, ii + D);
        }
        f32x4_v c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mm = 0; mm < 4; mm++) {
            const int j0 = 2 * (mm & 1);
            const u32x4_v rec = mm < 2 ? r0 : r1;
            u32x4_v b = {0u, 0u, 0u, 0u};
            if (MT == 16 || i < MT)
                b = *reinterpret_cast<const u32x4_v*>(&xl[(xrow + (i < MT ? i : 0)) * kXStride + (4 * (mm >> 1) + qg) * 8 + 2 * j0]);
            const uint32_t w0 = rec[j0], w1 = rec[j0 + 1];
            const uint32_t t0 = (w0 >> sh) & kNib, t1 = (w1 >> sh) & kNib;  // row i: k0, k0 + 8, k0 + 1, k0 + 9
            const u32x4_v a = {bf16x2_b02(t0), bf16x2_b13(t0), bf16x2_b02(t1), bf16x2_b13(t1)};
            const bf16x8_v bb = __builtin_bit_cast(bf16x8_v, b);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, a), bb, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_bias, bb, c, 0, 0, 0);
        }
        // rows 4 qg .. 4 qg + 3 of the group's scales
        const uint2 sv = *reinterpret_cast<const uint2*>(&sl16[ii * 16 + 4 * qg]);
        acc[0] = fmaf(scale_rt<SDT>((uint16_t)(sv.x & 0xffffu), sdt), c[0], acc[0]);
        acc[1] = fmaf(scale_rt<SDT>((uint16_t)(sv.x >> 16), sdt), c[1], acc[1]);
        acc[2] = fmaf(scale_rt<SDT>((uint16_t)(sv.y & 0xffffu), sdt), c[2], acc[2]);
        acc[3] = fmaf(scale_rt<SDT>((uint16_t)(sv.y >> 16), sdt), c[3], acc[3]);
        if constexpr (!UPX) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }

    // 2. slices through LDS in a fixed order: red[w][tok][row], lane (qg, i) holds rows 4 qg .. + 3 of column i
    *reinterpret_cast<f32x4_v*>(&red[(w * 16 + i) * 16 + 4 * qg]) = acc;
    __syncthreads();
    auto rsum = [&](int tok, int rr) {
        float v = 0.f;
        for (int ws = 0; ws < S; ws++) v += red[(ws * 16 + tok) * 16 + rr];
        return v;
    };
    const int row0 = 16 * tile;
    if (out == kOutGLU) {
        for (int idx = threadIdx.x; idx < m * 8; idx += blockDim.x) {
            const int tok = idx >> 3, gg = idx & 7;
            reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 / 2 + gg] =
                f32_to_bf16(silu_f32(rsum(tok, gg)) * rsum(tok, gg + 8));
        }
    } else {
        for (int idx = threadIdx.x; idx < m * 16; idx += blockDim.x) {
            const int tok = idx >> 4, rr = idx & 15;
            const float v = rsum(tok, rr);
            if (out == kOutBF16) reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 + rr] = f32_to_bf16(v);
            else reinterpret_cast<float*>(y)[(size_t)tok * ldy + row0 + rr] = v;
        }
    }
}

template <int SDT>
void launch(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy, int m,
            int out, int sdt, hipStream_t st) {
    // even slices of the matrix-core decode kernels where they divide K, else the generic uneven slices
    const int dg = decode_groups(n, k);
    const Slicing sc = dg > 0 ? Slicing{dg, (k >> 7) / dg} : gemv_slicing(n, k);
    const int mt = m == 1 ? 1 : m == 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16;
    const dim3 grid((unsigned)(n / 16)), block(64 * sc.S);
#define QE_SK_K(MT_, NG_)                                                                                         \
    skinny_kernel<MT_, SDT, NG_, skinny_d<MT_, NG_>()><<<grid, block, (size_t)sc.S * (skinny_wsz<MT_, NG_>() + 256) * 4, st>>>( \
        q, s, n, k, x, ldx, y, ldy, m, out, sdt)
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
    else QE_SK_NG(16);
#undef QE_SK_NG
#undef QE_SK_K
    HIP_CHECK(hipGetLastError());
}

}  // namespace qe_skinny

void skinny_w4_mfma(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, int out, hipStream_t st) {
    if (w.sdt == kScaleF16) qe_skinny::launch<kScaleF16>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
    else qe_skinny::launch<kScaleBF16>(w.q, w.s, w.n, w.k, x, ldx, y, ldy, m, out, w.sdt, st);
}
