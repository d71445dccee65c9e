// Prefill GEMM with the reference's fp16-accumulate numerics (reference gemm_h_kernel + x_to_h_kernel,
// src/kernels/gemm.cu:236-461, launched by gemm_cfg, gemm.cu:4047-4070): C[t][n] = sum_k X[t][k] W[n][k] where
//   * the activations are scaled per token so that |x| <= 16 and rounded to fp16: xs[t] = amax_k |x[t][k]| / 16
//     (1 for a zero row), xh[t][k] = fp16_rn(fp32(x[t][k] * fp32(1 / xs[t]))) (x_to_h_kernel, gemm.cu:262-289);
//   * the weights enter as the exact integers u - 8 in fp16;
//   * each 64-k chunk's products are summed (the reference: m16n8k16 MMAs into an fp16 accumulator; here
//     v_mfma_f32_32x32x16_f16 into fp32, the chunk partial rounded once to fp16), scaled by the chunk's 128-k
//     group scale into fp32 accumulators, and the token scale multiplies the result in the epilogue.
// So the results follow the reference's rounding points except inside a chunk, where this build rounds once:
// they agree to about one fp16 ulp of a chunk partial (times its scale), not bit for bit.
//
//   block: 512 threads = 8 waves in 2 (tokens) x 4 (weight rows), tile BM = 128 tokens x BN = 256 rows x BK = 64.
//   The MFMAs take X as A and W as B, so a lane of the 32 x 32 result holds one weight row (column l % 32) and
//   16 tokens: one group scale per lane and tile in the per-chunk flush. Two partial sets (the chunk being
//   summed, 4 x 16 registers) and the fp32 accumulators (4 x 16) per wave.
//   LDS, the pipeline and the tile order are those of the bf16 prefill GEMM: X by LDS DMA (global_load_lds) one
//   step ahead, raw W4 records by DMA two steps ahead, the next step's W tile unpacked to fp16 integers between
//   the MFMA rows of the current step (1 AND, 2 v_perm with the 0x64 exponent byte and 2 v_pk_add_f16 per
//   (row half, word)); the group scales by DMA into a small double buffer.
#include "mfma_tile.hpp"

#include <mutex>
#include <type_traits>
#include <vector>

namespace {

using namespace qe_tile;

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_v;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_v;

constexpr int BM = 128, BN = 256, BK = 64, NTH = 512, WMT = 2, WNT = 2;
constexpr int kStage = (BM + BN) * BK * 2;  // X [BM][64] and W [BN][64] fp16
constexpr int kRaw = BN * 32, kSc = BN * 2;
constexpr int kLds = 2 * kStage + 2 * kRaw + 2 * kSc;
constexpr float kXTarget = 16.f;
enum Out : int { kOutF32 = 0, kOutBF16 = 1, kOutGLU = 2 };

// one block per token (reference x_to_h_kernel, gemm.cu:262-289): the row's amax, xs = amax / 16 (1 for a zero
// row), xh = fp16_rn(x * (1 / xs)) with the product rounded to fp32 first. VEC: 16-byte aligned rows, 8 values per
// load and store
template <bool VEC>
__global__ void __launch_bounds__(256) x_to_h_kernel(const uint16_t* __restrict__ x, int ldx, int K,
                                                     uint16_t* __restrict__ xh, float* __restrict__ xs) {
    const int t = blockIdx.x;
    const uint16_t* r = x + (size_t)t * ldx;
    constexpr int V = VEC ? 8 : 2;
    auto load = [&](int k, float (&f)[V]) {
        if constexpr (VEC) {
            const u32x4_v a = *reinterpret_cast<const u32x4_v*>(r + k);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t wa = a[i];
                f[2 * i] = __builtin_bit_cast(float, wa << 16);
                f[2 * i + 1] = __builtin_bit_cast(float, wa & 0xFFFF0000u);
            }
        } else {
            f[0] = bf16_to_f32(r[k]);
            f[1] = bf16_to_f32(r[k + 1]);
        }
    };
    float mx = 0.f;
    for (int k = threadIdx.x * V; k < K; k += blockDim.x * V) {
        float f[V];
        load(k, f);
#pragma unroll
        for (int i = 0; i < V; i++) mx = fmaxf(mx, fabsf(f[i]));
    }
    __shared__ float red[4];
    for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = mx > 0.f ? mx / kXTarget : 1.f;
    const float inv = 1.f / sc;
    if (threadIdx.x == 0) xs[t] = sc;
    uint16_t* o = xh + (size_t)t * K;
    for (int k = threadIdx.x * V; k < K; k += blockDim.x * V) {
        float f[V];
        load(k, f);
        uint32_t hv[V / 2];
#pragma unroll
        for (int i = 0; i < V / 2; i++) {
            // the products are fp32 values first (med3 of one value keeps the compiler from fusing the multiply into
            // the fp16 conversion): the reference rounds twice
            const float a = f[2 * i] * inv, b = f[2 * i + 1] * inv;
            const f16x2_v h = {(_Float16)__builtin_amdgcn_fmed3f(a, a, a), (_Float16)__builtin_amdgcn_fmed3f(b, b, b)};
            hv[i] = __builtin_bit_cast(uint32_t, h);
        }
        if constexpr (VEC) *reinterpret_cast<u32x4_v*>(o + k) = u32x4_v{hv[0], hv[1], hv[2], hv[3]};
        else *reinterpret_cast<uint32_t*>(o + k) = hv[0];
    }
}

// fp16 pairs 1024 + u (bytes b, 0x64) -> u - 8, exact
__device__ __forceinline__ uint32_t f16_int_pair(uint32_t u, uint32_t sel) {
    const f16x2_v v = __builtin_bit_cast(f16x2_v, __builtin_amdgcn_perm(0x64646464u, u, sel)) -
                      f16x2_v{(_Float16)1032.f, (_Float16)1032.f};
    return __builtin_bit_cast(uint32_t, v);
}

template <int SDT, int OUT>
__global__ void __launch_bounds__(NTH) gemm_h_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s,
                                                     int N, int K, const uint16_t* __restrict__ xh,
                                                     const float* __restrict__ xs, int T, void* __restrict__ c,
                                                     int ldc, int nbn, int ntiles) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned lds32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);
    // XCD-aware order (block b on XCD b % 8 sweeps a contiguous band of the n-major tile sequence)
    const int per = (ntiles + 7) >> 3, b = blockIdx.x;
    const int tile = (b & 7) * per + (b >> 3);
    if (tile >= ntiles) return;
    const int n0 = (tile % nbn) * BN, t0 = (tile / nbn) * BM;
    const int G = K >> 7, KT = K / BK;
    const int ntile_last = (N >> 4) - 1;

    // X: 1 KB DMA = 8 rows of 128 B per wave instruction, chunks placed by the swizzle; rows past T re-read T - 1
    auto dma_x = [&](int kt, unsigned xt) {
#pragma unroll
        for (int i = 0; i < BM / 64; i++) {
            const int r0 = (wave * (BM / 64) + i) * 8, row = r0 + (lane >> 3);
            const int ch = (lane & 7) ^ swz_f(row);
            const int tok = t0 + row < T ? t0 + row : T - 1;
            dma16(xh + (size_t)tok * K + kt * BK + ch * 8, lds32 + xt + r0 * 128);
        }
    };
    // raw W4 records of one 64-k step: a 1 KB wave load covers two 16-row tiles, lane i record (tile 2 w + (i / 8) % 2,
    // g = i % 8, t = i / 16), so that the unpack reads below hit distinct banks
    auto dma_w4 = [&](int kt, unsigned raw) {
        if (wave < BN / 32) {
            const int tl = min((n0 >> 4) + 2 * wave + ((lane >> 3) & 1), ntile_last);
            dma16(q + ((size_t)tl * (K >> 6) + kt) * 32 + 4 * (lane & 7) + (lane >> 4), lds32 + raw + wave * 1024);
        }
    };
    auto dma_sc = [&](int grp, unsigned sc) {  // [BN / 16 tiles][16] scales of group grp
        if (wave < BN / 128) {
            const int tl = min((n0 >> 4) + 8 * wave + (lane >> 3), ntile_last);
            dma4(s + ((size_t)tl * G + grp) * 16 + 2 * (lane & 7), lds32 + sc + wave * 256);
        }
    };
    // unpack job of this thread: word jj (16 k) of the 4 records (g = jg, t = 0..3) of tile jtr -> rows jg and
    // jg + 8, chunks 2 jj (k 16 jj .. + 8) and 2 jj + 1
    const int jj = tid & 3, jg = (tid >> 2) & 7, jtr = tid >> 5;
    static_assert(BN * 2 == NTH, "one unpack job per thread");

    constexpr unsigned kRawOff = 2 * kStage, kScOff = kRawOff + 2 * kRaw;
    const int wm = wave >> 2, wn = wave & 3;
    f32x16_v acc[WMT][WNT], part[WMT][WNT];
#pragma unroll
    for (int a = 0; a < WMT; a++)
#pragma unroll
        for (int bb = 0; bb < WNT; bb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][bb][r] = 0.f;
    int lane_off[BK / 16];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) lane_off[ks] = swz(lane & 31, 2 * ks + (lane >> 5));

    // unit (h, t) of the unpack: word t, row half h -> the fp16 integer pairs at k0 (lo) and k0 + 8 (hi),
    // k0 = 16 jj + 2 t; each half's two 16-byte stores after its last word
    uint32_t wd[4], lo[2][4], hi[2][4];
    auto unit = [&](char* wtile, int h, int t) {
        const uint32_t u = (h ? wd[t] >> 4 : wd[t]) & nib_mask();  // bytes: k0, k0 + 8, k0 + 1, k0 + 9
        lo[h][t] = f16_int_pair(u, 0x04020400u);
        hi[h][t] = f16_int_pair(u, 0x04030401u);
        if (t == 3) {
            const int row = jtr * 16 + jg + 8 * h;
            *reinterpret_cast<u32x4_v*>(wtile + swz(row, 2 * jj)) = u32x4_v{lo[h][0], lo[h][1], lo[h][2], lo[h][3]};
            *reinterpret_cast<u32x4_v*>(wtile + swz(row, 2 * jj + 1)) = u32x4_v{hi[h][0], hi[h][1], hi[h][2], hi[h][3]};
        }
    };
    auto read_words = [&](const char* rawb) {
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(rawb + (jtr >> 1) * 1024) + (8 * (jtr & 1) + jg) * 4 + jj;
#pragma unroll
        for (int t = 0; t < 4; t++) wd[t] = rw[64 * t];
    };

    // prologue: X and raw W of step 0, raw W of step 1, scales of group 0; step 0's W tile
    dma_x(0, 0);
    dma_w4(0, kRawOff);
    if (KT > 1) dma_w4(1, kRawOff + kRaw);
    dma_sc(0, kScOff);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    read_words(lds + kRawOff);
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int t = 0; t < 4; t++) unit(lds + BM * BK * 2, h, t);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // step kt: DMA X (kt + 1), raw W (kt + 2) and the scales of its group; the MFMAs of step kt into the partials
    // with the unpack of step kt + 1 between the MFMA rows (order pinned); then the flush of the chunk:
    // acc += fp16_rn(part) * s
    auto kstep = [&](int kt, auto more) {
        constexpr bool MORE = decltype(more)::value;
        char* wnext = lds + ((kt + 1) & 1) * kStage + BM * BK * 2;
        if (MORE) dma_x(kt + 1, ((kt + 1) & 1) * kStage);
        if (kt + 2 < KT) {
            dma_w4(kt + 2, kRawOff + (kt & 1) * kRaw);
            if (((kt + 2) & 1) == 0) dma_sc((kt + 2) >> 1, kScOff + (((kt + 2) >> 1) & 1) * kSc);
        }
        const char* xt = lds + (kt & 1) * kStage;
        const char* wt = xt + BM * BK * 2;
        f16x8_v af[2][WMT], bfr[2][WNT];
        auto read_frags = [&](int ks, int buf) {
#pragma unroll
            for (int a = 0; a < WMT; a++)
                af[buf][a] = *reinterpret_cast<const f16x8_v*>(xt + lane_off[ks] + (wm * 32 * WMT + a * 32) * 128);
#pragma unroll
            for (int bb = 0; bb < WNT; bb++)
                bfr[buf][bb] = *reinterpret_cast<const f16x8_v*>(wt + lane_off[ks] + (wn * 32 * WNT + bb * 32) * 128);
        };
        read_frags(0, 0);
        if constexpr (MORE) read_words(lds + kRawOff + ((kt + 1) & 1) * kRaw);
        // this lane's weight row in each column tile: its group scale
        const uint16_t* scb = reinterpret_cast<const uint16_t*>(lds + kScOff + ((kt >> 1) & 1) * kSc);
        float scl[WNT];
#pragma unroll
        for (int bb = 0; bb < WNT; bb++) scl[bb] = scale_to_f32<SDT>(scb[wn * 32 * WNT + bb * 32 + (lane & 31)]);
        __builtin_amdgcn_sched_barrier(0);
        int slot = 0;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            if (ks + 1 < BK / 16) read_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
            for (int a = 0; a < WMT; a++) {
#pragma unroll
                for (int bb = 0; bb < WNT; bb++) {
                    const f32x16_v cin = ks == 0 ? f32x16_v{} : part[a][bb];
                    part[a][bb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks & 1][a], bfr[ks & 1][bb], cin, 0, 0, 0);
                }
                if constexpr (MORE) unit(wnext, slot >> 2, slot & 3);  // 8 rows per step: one unit after each
                slot++;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int a = 0; a < WMT; a++)
#pragma unroll
            for (int bb = 0; bb < WNT; bb++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[a][bb][r] = fmaf((float)(_Float16)part[a][bb][r], scl[bb], acc[a][bb][r]);
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    static_assert((BK / 16) * WMT == 8, "one unpack unit per MFMA row");
    for (int kt = 0; kt + 1 < KT; kt++) kstep(kt, std::true_type{});
    kstep(KT - 1, std::false_type{});

    // epilogue: lane = weight row n (column l % 32 of each tile), registers r = tokens 8 (r / 4) + 4 (l / 32) + r % 4
#pragma unroll
    for (int a = 0; a < WMT; a++) {
        float xsv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int tok = t0 + wm * 32 * WMT + a * 32 + c_row(lane, r);
            xsv[r] = xs[tok < T ? tok : T - 1];
        }
#pragma unroll
        for (int bb = 0; bb < WNT; bb++) {
            const int n = n0 + wn * 32 * WNT + bb * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int tok = t0 + wm * 32 * WMT + a * 32 + c_row(lane, r);
                const float v = acc[a][bb][r] * xsv[r];
                if constexpr (OUT == kOutGLU) {
                    // gate row g (n % 16 < 8) and up row g + 8 of a 16-row tile: lanes l and l + 8 of one DPP row
                    const float up = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                                          0x128, 0xF, 0xF, false));
                    if ((n & 15) < 8 && n < N && tok < T)
                        reinterpret_cast<uint16_t*>(c)[(size_t)tok * ldc + (n >> 4) * 8 + (n & 7)] = f32_to_bf16(silu_f32(v) * up);
                } else if (n < N && tok < T) {
                    if constexpr (OUT == kOutBF16) reinterpret_cast<uint16_t*>(c)[(size_t)tok * ldc + n] = f32_to_bf16(v);
                    else reinterpret_cast<float*>(c)[(size_t)tok * ldc + n] = v;
                }
            }
        }
    }
}

// the pre-pass buffer (xh [t][k] fp16, xs [t] fp32) of (device, stream): a capture that needs more than an eager call
// or gemm_h_reserve on its stream sized aborts with a message
void* h_ws(size_t bytes, hipStream_t st) {
    void* p = stream_ws(kWsH, bytes, st);
    CHECK(p != nullptr,
          "gemm_w4h: the pre-pass buffer (%zu bytes) must be sized by an eager call or qe_gemm_h_reserve(_s) on this "
          "stream before capture",
          bytes);
    return p;
}

size_t h_ws_bytes(int k, int t) { return ((size_t)t * k * 2 + 255) / 256 * 256 + (size_t)t * 4; }

}  // namespace

void gemm_h_reserve(int k, int t, hipStream_t st) {
    if (k > 0 && t > 0) stream_ws_reserve(kWsH, h_ws_bytes(k, t), st);
}

// out: 0 fp32, 1 bf16, 2 GLU (bf16 activation [t][n / 2])
void gemm_w4h(const W4& w, const uint16_t* x, int ldx, void* c, int ldc, int t, bool out_bf16, hipStream_t st) {
    CHECK(w.n > 0 && w.n % 16 == 0 && w.k >= 128 && w.k % 128 == 0, "gemm_w4h: n = %d, k = %d", w.n, w.k);
    CHECK(t > 0, "gemm_w4h: t = %d", t);
    CHECK(ldx >= w.k, "gemm_w4h: ldx = %d < k", ldx);
    CHECK(ldc >= (w.glu ? w.n / 2 : w.n), "gemm_w4h: ldc = %d", ldc);
    char* ws = static_cast<char*>(h_ws(h_ws_bytes(w.k, t), st));
    uint16_t* xh = reinterpret_cast<uint16_t*>(ws);
    float* xs = reinterpret_cast<float*>(ws + ((size_t)t * w.k * 2 + 255) / 256 * 256);
    if (((uintptr_t)x & 15) == 0 && ldx % 8 == 0) x_to_h_kernel<true><<<dim3((unsigned)t), dim3(256), 0, st>>>(x, ldx, w.k, xh, xs);
    else x_to_h_kernel<false><<<dim3((unsigned)t), dim3(256), 0, st>>>(x, ldx, w.k, xh, xs);
    HIP_CHECK(hipGetLastError());
    const int nbn = (w.n + BN - 1) / BN, nbt = (t + BM - 1) / BM, ntiles = nbn * nbt;
    const unsigned blocks = (unsigned)(8 * ((ntiles + 7) / 8));
    const int out = w.glu ? kOutGLU : out_bf16 ? kOutBF16 : kOutF32;
#define QE_GH(SDT_, OUT_) \
    gemm_h_kernel<SDT_, OUT_><<<dim3(blocks), dim3(NTH), kLds, st>>>(w.q, w.s, w.n, w.k, xh, xs, t, c, ldc, nbn, ntiles)
    if (w.sdt == kScaleF16) {
        if (out == kOutGLU) QE_GH(kScaleF16, kOutGLU);
        else if (out == kOutBF16) QE_GH(kScaleF16, kOutBF16);
        else QE_GH(kScaleF16, kOutF32);
    } else {
        if (out == kOutGLU) QE_GH(kScaleBF16, kOutGLU);
        else if (out == kOutBF16) QE_GH(kScaleBF16, kOutBF16);
        else QE_GH(kScaleBF16, kOutF32);
    }
#undef QE_GH
    HIP_CHECK(hipGetLastError());
}
