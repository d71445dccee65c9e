// Decode GEMV and skinny GEMM (m = 1..16 rows) on the W4 / W8 fragment layouts, for gfx950.
//
// Design (memory-bound: the packed weights are streamed once from HBM):
//   * one wave64 per (16-row tile, K slice); a wave-load is 64 lanes x 16 B = 1 KB, contiguous in the layout
//     (W4: one 128-k group of the tile, W8: half a group). Every weight load of the slice is issued up front
//     (<= 8 groups, non-temporal), so ~16 KB per wave and ~20 waves per CU are in flight.
//   * the activation slice is staged once per wave in LDS, permuted so that each lane reads the 8 dwords
//     (bf16 pairs) its nibbles need with two ds_read_b128; per lane class the sum of those x values is
//     staged beside them.
//   * nibbles become bf16 by OR-ing them into the mantissa of 128.0 (bf16 0x4300 -> 128 + u exactly), and
//     v_dot2_f32_bf16 accumulates (128 + u) * x in fp32; the bias is removed per group with the staged x sum:
//     sum_k (u - 8) x = sum_k (128 + u) x - 136 sum_k x. INT8 bytes (XOR 0x80 -> u = w + 128) take
//     v_cvt_f32_ubyte + v_cvt_pk_bf16 (exact) and the bias 128.
//   * the group partial is scaled once per group: acc += s * (a - bias * X) (fp32).
//   * lanes of one row are reduced with a fixed xor butterfly; K slices of a tile are reduced by the last
//     arriving wave (device-scope counter) in slice order, so results are deterministic and independent of m
//     and of the arrival order ("batch == alone", as the reference's skinny / GEMV pair, skinny.cu:1-14).
#include "qe_api.hpp"

#include <algorithm>
#include <mutex>

namespace {

typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));

constexpr int kSliceGroups = 8;   // max 128-k groups per K slice
constexpr size_t kPartFloats = (size_t)16 << 20;  // split-K partials workspace (64 MB)
constexpr int kMaxTiles = 1 << 16;
constexpr int kMaxDev = 16;

struct GemvWs {
    float* part = nullptr;
    unsigned* ctr = nullptr;
};
GemvWs g_ws[kMaxDev];
std::mutex g_ws_mu;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a), __builtin_bit_cast(bf16x2_v, b), c,
                                           false);
}
__device__ __forceinline__ u32x4_v ld_stream(const uint4* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p));
}

enum Fmt : int { kFmtW4 = 0, kFmtW8G = 1, kFmtW8C = 2 };
enum Out : int { kOutF32 = 0, kOutBF16 = 1, kOutGLU = 2 };

// lane layout shared by both formats: g = (L >> 2) & 7 (rows g and g + 8 of the tile), t = L & 3, h = L >> 5
// dword `dw` (0..63) of a 128-k group of x -> (lane class, slot)
template <int FMT>
__device__ __forceinline__ void x_class(int dw, int& cls, int& slot) {
    if constexpr (FMT == kFmtW4) {  // dw = 32 h + 8 j + 4 b + t: pair at k0 = 64 h + 16 j + 2 t (+ 8 b)
        cls = 4 * (dw >> 5) + (dw & 3);
        slot = 2 * ((dw >> 3) & 3) + ((dw >> 2) & 1);
    } else {  // dw = 16 (2 e + h) + 4 d + t: W8 wave-load e, dword d of the 16-byte record
        cls = 4 * ((dw >> 4) & 1) + (dw & 3);
        slot = 4 * (dw >> 5) + ((dw >> 2) & 3);
    }
}

template <int MT, int FMT, int SDT, int OUT>
__global__ void __launch_bounds__(64) gemv_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s,
                                                  int N, int K, const uint16_t* __restrict__ x, int ldx,
                                                  void* __restrict__ y, int ldy, int m, int S,
                                                  float* __restrict__ part, unsigned* __restrict__ ctr) {
    constexpr int NG = kSliceGroups;
    constexpr int LPG = FMT == kFmtW4 ? 1 : 2;  // wave-loads per group
    __shared__ __attribute__((aligned(16))) uint32_t xl[MT][NG][64];
    __shared__ float xsum[MT][NG][8];
    __shared__ unsigned s_last;

    const int L = threadIdx.x;
    const int tile = blockIdx.x / S, sl = blockIdx.x - tile * S;
    const int G = K >> 7;
    const int gb = sl * G / S, ge = (sl + 1) * G / S, ng = ge - gb;
    const int g = (L >> 2) & 7, t = L & 3, h = L >> 5;

    // 1. weights of the slice, all in flight at once
    u32x4_v wv[NG][LPG];
    {
        const uint4* qp = FMT == kFmtW4 ? q + ((size_t)tile * (K >> 6) + 2 * gb) * 32 + L
                                        : q + ((size_t)tile * (K >> 5) + 4 * gb) * 32 + L;
#pragma unroll
        for (int i = 0; i < NG; i++)
#pragma unroll
            for (int e = 0; e < LPG; e++)
                if (i < ng) wv[i][e] = ld_stream(qp + (size_t)(i * LPG + e) * 64);
    }
    // scales of rows g / g + 8
    float sc_lo[NG], sc_hi[NG];
    if constexpr (FMT == kFmtW8C) {
        const float a = scale_to_f32<SDT>(s[16 * tile + g]), b = scale_to_f32<SDT>(s[16 * tile + g + 8]);
#pragma unroll
        for (int i = 0; i < NG; i++) { sc_lo[i] = a; sc_hi[i] = b; }
    } else {
        const uint16_t* sp = s + ((size_t)tile * G + gb) * 16;
#pragma unroll
        for (int i = 0; i < NG; i++)
            if (i < ng) {
                sc_lo[i] = scale_to_f32<SDT>(sp[i * 16 + g]);
                sc_hi[i] = scale_to_f32<SDT>(sp[i * 16 + g + 8]);
            }
    }

    // 2. stage the x slice: lane L takes dword L of every group
    {
        int cls, slot;
        x_class<FMT>(L, cls, slot);
        const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
#pragma unroll
            for (int i = 0; i < NG; i++) {
                if (i < ng) {
                    const uint32_t v = tok < m ? xw[((size_t)tok * ldx + (size_t)(gb + i) * 128) / 2 + L] : 0u;
                    xl[tok][i][cls * 8 + slot] = v;
                    float sm = bf16_to_f32((uint16_t)v) + bf16_to_f32((uint16_t)(v >> 16));
                    if constexpr (FMT == kFmtW4) {
                        sm += __shfl_xor(sm, 4);
                        sm += __shfl_xor(sm, 8);
                        sm += __shfl_xor(sm, 16);
                        if ((L & 28) == 0) xsum[tok][i][cls] = sm;
                    } else {
                        sm += __shfl_xor(sm, 4);
                        sm += __shfl_xor(sm, 8);
                        sm += __shfl_xor(sm, 32);
                        if ((L & 44) == 0) xsum[tok][i][cls] = sm;
                    }
                }
            }
        }
    }
    __syncthreads();

    // 3. dot products
    const int cls = 4 * h + t;
    float acc_lo[MT], acc_hi[MT];
#pragma unroll
    for (int tok = 0; tok < MT; tok++) acc_lo[tok] = acc_hi[tok] = 0.f;
#pragma unroll
    for (int i = 0; i < NG; i++) {
        if (i >= ng) break;
        float a_lo[MT], a_hi[MT];
#pragma unroll
        for (int tok = 0; tok < MT; tok++) a_lo[tok] = a_hi[tok] = 0.f;
        if constexpr (FMT == kFmtW4) {
            const u32x4_v w = wv[i][0];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t wd = w[j];
                const uint32_t p0 = (wd & 0x000F000Fu) | 0x43004300u;          // row g,     k0, k0 + 1
                const uint32_t p1 = ((wd >> 4) & 0x000F000Fu) | 0x43004300u;   // row g + 8, k0, k0 + 1
                const uint32_t p2 = ((wd >> 8) & 0x000F000Fu) | 0x43004300u;   // row g,     k0 + 8, k0 + 9
                const uint32_t p3 = ((wd >> 12) & 0x000F000Fu) | 0x43004300u;  // row g + 8, k0 + 8, k0 + 9
#pragma unroll
                for (int tok = 0; tok < MT; tok++) {
                    const uint32_t xa = xl[tok][i][cls * 8 + 2 * j], xb = xl[tok][i][cls * 8 + 2 * j + 1];
                    a_lo[tok] = dot2_bf16(p0, xa, a_lo[tok]);
                    a_lo[tok] = dot2_bf16(p2, xb, a_lo[tok]);
                    a_hi[tok] = dot2_bf16(p1, xa, a_hi[tok]);
                    a_hi[tok] = dot2_bf16(p3, xb, a_hi[tok]);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const u32x4_v w = wv[i][e];
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t u = w[d] ^ 0x80808080u;  // bytes: (g, k) (g, k+1) (g+8, k) (g+8, k+1)
                    const uint32_t plo = pack_bf16x2((float)(u & 0xffu), (float)((u >> 8) & 0xffu));
                    const uint32_t phi = pack_bf16x2((float)((u >> 16) & 0xffu), (float)(u >> 24));
#pragma unroll
                    for (int tok = 0; tok < MT; tok++) {
                        const uint32_t xa = xl[tok][i][cls * 8 + 4 * e + d];
                        a_lo[tok] = dot2_bf16(plo, xa, a_lo[tok]);
                        a_hi[tok] = dot2_bf16(phi, xa, a_hi[tok]);
                    }
                }
            }
        }
        constexpr float bias = FMT == kFmtW4 ? 136.f : 128.f;
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
            const float X = xsum[tok][i][cls];
            acc_lo[tok] = fmaf(sc_lo[i], fmaf(-bias, X, a_lo[tok]), acc_lo[tok]);
            acc_hi[tok] = fmaf(sc_hi[i], fmaf(-bias, X, a_hi[tok]), acc_hi[tok]);
        }
    }

    // 4. rows g / g + 8: sum over t and h (fixed butterfly, identical in every lane of the row)
#pragma unroll
    for (int tok = 0; tok < MT; tok++) {
        float a = acc_lo[tok], b = acc_hi[tok];
        a += __shfl_xor(a, 1);
        b += __shfl_xor(b, 1);
        a += __shfl_xor(a, 2);
        b += __shfl_xor(b, 2);
        a += __shfl_xor(a, 32);
        b += __shfl_xor(b, 32);
        acc_lo[tok] = a;
        acc_hi[tok] = b;
    }
    const int row0 = 16 * tile;
    if (S == 1) {
        if ((L & 35) != 0) return;  // lanes 4 g (t = 0, h = 0) store
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
            if (tok >= m) break;
            if constexpr (OUT == kOutGLU) {
                reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 / 2 + g] =
                    f32_to_bf16(silu_f32(acc_lo[tok]) * acc_hi[tok]);
            } else if constexpr (OUT == kOutBF16) {
                uint16_t* yb = reinterpret_cast<uint16_t*>(y) + (size_t)tok * ldy + row0;
                yb[g] = f32_to_bf16(acc_lo[tok]);
                yb[g + 8] = f32_to_bf16(acc_hi[tok]);
            } else {
                float* yf = reinterpret_cast<float*>(y) + (size_t)tok * ldy + row0;
                yf[g] = acc_lo[tok];
                yf[g + 8] = acc_hi[tok];
            }
        }
        return;
    }
    // 5. split K: partial of slice sl -> part[sl][tok][n]; the last arriving slice sums all in slice order.
    // Cross-XCD visibility without an L2 writeback / invalidate: the partials are agent-scope atomic stores
    // (write-through) completed (s_waitcnt) before the counter update, and the last wave reads them with
    // agent-scope atomic loads.
    if ((L & 35) == 0) {
#pragma unroll
        for (int tok = 0; tok < MT; tok++) {
            if (tok >= m) break;
            float* pp = part + ((size_t)sl * m + tok) * N + row0;
            __hip_atomic_store(pp + g, acc_lo[tok], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + g + 8, acc_hi[tok], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (L == 0) s_last = __hip_atomic_fetch_add(ctr + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_last != (unsigned)(S - 1)) return;
    auto ld_part = [&](size_t i) { return __hip_atomic_load(part + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    if constexpr (OUT == kOutGLU) {
        for (int idx = L; idx < m * 8; idx += 64) {
            const int tok = idx >> 3, gg = idx & 7;
            float gate = 0.f, up = 0.f;
            for (int sj = 0; sj < S; sj++) {
                const size_t base = ((size_t)sj * m + tok) * N + row0;
                gate += ld_part(base + gg);
                up += ld_part(base + gg + 8);
            }
            reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 / 2 + gg] = f32_to_bf16(silu_f32(gate) * up);
        }
    } else {
        for (int idx = L; idx < m * 16; idx += 64) {
            const int tok = idx >> 4, rr = idx & 15;
            float v = 0.f;
            for (int sj = 0; sj < S; sj++) v += ld_part(((size_t)sj * m + tok) * N + row0 + rr);
            if constexpr (OUT == kOutBF16) reinterpret_cast<uint16_t*>(y)[(size_t)tok * ldy + row0 + rr] = f32_to_bf16(v);
            else reinterpret_cast<float*>(y)[(size_t)tok * ldy + row0 + rr] = v;
        }
    }
    if (L == 0) __hip_atomic_store(ctr + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
}

int g_cus = 0;

// K slices per tile: about 16 one-wave blocks per CU in total, at most 8 groups per slice. Depends on (n, k)
// only, so every row count of a matrix reduces in the same order.
int gemv_splits(int n, int k) {
    const int tiles = n / 16, G = k / 128;
    const int target = 16 * qe_num_cus();
    int S = (target + tiles - 1) / tiles;
    S = std::max(S, (G + kSliceGroups - 1) / kSliceGroups);
    return std::min(S, G);
}

template <int FMT, int SDT, int OUT>
void launch_gemv(const uint4* q, const uint16_t* s, int n, int k, const uint16_t* x, int ldx, void* y, int ldy,
                 int m, int S, float* part, unsigned* ctr, hipStream_t st) {
    const dim3 grid((unsigned)(n / 16 * S)), block(64);
#define QE_GEMV_CASE(MT_)                                                                                   \
    gemv_kernel<MT_, FMT, SDT, OUT><<<grid, block, 0, st>>>(q, s, n, k, x, ldx, y, ldy, m, S, part, ctr)
    if (m == 1) QE_GEMV_CASE(1);
    else if (m == 2) QE_GEMV_CASE(2);
    else if (m <= 4) QE_GEMV_CASE(4);
    else if (m <= 8) QE_GEMV_CASE(8);
    else QE_GEMV_CASE(16);
#undef QE_GEMV_CASE
    HIP_CHECK(hipGetLastError());
}

template <int FMT>
void gemv_dispatch(const uint4* q, const uint16_t* s, int sdt, bool glu, int n, int k, const uint16_t* x, int ldx,
                   void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    int dev;
    HIP_CHECK(hipGetDevice(&dev));
    CHECK(dev >= 0 && dev < kMaxDev && g_ws[dev].ctr, "gemv workspace not initialised (qe_gemv_workspace_init)");
    const int S = gemv_splits(n, k);
    CHECK(n / 16 <= kMaxTiles && (S == 1 || (size_t)S * m * n <= kPartFloats), "gemv workspace too small (n=%d k=%d)",
          n, k);
    float* part = g_ws[dev].part;
    unsigned* ctr = g_ws[dev].ctr;
#define QE_GEMV_OUT(SDT_)                                                                                     \
    do {                                                                                                      \
        if (glu) launch_gemv<FMT, SDT_, kOutGLU>(q, s, n, k, x, ldx, y, ldy, m, S, part, ctr, st);            \
        else if (out_bf16) launch_gemv<FMT, SDT_, kOutBF16>(q, s, n, k, x, ldx, y, ldy, m, S, part, ctr, st); \
        else launch_gemv<FMT, SDT_, kOutF32>(q, s, n, k, x, ldx, y, ldy, m, S, part, ctr, st);                \
    } while (0)
    if (sdt == kScaleF16) QE_GEMV_OUT(kScaleF16);
    else QE_GEMV_OUT(kScaleBF16);
#undef QE_GEMV_OUT
}

}  // namespace

int qe_num_cus() {
    if (g_cus == 0) {
        int dev, cus = 0;
        HIP_CHECK(hipGetDevice(&dev));
        HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_cus = cus > 0 ? cus : 256;
    }
    return g_cus;
}

void gemv_workspace_init() {
    int dev;
    HIP_CHECK(hipGetDevice(&dev));
    CHECK(dev >= 0 && dev < kMaxDev, "device %d", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (g_ws[dev].ctr) return;
    HIP_CHECK(hipMalloc(&g_ws[dev].part, kPartFloats * sizeof(float)));
    HIP_CHECK(hipMalloc(&g_ws[dev].ctr, kMaxTiles * sizeof(unsigned)));
    HIP_CHECK(hipMemset(g_ws[dev].ctr, 0, kMaxTiles * sizeof(unsigned)));
    HIP_CHECK(hipDeviceSynchronize());
    qe_num_cus();
}

static void gemv_check(int n, int k, const void* x, int ldx, int ldy, int m, bool glu) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0 && m >= 1 && m <= kMaxGemvRows, "gemv %d %d %d", n, k, m);
    CHECK(ldx >= k && ldx % 2 == 0 && ((uintptr_t)x & 3) == 0, "gemv ldx %d (even, >= k, x 4-byte aligned)", ldx);
    CHECK(ldy >= (glu ? n / 2 : n), "gemv ldy %d", ldy);
}

void gemv_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    gemv_check(w.n, w.k, x, ldx, ldy, m, w.glu);
    gemv_dispatch<kFmtW4>(w.q, w.s, w.sdt, w.glu, w.n, w.k, x, ldx, y, ldy, m, out_bf16, st);
}

void gemv_w8(const W8& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    gemv_check(w.n, w.k, x, ldx, ldy, m, false);
    if (w.per_channel) gemv_dispatch<kFmtW8C>(w.q, w.s, w.sdt, false, w.n, w.k, x, ldx, y, ldy, m, out_bf16, st);
    else gemv_dispatch<kFmtW8G>(w.q, w.s, w.sdt, false, w.n, w.k, x, ldx, y, ldy, m, out_bf16, st);
}
