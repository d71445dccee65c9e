// Load-time layout kernels: compressed-tensors INT4 -> W4 fragment layout, GLU row interleave, INT8 -> W8
// layout (RTN quantization or pre-quantized tiling), and standalone dequantization (bit-exact, for tests and
// for callers that want bf16 weights).
//
// The W4 fragment layout is a fixed format shared with the reference (gemv.cu:515-549): destination u32 `idx`
// holds, for tile r (16 rows), 64-k chunk c, lane l (g = l / 4, t = l % 4) and k-step j, the eight nibbles
// slot s = rowhalf + 2 * khalf + 4 * odd of rows 16 r + g + 8 rowhalf at k = 64 c + 16 j + 2 t + 8 khalf + odd.
#include "qe_api.hpp"

namespace {

__device__ __forceinline__ uint32_t src_nibble(const int32_t* __restrict__ q, int K, int row, int k) {
    return ((uint32_t)q[(size_t)row * (K >> 3) + (k >> 3)] >> (4 * (k & 7))) & 15u;
}

__global__ void repack_w4_kernel(const int32_t* __restrict__ src, int N, int K, uint32_t* __restrict__ dst) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * K / 8) return;
    const int j = (int)(idx & 3), lane = (int)((idx >> 2) & 31);
    const size_t chunk = idx >> 7;
    const int chunks = K >> 6;
    const int r = (int)(chunk / chunks), c = (int)(chunk % chunks);
    const int row = 16 * r + (lane >> 2);
    const int k0 = 64 * c + 16 * j + 2 * (lane & 3);
    uint32_t word = 0;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int rr = row + 8 * (s & 1), kk = k0 + 8 * ((s >> 1) & 1) + (s >> 2);
        word |= src_nibble(src, K, rr, kk) << (4 * s);
    }
    dst[idx] = word;
}

// [N][G] -> [N/16][G][16]
__global__ void repack_scales_kernel(const uint16_t* __restrict__ src, int N, int G, uint16_t* __restrict__ dst) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * G) return;
    const int i = (int)(idx & 15);
    const size_t rg = idx >> 4;
    const int r = (int)(rg / G), gi = (int)(rg % G);
    dst[idx] = src[(size_t)(16 * r + i) * G + gi];
}

// one block per destination row: rows [gate 0..I)[up 0..I) -> per 16-row tile 8 gate rows then 8 up rows
__global__ void glu_rows_kernel(const int32_t* __restrict__ sq, const uint16_t* __restrict__ ss, int N, int G,
                                int32_t* __restrict__ dq, uint16_t* __restrict__ ds, int wpr) {
    const int dr = blockIdx.x, half = N / 2;
    const int tile = dr >> 4, j = dr & 15;
    const int sr = (j < 8) ? 8 * tile + j : half + 8 * tile + (j - 8);
    for (int i = threadIdx.x; i < wpr; i += blockDim.x) dq[(size_t)dr * wpr + i] = sq[(size_t)sr * wpr + i];
    for (int i = threadIdx.x; i < G; i += blockDim.x) ds[(size_t)dr * G + i] = ss[(size_t)sr * G + i];
}

// W4 fragment layout -> bf16 row-major [N][K], d = bf16_rn((u - 8) * s); one thread per packed u32
template <int SDT>
__global__ void dequant_w4_kernel(const uint32_t* __restrict__ q, const uint16_t* __restrict__ s, int N, int K,
                                  uint16_t* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * K / 8) return;
    const int j = (int)(idx & 3), lane = (int)((idx >> 2) & 31);
    const size_t chunk = idx >> 7;
    const int chunks = K >> 6, G = K >> 7;
    const int r = (int)(chunk / chunks), c = (int)(chunk % chunks);
    const int row = 16 * r + (lane >> 2);
    const int k0 = 64 * c + 16 * j + 2 * (lane & 3);
    const uint32_t word = q[idx];
#pragma unroll
    for (int sl = 0; sl < 8; sl++) {
        const int rr = row + 8 * (sl & 1), kk = k0 + 8 * ((sl >> 1) & 1) + (sl >> 2);
        const float sc = scale_to_f32<SDT>(s[((size_t)r * G + (kk >> 7)) * 16 + (rr & 15)]);
        const float d = (float)((int)((word >> (4 * sl)) & 15u) - 8) * sc;  // exact in fp32
        out[(size_t)rr * K + kk] = f32_to_bf16(d);
    }
}

// byte offset of element (row, k) in the W8 layout (reference gemv.cu:1102-1113)
__device__ __forceinline__ size_t w8_pos(int row, int k, int K) {
    const int rt = row >> 4, rr = row & 15;
    const int ks = k >> 4, col = k & 15;
    const int tq = (col & 7) >> 1, half = col >> 3, odd = col & 1;
    const int ln = (rr & 7) * 4 + tq;
    const int ai = (half * 2 + (rr >> 3)) * 2 + odd;
    return (((size_t)rt * (K >> 5) + (ks >> 1)) * 32 + ln) * 16 + (ks & 1) * 8 + ai;
}

// RTN INT8, group 128, bf16 scale = bf16(amax / 127), q = clamp(rint(v / scale), -127, 127) (the closed form of
// reference tests/test_w8.py:6-9). One wave per (row, group): lane holds 2 consecutive values.
__global__ void quantize_w8_kernel(const uint16_t* __restrict__ src, int N, int K, uint8_t* __restrict__ q,
                                   uint16_t* __restrict__ s) {
    const int wave = (int)(((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6), lane = threadIdx.x & 63;
    const int G = K >> 7;
    if (wave >= N * G) return;
    const int row = wave / G, gi = wave % G;
    const int k = gi * 128 + 2 * lane;
    const float v0 = bf16_to_f32(src[(size_t)row * K + k]), v1 = bf16_to_f32(src[(size_t)row * K + k + 1]);
    float mx = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const uint16_t sb = f32_to_bf16(mx / 127.f);
    const float sc = bf16_to_f32(sb);
    const float div = sc > 0.f ? sc : 1.f;
    const int q0 = max(-127, min(127, (int)rintf(v0 / div)));
    const int q1 = max(-127, min(127, (int)rintf(v1 / div)));
    q[w8_pos(row, k, K)] = (uint8_t)(int8_t)q0;
    q[w8_pos(row, k + 1, K)] = (uint8_t)(int8_t)q1;
    if (lane == 0) s[((size_t)(row >> 4) * G + gi) * 16 + (row & 15)] = sb;
}

// pre-quantized int8 [N][K] row-major (+ scales) -> W8 layout. per_channel: scales [N] copied as they are;
// else group-128 scales [N][K/128] -> [N/16][K/128][16]
__global__ void tile_w8_kernel(const int8_t* __restrict__ src, const uint16_t* __restrict__ ssrc, int N, int K,
                               uint8_t* __restrict__ q, uint16_t* __restrict__ s, bool per_channel) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int row = (int)(i / K), k = (int)(i % K);
    q[w8_pos(row, k, K)] = (uint8_t)src[i];
    if (per_channel) {
        if (k == 0) s[row] = ssrc[row];
    } else if ((k & 127) == 0) {
        s[((size_t)(row >> 4) * (K >> 7) + (k >> 7)) * 16 + (row & 15)] = ssrc[(size_t)row * (K >> 7) + (k >> 7)];
    }
}

template <int SDT>
__global__ void dequant_w8_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s, int N, int K,
                                  bool per_channel, uint16_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int row = (int)(i / K), k = (int)(i % K);
    const float w = (float)(int8_t)q[w8_pos(row, k, K)];
    const float sc = per_channel ? scale_to_f32<SDT>(s[row])
                                 : scale_to_f32<SDT>(s[((size_t)(row >> 4) * (K >> 7) + (k >> 7)) * 16 + (row & 15)]);
    out[i] = f32_to_bf16(w * sc);
}

unsigned grid_for(size_t items, int block) { return (unsigned)((items + block - 1) / block); }

// compressed-tensors 8-bit -> Q8: one thread per destination word (lane (g, t), word 2 s + hi of tile r, 32-k chunk
// c): its 4 bytes are rows g + 8 hi at k = 32 c + 16 s + 2 t + {0, 8, 1, 9}, each u ^ 0x80 = the signed weight
__global__ void repack_q8_kernel(const int32_t* __restrict__ src, int N, int K, uint32_t* __restrict__ dst) {
    const size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * K / 4) return;
    const int word = idx & 3, lane = (idx >> 2) & 31;
    const size_t tc = idx >> 7;  // tile * (K / 32) + chunk
    const int r = (int)(tc / (K >> 5)), c = (int)(tc % (K >> 5));
    const int row = 16 * r + (lane >> 2) + 8 * (word & 1);
    const int k0 = 32 * c + 16 * (word >> 1) + 2 * (lane & 3);
    const uint32_t* sr = reinterpret_cast<const uint32_t*>(src) + (size_t)row * (K >> 2);
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int k = k0 + (i & 1) * 8 + (i >> 1);
        v |= (((sr[k >> 2] >> (8 * (k & 3))) & 0xFFu) ^ 0x80u) << (8 * i);
    }
    dst[idx] = v;
}

}  // namespace

void repack_q8(const int32_t* src_q, const uint16_t* src_s, int n, int k, uint4* dst_q, uint16_t* dst_s,
               hipStream_t st) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0, "repack_q8 %d %d", n, k);
    const size_t words = (size_t)n * k / 4, ns = (size_t)n * (k / 128);
    repack_q8_kernel<<<grid_for(words, 256), 256, 0, st>>>(src_q, n, k, reinterpret_cast<uint32_t*>(dst_q));
    repack_scales_kernel<<<grid_for(ns, 256), 256, 0, st>>>(src_s, n, k / 128, dst_s);
    HIP_CHECK(hipGetLastError());
}

void repack_w4(const int32_t* src_q, const uint16_t* src_s, int n, int k, uint4* dst_q, uint16_t* dst_s,
               hipStream_t st) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0, "repack_w4 %d %d", n, k);
    const size_t words = (size_t)n * k / 8;
    repack_w4_kernel<<<grid_for(words, 256), 256, 0, st>>>(src_q, n, k, reinterpret_cast<uint32_t*>(dst_q));
    HIP_CHECK(hipGetLastError());
    const size_t ns = (size_t)n * (k / 128);
    repack_scales_kernel<<<grid_for(ns, 256), 256, 0, st>>>(src_s, n, k / 128, dst_s);
    HIP_CHECK(hipGetLastError());
}

void glu_interleave_rows(const int32_t* src_q, const uint16_t* src_s, int n, int k, int32_t* dst_q,
                         uint16_t* dst_s, hipStream_t st, int bits) {
    CHECK(n > 0 && n % 16 == 0 && k % 128 == 0 && (bits == 4 || bits == 8), "glu rows %d %d bits %d", n, k, bits);
    glu_rows_kernel<<<n, 256, 0, st>>>(src_q, src_s, n, k / 128, dst_q, dst_s, k * bits / 32);
    HIP_CHECK(hipGetLastError());
}

void dequant_w4(const W4& w, uint16_t* out, hipStream_t st) {
    CHECK(w.n > 0 && w.k > 0 && w.n % 16 == 0 && w.k % 128 == 0, "dequant_w4 %d %d", w.n, w.k);
    const size_t words = (size_t)w.n * w.k / 8;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(w.q);
    if (w.sdt == kScaleF16) dequant_w4_kernel<kScaleF16><<<grid_for(words, 256), 256, 0, st>>>(q, w.s, w.n, w.k, out);
    else dequant_w4_kernel<kScaleBF16><<<grid_for(words, 256), 256, 0, st>>>(q, w.s, w.n, w.k, out);
    HIP_CHECK(hipGetLastError());
}

void quantize_w8(const uint16_t* src, int n, int k, uint4* dst_q, uint16_t* dst_s, hipStream_t st) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0, "quantize_w8 %d %d", n, k);
    const size_t waves = (size_t)n * (k / 128);
    quantize_w8_kernel<<<grid_for(waves * 64, 256), 256, 0, st>>>(src, n, k, reinterpret_cast<uint8_t*>(dst_q), dst_s);
    HIP_CHECK(hipGetLastError());
}

void tile_w8(const int8_t* src, const uint16_t* ssrc, int n, int k, uint4* dst_q, uint16_t* dst_s, bool per_channel,
             hipStream_t st) {
    CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0, "tile_w8 %d %d", n, k);
    const size_t e = (size_t)n * k;
    tile_w8_kernel<<<grid_for(e, 256), 256, 0, st>>>(src, ssrc, n, k, reinterpret_cast<uint8_t*>(dst_q), dst_s,
                                                     per_channel);
    HIP_CHECK(hipGetLastError());
}

void dequant_w8(const W8& w, uint16_t* out, hipStream_t st) {
    CHECK(w.n > 0 && w.k > 0 && w.n % 16 == 0 && w.k % 128 == 0, "dequant_w8 %d %d", w.n, w.k);
    const size_t e = (size_t)w.n * w.k;
    const uint8_t* q = reinterpret_cast<const uint8_t*>(w.q);
    if (w.sdt == kScaleF16)
        dequant_w8_kernel<kScaleF16><<<grid_for(e, 256), 256, 0, st>>>(q, w.s, w.n, w.k, w.per_channel, out);
    else
        dequant_w8_kernel<kScaleBF16><<<grid_for(e, 256), 256, 0, st>>>(q, w.s, w.n, w.k, w.per_channel, out);
    HIP_CHECK(hipGetLastError());
}
