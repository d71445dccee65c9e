// Shared pieces of the MFMA matmul kernels (prefill GEMM, MoE grouped GEMMs): the swizzled [rows][64] bf16 LDS
// tile and the in-register dequantization of W4 / W8 records to the reference's bf16 operand.
#pragma once
#include "qe_api.hpp"

namespace qe_tile {

typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));

// byte offset of the 16-byte chunk `c` (0..7) of row `r` in a [rows][64] bf16 tile: 128-byte rows, chunks XOR-swizzled
// by f(r) = (r & 7) ^ ((r >> 3) & 3). Measured on gfx950 (SQ_LDS_BANK_CONFLICT): with this f the MFMA fragment
// reads (32 consecutive rows x one 16-byte chunk per half-wave), the 4-byte dequantized-weight stores of two
// 16-row tiles per wave and the 16-byte row-pair stores are all conflict-free; with f = r & 7 the fragment reads
// take 4 extra cycles per instruction. f depends on r % 32 only, so the fragment rows of a 32-aligned block share
// one set of per-lane offsets.
__device__ __forceinline__ int swz_f(int r) { return (r & 7) ^ ((r >> 3) & 3); }
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ swz_f(r)) << 4); }

// byte B of v as float: one v_cvt_f32_ubyte{B}, as long as the compiler cannot see that the high nibbles of v are
// zero (then it extracts a 4-bit field and converts byte 0 instead): nibble masks come from nib_mask()
template <int B>
__device__ __forceinline__ float cvt_ubyte(uint32_t v) {
    return static_cast<float>((v >> (8 * B)) & 0xFFu);
}
// 0x0F0F0F0F in an SGPR, opaque to the compiler's known-bits analysis (a scalar move: no VALU work goes through
// inline asm in these kernels, since the compiler's MFMA hazard checks do not look into asm operands)
__device__ __forceinline__ uint32_t nib_mask() {
    uint32_t m;
    asm("s_mov_b32 %0, 0x0f0f0f0f" : "=s"(m));
    return m;
}

template <int SDT>
__device__ __forceinline__ float scale_rt(uint16_t v, int sdt) {
    if constexpr (SDT >= 0) return scale_to_f32<SDT>(v);
    else return sdt == kScaleF16 ? scale_to_f32<kScaleF16>(v) : scale_to_f32<kScaleBF16>(v);
}

// The reference operand of a nibble byte v (v = u, or v = 16 u where a high nibble is kept in place), with fewer VALU
// instructions than a per-weight int -> float conversion:
//   bf16: the 0x64 byte magic makes fp16 1024 + v (one v_perm per pair of weights), and one v_fma_mix_f32 per weight
//         gives (1024 + v) sv + bv = (u - 8) s exactly in fp32 (sv = s, bv = -1032 s for v = u; sv = s / 16,
//         bv = -72 s for v = 16 u: every product and the sum fit fp32's 24 bits), rounded once to bf16
//   fp16 (v = u only): (1024 + u) - 1032 = u - 8 exactly in packed fp16, then one packed fp16 multiply by s rounds
//         the exact product (u - 8) s once: fp16_rn((u - 8) s)
// Pairs are bytes (0, 2) and (1, 3) of t.
__device__ __forceinline__ uint32_t magic_f16_b02(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04020400u); }
__device__ __forceinline__ uint32_t magic_f16_b13(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04030401u); }
__device__ __forceinline__ uint32_t dq_bf16_pair(uint32_t magic_pair, float sv, float bv) {
    const f16x2_v h = __builtin_bit_cast(f16x2_v, magic_pair);
    return pack_bf16x2(fmaf((float)h[0], sv, bv), fmaf((float)h[1], sv, bv));
}
__device__ __forceinline__ uint32_t dq_f16_pair(uint32_t magic_pair, f16x2_v s2) {
    const f16x2_v w = __builtin_bit_cast(f16x2_v, magic_pair) - f16x2_v{(_Float16)1032.f, (_Float16)1032.f};
    return __builtin_bit_cast(uint32_t, w * s2);
}

// dequantize the 8 nibbles of one W4 word (rows g / g + 8, k0 + {0, 1, 8, 9}) to bf16_rn((u - 8) * s) and store them
// as 4 bf16 pairs at (row, k0) (row, k0 + 8) (row + 8, k0) (row + 8, k0 + 8) of the tile
__device__ __forceinline__ void dq_w4_word(uint32_t wd, float s_lo, float s_hi, char* wt, int row, int k0) {
    const uint32_t nm = nib_mask();
    const uint32_t ev = wd & nm;         // bytes: slots 0, 2, 4, 6 (row g: k0, k0+8, k0+1, k0+9)
    const uint32_t od = (wd >> 4) & nm;  // slots 1, 3, 5, 7 (row g + 8)
    const float b_lo = -8.f * s_lo, b_hi = -8.f * s_hi;
    // (u - 8) * s = fma(u, s, -8 s): exact in fp32, then one rounding to bf16
    const uint32_t g0 = pack_bf16x2(fmaf(cvt_ubyte<0>(ev), s_lo, b_lo), fmaf(cvt_ubyte<2>(ev), s_lo, b_lo));
    const uint32_t g8 = pack_bf16x2(fmaf(cvt_ubyte<1>(ev), s_lo, b_lo), fmaf(cvt_ubyte<3>(ev), s_lo, b_lo));
    const uint32_t h0 = pack_bf16x2(fmaf(cvt_ubyte<0>(od), s_hi, b_hi), fmaf(cvt_ubyte<2>(od), s_hi, b_hi));
    const uint32_t h8 = pack_bf16x2(fmaf(cvt_ubyte<1>(od), s_hi, b_hi), fmaf(cvt_ubyte<3>(od), s_hi, b_hi));
    // k0 = 16 j + 2 t: pair (k0, k0+1) lives in chunk k0 / 8, byte (k0 % 8) * 2
    const int c0 = k0 >> 3, o0 = (k0 & 7) * 2;
    *reinterpret_cast<uint32_t*>(wt + swz(row, c0) + o0) = g0;
    *reinterpret_cast<uint32_t*>(wt + swz(row, c0 + 1) + o0) = g8;
    *reinterpret_cast<uint32_t*>(wt + swz(row + 8, c0) + o0) = h0;
    *reinterpret_cast<uint32_t*>(wt + swz(row + 8, c0 + 1) + o0) = h8;
}

// global_load_lds_dwordx4: lane i's 16 bytes land at LDS byte m0 + 16 i. Issued from inline asm so that the
// compiler, which cannot tell these LDS writes from the stage the MFMAs read, does not wait for them before every
// LDS read; the kernel waits for them itself (vmcnt) before the barrier that publishes the stage. An LDS DMA that
// reads m0 needs one wait state after the scalar write of m0 (GFX9): the s_nop.
// lds_dst: LDS byte address, wave-uniform
__device__ __forceinline__ void dma16(const void* src, unsigned lds_dst) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_dst), "v"(src) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* src, unsigned lds_dst) {  // 4 bytes per lane
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_dst), "v"(src) : "memory", "m0");
}

// 32x32 MFMA C fragment: lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 for r = 0..15
__device__ __forceinline__ int c_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

}  // namespace qe_tile
