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

// 0x0F0F0F0F in an SGPR, opaque to the compiler's known-bits analysis (a scalar move: no VALU work goes through
// inline asm in these kernels, since the compiler's MFMA hazard checks do not look into asm operands)
__device__ __forceinline__ uint32_t nib_mask() {
    uint32_t m;
    asm("s_mov_b32 %0, 0x0f0f0f0f" : "=s"(m));
    return m;
}
// 0xF0F0F0F0 in an SGPR (as nib_mask)
__device__ __forceinline__ uint32_t nib_mask_hi() {
    uint32_t m;
    asm("s_mov_b32 %0, 0xf0f0f0f0" : "=s"(m));
    return m;
}

template <int SDT>
__device__ __forceinline__ float scale_rt(uint16_t v, int sdt) {
    if constexpr (SDT >= 0) return scale_to_f32<SDT>(v);
    else return sdt == kScaleF16 ? scale_to_f32<kScaleF16>(v) : scale_to_f32<kScaleBF16>(v);
}

// The reference operand (w s rounded once to bf16, or fp16) of packed weight bytes, with fewer VALU instructions than
// a per-weight int -> float conversion: the 0x64 byte magic makes fp16 1024 + v of two bytes v at once (one v_perm per
// pair, SEL picks the bytes), and one v_fma_mix_f32 per weight gives (1024 + v) sv + bv = w s exactly in fp32:
//   W4 nibble in place  v = u:     sv = s,      bv = -1032 s   (w = u - 8)
//   W4 nibble kept high v = 16 u:  sv = s / 16, bv = -72 s
//   W8 byte             v = w + 128: sv = s,    bv = -1152 s
// With s an fp16 or bf16 scale (11 significant bits at most) every product and the sum fit fp32's 24 bits (for
// |s| >= 2^-120, so s / 16 stays normal), and the pack rounds the exact w s once.
constexpr uint32_t kSel02 = 0x04020400u, kSel13 = 0x04030401u, kSel01 = 0x04010400u, kSel23 = 0x04030402u;
template <uint32_t SEL>
__device__ __forceinline__ uint32_t magic_f16(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, SEL); }
template <bool F16 = false>
__device__ __forceinline__ uint32_t dq_pair(uint32_t magic_pair, float sv, float bv) {
    const f16x2_v h = __builtin_bit_cast(f16x2_v, magic_pair);
    const float lo = fmaf((float)h[0], sv, bv), hi = fmaf((float)h[1], sv, bv);
    return F16 ? pack_f16x2(lo, hi) : pack_bf16x2(lo, hi);
}
// fp16 operand of nibbles v = u (the low nibble of each byte): (1024 + u) - 1032 = u - 8 exactly in packed fp16, then
// one packed fp16 multiply by s rounds the exact product (u - 8) s once: fp16_rn((u - 8) s)
__device__ __forceinline__ uint32_t dq_f16_pair(uint32_t magic_pair, f16x2_v s2) {
    const f16x2_v w = __builtin_bit_cast(f16x2_v, magic_pair) - f16x2_v{(_Float16)1032.f, (_Float16)1032.f};
    return __builtin_bit_cast(uint32_t, w * s2);
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
