// Shared definitions of the qengine_amd kernel library (gfx950 / CDNA4, HIP).
//
// Error convention (the reference's, src/common.h:10-36): a violated shape precondition prints
// "check failed <cond> at <file>:<line>: <message>" to stderr and aborts; a failing HIP call prints the
// HIP error string and aborts. Shape checks always run on the host before anything touches the GPU.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

[[noreturn]] void qe_fatal_check();
[[noreturn]] void qe_fatal_hip(hipError_t err, const char* what, const char* file, int line);

#define HIP_CHECK(x)                                                          \
    do {                                                                      \
        hipError_t err__ = (x);                                               \
        if (err__ != hipSuccess) qe_fatal_hip(err__, #x, __FILE__, __LINE__); \
    } while (0)

#define CHECK(cond, ...)                                                                   \
    do {                                                                                   \
        if (!(cond)) {                                                                     \
            fprintf(stderr, "check failed %s at %s:%d: ", #cond, __FILE__, __LINE__);      \
            fprintf(stderr, __VA_ARGS__);                                                  \
            fprintf(stderr, "\n");                                                         \
            qe_fatal_check();                                                              \
        }                                                                                  \
    } while (0)

// 16-bit float storage types as they cross the C-ABI (raw bit patterns).
typedef uint16_t bf16_t;
typedef uint16_t f16_t;

// Scale dtype of an INT4 / INT8 matrix. The 27B checkpoints store bf16 group scales, the Flash-Next experts
// and the BASELINE workloads fp16 (reference gemv.cuh:14, flash.h:203-218); the repack copies 16-bit patterns.
enum QeScale : int { kScaleBF16 = 0, kScaleF16 = 1 };

// Flags of the build-defined *_ex entry points.
enum QeFlags : int {
    kFlagScaleF16 = 1,  // scales are fp16 (default bf16)
    kFlagOutBF16 = 2,   // y is bf16 [m][ldy] (round to nearest even), default fp32
    kFlagGLU = 4,       // GLU matrix: y is the bf16 activation [m][ldy], ldy >= n / 2
};

constexpr int kMaxGemvRows = 16;   // VALU decode GEMV / skinny GEMM: m = 1..16 rows per launch
constexpr int kWideRows = 32;      // the INT4 skinny kernel's wide variant: 17..32 rows per launch
constexpr int kMaxGemvW4Tokens = 32;  // reference matmul(): m <= 32 -> GEMV, else GEMM (gemv.cuh:187-190)
// this build's matmul_w4 dispatch: the decode kernels up to 64 rows, the GEMM above. Measured on MI355X (N = 17408,
// K = 5120): the 256-token-tile GEMM takes about 82 us for any m in 33..64 (68 tiles on 256 CUs). 17..64 rows run the
// one-pass kernel (wdec.hip: m = 32 / 64 in 26 / 40 us against 29 / 58 us for 32-row skinny launches); with
// batch_invariant, 16- and 32-row skinny launches, so every row of a 1..64-row call has the same bits as alone
constexpr int kMatmulGemvRows = 64;

#ifdef __HIPCC__
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_v;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_v;
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef __attribute__((ext_vector_type(4))) float f32x4_v;
typedef __attribute__((ext_vector_type(16))) float f32x16_v;

// 16-bit scale pattern -> float (exact for both dtypes)
template <int SDT>
__device__ __forceinline__ float scale_to_f32(uint16_t v) {
    if constexpr (SDT == kScaleF16) {
        return (float)__builtin_bit_cast(_Float16, v);
    } else {
        return __builtin_bit_cast(float, (uint32_t)v << 16);
    }
}
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }
// float -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32); NaN stays NaN
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) float f32x2_v;
    const f32x2_v v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}
// two floats -> an fp16 pair, round to nearest even (gfx950 v_cvt_pk_f16_f32); fp16 bits -> float (exact)
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) float f32x2_v;
    const f32x2_v v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_v));
}
__device__ __forceinline__ float f16_to_f32(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ float f16_round(float f) { return (float)(_Float16)f; }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
// MoE intermediates (the GLU activation and the per-(token, k) down outputs) are fp16 of the value / 16, the
// reference's formats (its XH activation scale and kSlotScale, flash_kernels.cuh:6185,6308,6421-6427)
constexpr float kMoeF16Scale = 0.0625f;
__device__ __forceinline__ float silu_f32(float x) { return x / (1.f + __expf(-x)); }
#endif
