// Decode GEMM for up to 64 activation rows on the W4 layout, one pass over the weights (the reference's wide decode
// GEMVs, src/kernels/gemv_x.cu:1-12,902-980, read the matrix once for m 9..64).
//
// The skinny kernel (skinny.hip) stages every activation row of its K slice per wave and multiplies 16-row weight
// tiles on 16 x 16 MFMAs; past 16 rows its cost is the activation staging and the B operand reads, which grow with m,
// so 64 rows took two 32-row launches at ~29 us each on C0's matrix. Here the weights are the A operand of
// v_mfma_f32_32x32x16_bf16 built in registers (the MoE prefill GEMM's record-to-operand map, moe_pf.hip): a wave owns the 64
// weight rows (four 16-row tiles) of its block, and lane l = 32 kh + mr is A row mr = 8 q + g (tile q, row pair
// g / g + 8) for k half kh; bytes (h, h + 2) of word j of the pair's four records t = 0..3 are the 8 consecutive k of
// 16-byte chunk 2 j + h, and the MFMAs of a 64-k step take the chunks in the order c(ks, kh) = 2 (2 (ks % 2) + kh) +
// ks / 2, so a lane needs words kh and 2 + kh of its four records. Low nibbles are the A operand of row g, high
// nibbles (shifted down) that of row g + 8. The B operand is chunk c of a token row:
// one ds_read_b128 of the wave's staged activation tile ([32 rows][64 k] bf16, 16-byte chunks XOR-swizzled).
//
// Block = 4 waves = TB token blocks of 32 rows x KP = 4 / TB contiguous K parts, over one 64-row weight slab (N / 64
// blocks). Every wave stages its own activation rows, records and scales by LDS DMA (global_load_lds) into a ring of
// NBUF buffers, DEPTH = NBUF - 1 steps ahead, so no wave waits for another until the end; per 64-k step a wave issues 7 DMAs
// (four 1 KB activation pieces, two 1 KB record pieces, one 256-byte scale piece), and every wait is a compile-time
// vmcnt. The next k16 step's A operands are built between the MFMAs of the current one. After the K loop each
// wave stores its fp32 sums [32 tokens][64 rows] in LDS and the KP parts of a token are added in a fixed tree order,
// then the epilogue (fp32, bf16 or the GLU activation) stores the rows below m.
//
// Numerics: this build's decode arithmetic (as the m = 1 and skinny kernels): the A operands are the exact bf16
// 128 + u (a byte permute puts 0x43 above each nibble byte), one more MFMA per k16 step with A = -136 sums -136 x,
// and per 128-k group each output row takes acc += s (C + Cb) with its group scale s: the exact products (u - 8) x
// summed in fp32 and scaled once per group, i.e. the unrounded weights (u - 8) s. The result does not depend on
// timing (fixed K parts and sum order). Rows past m re-read row m - 1 and are not stored.
#include "mfma_tile.hpp"

#include <type_traits>

namespace qe_wdec {
using namespace qe_tile;

constexpr int NW = 4, NTH = 64 * NW, BK = 64, NBUF = 3, DEPTH = NBUF - 1;  // DMAs DEPTH steps ahead
constexpr int kX = 32 * BK * 2;               // a wave's 32 activation rows of one k step: [32][64] bf16, swizzled
constexpr int kRaw = 2048;                    // the wave's records of one k step: 4 tiles x 512 B
constexpr int kSc = 256;                      // the scales of the step's group, [4 tiles][16 rows] (+ a copy)
constexpr int kBuf = kX + kRaw + kSc;         // 6400 B per wave and buffer
constexpr int kLds = NBUF * NW * kBuf;        // 76800 B: two blocks per CU
constexpr int kPart = 68;                     // floats per token row of a wave's partial sums (64 rows + pad)
static_assert(NW * 32 * kPart * 4 <= kLds, "the partial sums fit the staging buffers");

// TB token blocks of 32 rows (m <= 32 TB), out: 0 fp32, 1 bf16, 2 GLU (bf16 activation, n / 2 columns)
// Blocks [0, nmain): one slab each over the whole K. Blocks past nmain: part p = u % P of tail slab nmain + u / P
// (u = block - nmain), over K steps [p KT / P, (p + 1) KT / P); its sums go to tpart[u] ([TB * 32 tokens][64 rows]
// fp32, written through to the device-coherent level), then it adds one to tctr[u / P]; the part that brings the
// count to P adds the P parts in order p = 0..P-1, stores the outputs and sets the count back to zero (the counters
// are zero when their buffer is allocated). P = 1: no tail blocks.
template <int SDT, int TB>
__global__ void __launch_bounds__(NTH, 2) wdec_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ s,
                                                      int K, const uint16_t* __restrict__ x, int ldx, int M,
                                                      void* __restrict__ y, int ldy, int out, int nmain, int P,
                                                      float* __restrict__ tpart, uint32_t* __restrict__ tctr) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    constexpr int KP = NW / TB;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned lds32 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);
    const int tb = wave / KP, kp = wave - tb * KP;
    const int b = blockIdx.x, tail = b >= nmain ? b - nmain : -1;  // tail part index u, or -1
    const int slab = tail < 0 ? b : nmain + tail / P, KTb = tail < 0 ? K / BK : K / BK / P;
    const int KTw = KTb / KP, kt0 = (tail < 0 ? 0 : (tail % P) * KTb) + kp * KTw, G = K >> 7;
    const int tile0 = slab * 4;  // the block's four 16-row tiles
    const int mr = lane & 31, kh = lane >> 5;
    auto buf_at = [&](int b) { return (b * NW + wave) * kBuf; };  // byte offset of this wave's buffer b

    // DMA sources. Activations: piece r (rows 8 r .. 8 r + 7), lane i lands at slot i of the piece, so it loads the
    // chunk that the swizzle puts there (row 8 r + i / 8, chunk (i % 8) ^ swz_f(row)). Records: lane i fetches record
    // (g = i % 8, t = i / 32, + 2 for the second piece) of tile (i / 8) % 4, landing at slot 32 t + mr. Scales: lane
    // i fetches the dword of rows 2 (i % 8), + 1 of tile (i / 8) % 4 (lanes 32..63 repeat lanes 0..31).
    const uint16_t* xsrc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int row = 8 * r + (lane >> 3), tok = 32 * tb + row;
        xsrc[r] = x + (size_t)(tok < M ? tok : M - 1) * ldx + (((lane & 7) ^ swz_f(row)) << 3);
    }
    const int dtl = tile0 + ((lane >> 3) & 3);
    const uint4* wsrc = q + (size_t)dtl * (K >> 6) * 32 + 4 * (lane & 7) + kh;
    const uint16_t* ssrc = s + (size_t)dtl * G * 16 + 2 * (lane & 7);
    // local step j (k step kt0 + j) into buffer j % NBUF (the buffer of step j - NBUF, finished): 7 DMAs. Steps past
    // the wave's last re-read its last step, so every wait below has the same count.
    auto dma_step = [&](int j) {
        const int kt = kt0 + (j < KTw ? j : KTw - 1);
        const unsigned b = lds32 + buf_at(j % NBUF);
#pragma unroll
        for (int r = 0; r < 4; r++) dma16(xsrc[r] + kt * BK, b + r * 1024);
        dma16(wsrc + (size_t)kt * 32, b + kX);
        dma16(wsrc + (size_t)kt * 32 + 2, b + kX + 1024);
        dma4(ssrc + (kt >> 1) * 16, b + kX + kRaw);
    };
    auto wait_dma = [&]() {  // all DMAs but those of the DEPTH - 1 steps issued last
        static_assert(DEPTH >= 2 && DEPTH <= 5, "DMA depth");
        if constexpr (DEPTH == 2) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
        else if constexpr (DEPTH == 3) asm volatile("s_waitcnt vmcnt(14)" ::: "memory");
        else if constexpr (DEPTH == 4) asm volatile("s_waitcnt vmcnt(21)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(28)" ::: "memory");
    };

    f32x16_v acc[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[h][r] = 0.f;
    int xo[BK / 16];  // B operand of k16 step ks: chunk c(ks, kh) of activation row mr (swizzled)
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) xo[ks] = mr * 128 + (((4 * (ks & 1) + 2 * kh + (ks >> 1)) ^ swz_f(mr)) << 4);

    // operand state, two sets by step parity: the words kh and 2 + kh of records t = 0..3, masked to their low
    // nibbles (rows g) and to their high nibbles shifted down (rows g + 8)
    uint32_t mlo[2][4][2], mhi[2][4][2];
    auto load_step = [&](int j, auto set) {  // records of local step j (its DMAs landed)
        constexpr int S = decltype(set)::value;
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(lds + buf_at(j % NBUF) + kX) + mr * 4 + kh;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const uint32_t v = rw[t * 128 + 2 * w];  // slot 32 t + mr, word kh + 2 w
                mlo[S][t][w] = v & nib_mask();
                mhi[S][t][w] = (v >> 4) & nib_mask();
            }
    };
    // A operand of k16 step ks (word kh + 2 (ks % 2), bytes (h, h + 2) with h = ks / 2) from masked words: 0x43 above
    // each nibble byte makes the exact bf16 pair 128 + u of k and k + 1, for records t = 0..3
    auto opnd = [&](const uint32_t (&mw)[4][2], int ks) {
        u32x4_v a;
#pragma unroll
        for (int t = 0; t < 4; t++)
            a[t] = (ks >> 1) ? __builtin_amdgcn_perm(0x43434343u, mw[t][ks & 1], kSel13)
                             : __builtin_amdgcn_perm(0x43434343u, mw[t][ks & 1], kSel02);
        return a;
    };
    // per 128-k group: c[op] = sum (128 + u) x and cb = -136 sum x on the matrix cores, then acc[op] += s (c[op] + cb)
    // for each output row (its group scale): the exact (u - 8) x products summed in fp32, scaled once per group
    f32x16_v c[2], cb;
    const f32x16_v zero = {};
    const u32x4_v bias_w = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};  // bf16 -136 pairs
    const bf16x8_v abias = __builtin_bit_cast(bf16x8_v, bias_w);
    auto group_end = [&](int j) {  // the group of local steps j - 1, j; its scales are in buffer j
        const uint16_t* sc = reinterpret_cast<const uint16_t*>(lds + buf_at(j % NBUF) + kX + kRaw) + 4 * kh;
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            // register 4 qq + i of operand op is row 4 kh + i (+ 8 op) of tile qq
            const uint2 s0 = *reinterpret_cast<const uint2*>(sc + 16 * qq);
            const uint2 s1 = *reinterpret_cast<const uint2*>(sc + 16 * qq + 8);
            const uint16_t sv0[4] = {(uint16_t)s0.x, (uint16_t)(s0.x >> 16), (uint16_t)s0.y, (uint16_t)(s0.y >> 16)};
            const uint16_t sv1[4] = {(uint16_t)s1.x, (uint16_t)(s1.x >> 16), (uint16_t)s1.y, (uint16_t)(s1.y >> 16)};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 4 * qq + i;
                acc[0][r] = fmaf(scale_to_f32<SDT>(sv0[i]), c[0][r] + cb[r], acc[0][r]);
                acc[1][r] = fmaf(scale_to_f32<SDT>(sv1[i]), c[1][r] + cb[r], acc[1][r]);
            }
        }
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using T_ = std::true_type;
    using F_ = std::false_type;

    // prologue: steps 0 .. DEPTH - 1 in flight, wait for step 0, its first operands
#pragma unroll
    for (int d = 0; d < DEPTH; d++) dma_step(d);
    wait_dma();
    load_step(0, P0{});
    u32x4_v an[2][2];  // A operands by k16 parity: [parity][op]
    an[0][0] = opnd(mlo[0], 0);
    an[0][1] = opnd(mhi[0], 0);

    bf16x8_v xf[2];
    // step j (set S = j % 2; groups start at even steps): the DMAs of step j + DEPTH; per k16 step ks the MFMAs of
    // rows g, rows g + 8 and the bias, with the next k16 step's operands (or step j + 1's first, from the other set,
    // whose records are read at ks = 2 after the wait for its DMAs) built between them. The LDS reads of buffer j end
    // before the next step's DMAs reuse it.
    auto kstep = [&](int j, auto more, auto set) {
        constexpr bool MORE = decltype(more)::value;
        constexpr int S = decltype(set)::value;
        using SN = std::integral_constant<int, S ^ 1>;
        dma_step(j + DEPTH);
        const char* xt = lds + buf_at(j % NBUF);
        xf[0] = *reinterpret_cast<const bf16x8_v*>(xt + xo[0]);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            const u32x4_v a0 = an[ks & 1][0], a1 = an[ks & 1][1];  // bit casts take a named temporary
            const bf16x8_v A0 = __builtin_bit_cast(bf16x8_v, a0);
            const bf16x8_v A1 = __builtin_bit_cast(bf16x8_v, a1);
            const bool first = S == 0 && ks == 0;  // the group's first k16 step starts its sums at zero
            if (ks + 1 < BK / 16) xf[(ks + 1) & 1] = *reinterpret_cast<const bf16x8_v*>(xt + xo[ks + 1]);
            if (ks == 2 && MORE) {
                wait_dma();
                load_step(j + 1, SN{});
            }
            __builtin_amdgcn_sched_barrier(0);
            c[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A0, xf[ks & 1], first ? zero : c[0], 0, 0, 0);
            if (ks + 1 < BK / 16) an[(ks + 1) & 1][0] = opnd(mlo[S], ks + 1);
            else if (MORE) an[0][0] = opnd(mlo[S ^ 1], 0);
            __builtin_amdgcn_sched_barrier(0);
            c[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A1, xf[ks & 1], first ? zero : c[1], 0, 0, 0);
            if (ks + 1 < BK / 16) an[(ks + 1) & 1][1] = opnd(mhi[S], ks + 1);
            else if (MORE) an[0][1] = opnd(mhi[S ^ 1], 0);
            __builtin_amdgcn_sched_barrier(0);
            cb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(abias, xf[ks & 1], first ? zero : cb, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (S == 1) group_end(j);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    // KTw even, >= 2: pairs of steps (one group), the last one without a next step
    for (int j = 0; j + 2 < KTw; j += 2) {
        kstep(j, T_{}, P0{});
        kstep(j + 1, T_{}, P1{});
    }
    kstep(KTw - 2, T_{}, P0{});
    kstep(KTw - 1, F_{}, P1{});

    // partial sums: lane l holds token mr, register r = 4 q' + i of operand op is weight row 16 q' + 4 kh + i + 8 op
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-read steps' DMAs have landed
    __syncthreads();  // every wave is done with the staging buffers
    float* part = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int qq = 0; qq < 4; qq++)
#pragma unroll
        for (int op = 0; op < 2; op++)
            *reinterpret_cast<f32x4_v*>(part + (wave * 32 + mr) * kPart + 16 * qq + 8 * op + 4 * kh) =
                f32x4_v{acc[op][4 * qq], acc[op][4 * qq + 1], acc[op][4 * qq + 2], acc[op][4 * qq + 3]};
    __syncthreads();
    // the KP parts of a token block added in a fixed tree order (parts i and i + h, h = KP / 2, ..., 1)
    auto sum4 = [&](int otb, int tok, int r4) {  // rows r4 .. r4 + 3 of the slab
        f32x4_v p[KP];
#pragma unroll
        for (int k = 0; k < KP; k++)
            p[k] = *reinterpret_cast<const f32x4_v*>(part + ((otb * KP + k) * 32 + tok) * kPart + r4);
#pragma unroll
        for (int h = KP / 2; h >= 1; h >>= 1)
#pragma unroll
            for (int i = 0; i < h; i++) p[i] = p[i] + p[i + h];
        return p[0];
    };
    const int n0 = tile0 * 16;
    // the epilogue of 4 consecutive rows r4 of token otb * 32 + tok, from get4(otb, tok, r4)
    auto emit = [&](auto&& get4) {
        if (out == 2) {  // thread = (token, tile, row quad of the 8 gate rows): gate rows g, up rows g + 8
            for (int o = tid; o < TB * 32 * 8; o += NTH) {
                const int otb = o >> 8, tok = (o >> 3) & 31, qq = (o >> 1) & 3, gq = o & 1;
                const int t = 32 * otb + tok;
                if (t >= M) continue;
                const f32x4_v ga = get4(otb, tok, 16 * qq + 4 * gq), up = get4(otb, tok, 16 * qq + 8 + 4 * gq);
                uint16_t* p = reinterpret_cast<uint16_t*>(y) + (size_t)t * ldy + (tile0 + qq) * 8 + 4 * gq;
#pragma unroll
                for (int i = 0; i < 4; i++) p[i] = f32_to_bf16(silu_f32(ga[i]) * up[i]);
            }
            return;
        }
        for (int o = tid; o < TB * 32 * 16; o += NTH) {  // thread = (token, 4 consecutive rows)
            const int otb = o >> 9, tok = (o >> 4) & 31, r4 = 4 * (o & 15);
            const int t = 32 * otb + tok;
            if (t >= M) continue;
            const f32x4_v v = get4(otb, tok, r4);
            if (out == 1) {
                uint16_t* p = reinterpret_cast<uint16_t*>(y) + (size_t)t * ldy + n0 + r4;
#pragma unroll
                for (int i = 0; i < 4; i++) p[i] = f32_to_bf16(v[i]);
            } else {
                float* p = reinterpret_cast<float*>(y) + (size_t)t * ldy + n0 + r4;
#pragma unroll
                for (int i = 0; i < 4; i++) p[i] = v[i];
            }
        }
    };
    if (tail < 0) {
        emit(sum4);
        return;
    }
    // a tail part: its sums to tpart[tail] (device-coherent stores), completed before the count
    constexpr int kPartFloats = TB * 32 * 64;
    float* mine = tpart + (size_t)tail * kPartFloats;
    for (int o = tid; o < TB * 32 * 16; o += NTH) {
        const int otb = o >> 9, tok = (o >> 4) & 31, r4 = 4 * (o & 15);
        const f32x4_v v = sum4(otb, tok, r4);
#pragma unroll
        for (int i = 0; i < 4; i++)
            __hip_atomic_store(mine + (otb * 32 + tok) * 64 + r4 + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __shared__ uint32_t last;
    __syncthreads();
    const int ts = tail / P;
    if (tid == 0) last = atomicAdd(&tctr[ts], 1u) == (uint32_t)P - 1u;
    __syncthreads();
    if (!last) return;
    const float* all = tpart + (size_t)ts * P * kPartFloats;  // parts p = 0..P-1 of this tail slab
    emit([&](int otb, int tok, int r4) {  // the parts in order p = 0..P-1
        f32x4_v v = {0.f, 0.f, 0.f, 0.f};
        for (int pp = 0; pp < P; pp++) {
            float* src = const_cast<float*>(all) + (size_t)pp * kPartFloats + (otb * 32 + tok) * 64 + r4;
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] += __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return v;
    });
    if (tid == 0) __hip_atomic_store(&tctr[ts], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int token_blocks(int m) { return m > 32 ? 2 : 1; }

}  // namespace qe_wdec

namespace qe_wdec {
// K parts per tail slab (1: none): for the slabs past the last whole round of CUs, and for every slab where the slabs
// fill at most half of the CUs (N = 5120: 80 slabs; then the most parts that fit the CUs), the first P of the list with
// the tail blocks within one round and an even number of K steps per wave
int tail_parts(int nslabs, int KT, int KP, int ncu) {
    const bool few = 2 * nslabs <= ncu;
    if (!few && (nslabs <= ncu || nslabs % ncu == 0)) return 1;
    const int rem = few ? nslabs : nslabs % ncu;
    for (int p : few ? std::initializer_list<int>{10, 8, 5, 4, 3, 2} : std::initializer_list<int>{5, 4, 8, 10, 2})
        if (rem * p <= ncu && KT % (p * KP) == 0 && (KT / (p * KP)) % 2 == 0) return p;
    return 1;
}
}  // namespace qe_wdec

bool wdec_w4_fits(const W4& w, const uint16_t* x, int ldx, int m) {
    using namespace qe_wdec;
    if (m < 1 || m > 64 || w.n % 64 != 0 || w.k % BK != 0 || ((uintptr_t)x & 15) != 0 || ldx % 8 != 0) return false;
    const int KP = NW / token_blocks(m), KT = w.k / BK;
    return KT % KP == 0 && (KT / KP) % 2 == 0;
}

namespace qe_gemv {
int decode_groups(int n, int k);
}

// Where the one-pass kernel beats the skinny kernel's 32-row launches (measured in one process, bf16 out, us one-pass
// / skinny): one round of slabs or more (N = 17408, K = 5120, m = 32: 20.7 / 28.9), K without an even skinny slicing
// (the skinny kernel's uneven slices; N = 3072, K = 9216, m = 32: 14.5 / 20.4), and more than 48 rows from ~26 M
// weights (N = K = 8192, m = 64: 27.6 / 30.2; N = K = 5120: 20.3 / 21.5). Small matrices keep the skinny launches:
// N = K = 4096, m = 32: 11.8 / 7.8; N = K = 2048: 9.4 / 5.0; N = 6144, K = 4096, m = 64: 18.9 / 18.2.
bool wdec_w4_pick(const W4& w, const uint16_t* x, int ldx, int m) {
    using namespace qe_wdec;
    if (!wdec_w4_fits(w, x, ldx, m)) return false;
    const int nslabs = w.n / 64, ncu = qe_num_cus();
    // slabs filling at most half the CUs only with K parts (N = 4096, K = 11008, m = 48: 64 slabs, no part count fits
    // 172 steps: 48.4 us against 35.2)
    if (2 * nslabs <= ncu && tail_parts(nslabs, w.k / BK, NW / token_blocks(m), ncu) == 1) return false;
    if (nslabs >= ncu || qe_gemv::decode_groups(w.n, w.k) == 0) return true;
    return m > 48 && (long)w.n * w.k >= (26L << 20);
}

// Slabs past the last whole round of CUs (N / 64 = 272 on 256 CUs: 16) would give 16 CUs two slabs; they run as P
// K parts each instead (tail blocks, sharing CUs with the whole slabs), so no CU gets two slabs' work: P the first
// of 5, 4, 8, 10, 2 with the tail blocks at most one round and an even number of steps per wave, if the stream's
// zero-initialised workspace (kWsDec: counters, then the parts' sums) is at hand (not allocated during graph
// capture: then P = 1). The last part's in-order sum reads the P parts from the device-coherent level, one part at
// a time, so fewer parts finish sooner: on C0's matrix (16 tail slabs, 80 K steps) P = 5 measured m = 32 / 64
// 20.7 / 31.7 us against 22.9 / 36.9 us at P = 10, 23.1 / 33.3 us at P = 2, and 26.7 / 40.0 us with no tail split.
void wdec_w4(const W4& w, const uint16_t* x, int ldx, void* y, int ldy, int m, bool out_bf16, hipStream_t st) {
    using namespace qe_wdec;
    CHECK(wdec_w4_fits(w, x, ldx, m), "wdec_w4: n %d k %d m %d ldx %d", w.n, w.k, m, ldx);
    CHECK(ldy >= (w.glu ? w.n / 2 : w.n), "wdec_w4 ldy %d", ldy);
    const int out = w.glu ? 2 : out_bf16 ? 1 : 0;
    const int TB = token_blocks(m), KP = NW / TB, KT = w.k / BK, nslabs = w.n / 64, ncu = qe_num_cus();
    int nmain = nslabs, P = 1, rem = 0;
    float* tpart = nullptr;
    uint32_t* tctr = nullptr;
    const int p = qe_wdec::tail_parts(nslabs, KT, KP, ncu);
    if (p > 1) {
        // one size for every shape (at most ncu tail blocks of two token blocks), so a stream's first call sizes it
        // for all later ones, graph captures included
        char* ws = dec_tail_ws(st);
        if (ws) {
            rem = 2 * nslabs <= ncu ? nslabs : nslabs % ncu;
            P = p;
            tctr = reinterpret_cast<uint32_t*>(ws);
            tpart = reinterpret_cast<float*>(ws + dec_tail_ctr_bytes());
            nmain = nslabs - rem;
        }
    }
    const dim3 grid((unsigned)(nmain + (P > 1 ? rem * P : 0))), block(NTH);
#define QE_WDEC(SDT_, TB_)                                                                                    \
    wdec_kernel<SDT_, TB_><<<grid, block, kLds, st>>>(w.q, w.s, w.k, x, ldx, m, y, ldy, out, nmain, P, tpart, \
                                                      tctr)
    if (w.sdt == kScaleF16) {
        if (token_blocks(m) == 2) QE_WDEC(kScaleF16, 2);
        else QE_WDEC(kScaleF16, 1);
    } else {
        if (token_blocks(m) == 2) QE_WDEC(kScaleBF16, 2);
        else QE_WDEC(kScaleBF16, 1);
    }
#undef QE_WDEC
    HIP_CHECK(hipGetLastError());
}
