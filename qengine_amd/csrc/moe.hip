// MoE grouped INT4 expert layer on one GPU: router -> sort & segment tokens by expert -> grouped gate_up (GLU,
// routing weight) -> grouped down -> fixed-order combine.
//
// Expert weights use the reference's Flash-Next group-record format (flash.h:203-218): every expert's intermediate
// dimension I is split into NGRP = I / 128 groups; record (e, g) is
//   gq [256 rows x H] W4 (gate rows 128 g .. +128 and the matching up rows, GLU-interleaved per 16-row tile)
//   gs fp16 W4 scales, dq [H rows x 128] W4 (down columns 128 g .. +128), ds fp16 W4 scales,
// and records are stored expert-major (record index e * NGRP + g). On one GPU every group is local.
//
// Routing (reference k_topk_rows, flash_kernels.cuh:4351-4399): top-k logits per token, ties to the lower expert
// index, weights exp(l_i - l_max) / sum_sel exp(l_j - l_max). Segmentation (reference k_jobs_pf, :6007-6100) is a
// counting sort whose order inside an expert is ascending (token, k) (the reference's atomics leave it open):
// tokens are processed in chunks of 64 with per-expert 64-bit token masks, so every slot is a pure function of
// the routing. The GLU activations and the per-(token, k) down outputs are stored as fp16 of the value / 16 (the
// reference's fp16 intermediates: its XH activations and kSlotScale slots, :6185,6308,6421-6427); the slots are summed
// in k order (reference k_moe_sum, :6436-6482), so the layer is deterministic. The down projection multiplies the
// fp16 activation by the weights fp16_rn((u - 8) s) on the f16 matrix cores, gate_up the bf16 input by
// bf16_rn((u - 8) s) on the bf16 ones.
//
// Decode (T <= 32): the grouped GEMVs reuse the decode GEMV tile (gemv_impl.hpp) with gathered activation rows,
// jobs = (expert, chunk of <= 2 rows). Prefill: grouped MFMA GEMMs over (expert, 128-row tile) jobs, one block per
// (job, 512 weight rows), the weights dequantized in registers (moe_pf.hip): every expert's weights are read once
// per 128 of its rows.
#include "gemv_impl.hpp"
#include "mfma_tile.hpp"
#include "../../include/qe_kernels.h"

#include <mutex>

namespace {

using namespace qe_gemv;

struct MoeShape {
    int E, topk, H, I, ngrp;
    size_t gg_q, gg_s, gd_q, gd_s, rec;  // bytes of the record parts and of a record
};

MoeShape moe_shape(int E, int topk, int H, int I) {
    MoeShape s;
    s.E = E;
    s.topk = topk;
    s.H = H;
    s.I = I;
    s.ngrp = I / 128;
    s.gg_q = (size_t)256 * H / 2;
    s.gg_s = (size_t)256 * (H / 128) * 2;
    s.gd_q = (size_t)H * 128 / 2;
    s.gd_s = (size_t)H * 2;
    s.rec = s.gg_q + s.gg_s + s.gd_q + s.gd_s;
    return s;
}

__device__ __forceinline__ const char* rec_ptr(const char* recs, const MoeShape& sh, int e, int g) {
    return recs + ((size_t)e * sh.ngrp + g) * sh.rec;
}

// ------------------------------------------------------------------ router: one wave per token
constexpr int kRouteThreads = 256;  // 4 tokens per block
constexpr int kMaxExperts = 1024;

// Routing key of (logit v, expert i): unsigned 64-bit order = (v desc, i asc). High word: the float bits made monotone
// (-0 taken as +0, so equal logits compare equal as floats do), low word: ~i.
__device__ __forceinline__ uint64_t route_key(float v, int i) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b = (b & 0x7FFFFFFFu) == 0u ? 0u : b;
    b = (b & 0x80000000u) != 0u ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint64_t)(~(uint32_t)i);
}
__device__ __forceinline__ float route_key_value(uint64_t k) {
    const uint32_t b = (uint32_t)(k >> 32);
    return __builtin_bit_cast(float, (b & 0x80000000u) != 0u ? (b & 0x7FFFFFFFu) : ~b);
}

// one max step of the wave reduction over a DPP pattern; lanes of rows outside ROWMASK keep their key (every lane
// is written when ROWMASK is 0xF, so no old value has to be kept)
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ void route_step(uint64_t& k) {
    const int hi = (int)(k >> 32), lo = (int)(uint32_t)k;
    int h2, l2;
    if constexpr (ROWMASK == 0xF) {
        h2 = __builtin_amdgcn_mov_dpp(hi, CTRL, 0xF, 0xF, false);
        l2 = __builtin_amdgcn_mov_dpp(lo, CTRL, 0xF, 0xF, false);
    } else {
        h2 = __builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWMASK, 0xF, false);
        l2 = __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWMASK, 0xF, false);
    }
    const uint64_t k2 = ((uint64_t)(uint32_t)h2 << 32) | (uint32_t)l2;
    k = k2 > k ? k2 : k;
}

// Lane l holds the keys of experts l + 64 i (i < PER = ceil(E / 64); missing experts key 0), sorted descending in
// its registers (a bitonic network, no cross-lane dependence). Each of the topk rounds reduces the lanes' heads to the
// wave's largest key by DPP (quad swaps, row rotations by 4 and 8, row broadcasts 15 and 31: lane 63 holds it), and
// the lane whose head it was shifts its list by one: no LDS traffic, no barriers, one 64-bit compare per step. Keys
// are distinct, so the order is total and exactly one lane wins each round.
// one token t by the calling wave; sel / w: the token's topk outputs (global or LDS)
template <int PER>
__device__ __forceinline__ void route_token(const float* __restrict__ logits, int t, int E, int topk, int32_t* sel,
                                            float* w) {
    const int lane = threadIdx.x & 63;
    uint64_t k[PER];
    float v[PER];
    const float* l = logits + (size_t)t * E;
#pragma unroll
    for (int i = 0; i < PER; i++) v[i] = l[lane + 64 * i < E ? lane + 64 * i : E - 1];  // all loads before any use
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = lane + 64 * i;
        k[i] = route_key(v[i], e) & (0ull - (uint64_t)(e < E));  // missing experts: key 0 (no branch)
    }
    // bitonic sort, descending (PER is a power of two)
#pragma unroll
    for (int size = 2; size <= PER; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
            for (int i = 0; i < PER; i++) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const bool swap = desc ? k[j] > k[i] : k[i] > k[j];
                    const uint64_t a = k[i], b = k[j];
                    k[i] = swap ? b : a;
                    k[j] = swap ? a : b;
                }
            }
    uint64_t mine = 0;  // lane r keeps round r's key
    for (int r = 0; r < topk; r++) {
        uint64_t bk = k[0];
        route_step<0xB1>(bk);        // quad_perm [1,0,3,2]
        route_step<0x4E>(bk);        // quad_perm [2,3,0,1]
        route_step<0x124>(bk);       // row_ror:4
        route_step<0x128>(bk);       // row_ror:8: every lane of a row holds the row's largest
        route_step<0x142, 0xA>(bk);  // row_bcast:15 into rows 1 and 3
        route_step<0x143, 0xC>(bk);  // row_bcast:31 into rows 2 and 3: lane 63 holds the wave's largest
        const uint64_t best = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(bk >> 32), 63) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)bk, 63);
        // the winning lane's shift as bit-field merges with an all-ones / zero mask (the empty asm keeps the compiler
        // from rewriting the shift into a register-indexed select over every key)
        uint64_t wm = 0ull - (uint64_t)(k[0] == best);
        asm volatile("" : "+v"(wm));
#pragma unroll
        for (int i = 0; i + 1 < PER; i++) k[i] = (k[i + 1] & wm) | (k[i] & ~wm);
        k[PER - 1] &= ~wm;
        mine = lane == r ? best : mine;
    }
    // weights exp(l_k - l_max) / sum, the sum in k order
    const float v0 = route_key_value(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(mine >> 32), 0) << 32));
    const float ex = expf(route_key_value(mine) - v0);
    float tot = 0.f;
    for (int r = 0; r < topk; r++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
    if (lane < topk) {
        sel[lane] = (int)~(uint32_t)mine;
        w[lane] = ex / tot;
    }
}

template <int PER>
__global__ void __launch_bounds__(kRouteThreads) moe_route_kernel(const float* __restrict__ logits, int T, int E,
                                                                  int topk, int32_t* __restrict__ sel,
                                                                  float* __restrict__ w) {
    const int t = blockIdx.x * (kRouteThreads / 64) + (threadIdx.x >> 6);
    if (t >= T) return;
    route_token<PER>(logits, t, E, topk, sel + (size_t)t * topk, w + (size_t)t * topk);
}

void launch_route(const float* logits, int T, int E, int topk, int32_t* sel, float* w, hipStream_t st) {
    const dim3 grid((T + 3) / 4), block(kRouteThreads);
    const int per = (E + 63) / 64;
    if (per <= 1) moe_route_kernel<1><<<grid, block, 0, st>>>(logits, T, E, topk, sel, w);
    else if (per <= 2) moe_route_kernel<2><<<grid, block, 0, st>>>(logits, T, E, topk, sel, w);
    else if (per <= 4) moe_route_kernel<4><<<grid, block, 0, st>>>(logits, T, E, topk, sel, w);
    else if (per <= 8) moe_route_kernel<8><<<grid, block, 0, st>>>(logits, T, E, topk, sel, w);
    else moe_route_kernel<16><<<grid, block, 0, st>>>(logits, T, E, topk, sel, w);
    HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------ sort & segment
constexpr int kSegThreads = 1024;
constexpr int kSegChunk = 64;  // tokens per chunk (64-bit masks)

// exclusive scans of the expert counts cnt[] (slot offsets pre[], written to off[]) and of their job counts (jobs
// (expert, first row) of `chunk` rows each, njobs), E <= 1024: thread e, wave scans by shuffles, then the 16 wave
// totals. Block of kSegThreads; ends with a barrier.
__device__ void seg_scan_jobs(const int* cnt, int* pre, int E, int chunk, int32_t* __restrict__ off,
                              int32_t* __restrict__ jobs, int32_t* __restrict__ njobs) {
    __shared__ int wa[kSegThreads / 64], wb[kSegThreads / 64], jpre[kMaxExperts + 1];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c0 = tid < E ? cnt[tid] : 0;
    const int j0 = (c0 + chunk - 1) / chunk;
    int a = c0, bsum = j0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int a2 = __shfl_up(a, o), b2 = __shfl_up(bsum, o);
        if (lane >= o) {
            a += a2;
            bsum += b2;
        }
    }
    if (lane == 63) {
        wa[wv] = a;
        wb[wv] = bsum;
    }
    __syncthreads();
    int ao = 0, bo = 0;
    for (int q = 0; q < wv; q++) {
        ao += wa[q];
        bo += wb[q];
    }
    if (tid < E) {
        pre[tid] = ao + a - c0;
        jpre[tid] = bo + bsum - j0;
    }
    if (tid == E - 1) {
        pre[E] = ao + a;
        jpre[E] = bo + bsum;
        *njobs = bo + bsum;
    }
    __syncthreads();
    for (int e = tid; e <= E; e += kSegThreads) off[e] = pre[e];
    for (int e = tid; e < E; e += kSegThreads) {
        const int nj = (cnt[e] + chunk - 1) / chunk;
        for (int j = 0; j < nj; j++) {
            jobs[2 * (jpre[e] + j)] = e;
            jobs[2 * (jpre[e] + j) + 1] = j * chunk;
        }
    }
    __syncthreads();
}

// place the pairs of the 64-token chunk starting at token t0: a pair's slot is base[e] (the expert's first slot
// for this chunk) + the number of earlier tokens of the chunk on the same expert (a 64-bit token mask per expert:
// ascending (token, k) inside an expert, as a pair's experts are distinct). mark[E] in LDS; ends with a barrier.
__device__ void seg_place_chunk(const int32_t* __restrict__ sel, const float* __restrict__ w, int T, int E, int topk,
                                int t0, const int* base, unsigned long long* mark, int32_t* __restrict__ slot_pair,
                                int32_t* __restrict__ slot_tok, float* __restrict__ slot_w, int32_t* __restrict__ inv) {
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kSegThreads) mark[e] = 0ull;
    __syncthreads();
    const int tl = tid / topk;  // token of this thread within the chunk (topk <= 16)
    const int p = t0 * topk + tid;
    const bool act = tl < kSegChunk && t0 + tl < T;
    int e = 0;
    if (act) {
        e = sel[p];
        atomicOr(&mark[e], 1ull << tl);
    }
    __syncthreads();
    if (act) {
        const int slot = base[e] + __popcll(mark[e] & ((1ull << tl) - 1ull));
        slot_pair[slot] = p;
        slot_tok[slot] = t0 + tl;
        slot_w[slot] = w[p];
        inv[p] = slot;
    }
    __syncthreads();
}

// One block (small T, and the qe_moe_segment entry point). out: off [E+1]; per slot: pair (t * topk + k), token,
// weight; inv [pair] = slot; jobs (expert, first row) of `chunk` rows each, njobs
__global__ void __launch_bounds__(kSegThreads) moe_segment_kernel(const int32_t* __restrict__ sel,
                                                                  const float* __restrict__ w, int T, int E, int topk,
                                                                  int chunk, int32_t* __restrict__ off,
                                                                  int32_t* __restrict__ slot_pair,
                                                                  int32_t* __restrict__ slot_tok,
                                                                  float* __restrict__ slot_w, int32_t* __restrict__ inv,
                                                                  int32_t* __restrict__ jobs, int32_t* __restrict__ njobs) {
    __shared__ int cnt[kMaxExperts], pre[kMaxExperts + 1], fill[kMaxExperts];
    __shared__ unsigned long long mark[kMaxExperts];
    const int tid = threadIdx.x;
    const int P = T * topk;
    for (int e = tid; e < E; e += kSegThreads) cnt[e] = 0;
    __syncthreads();
    for (int i = tid; i < P; i += kSegThreads) atomicAdd(&cnt[sel[i]], 1);
    __syncthreads();
    seg_scan_jobs(cnt, pre, E, chunk, off, jobs, njobs);
    for (int e = tid; e < E; e += kSegThreads) fill[e] = pre[e];  // first free slot of each expert
    __syncthreads();
    for (int t0 = 0; t0 < T; t0 += kSegChunk) {
        seg_place_chunk(sel, w, T, E, topk, t0, fill, mark, slot_pair, slot_tok, slot_w, inv);
        for (int e2 = tid; e2 < E; e2 += kSegThreads) fill[e2] += __popcll(mark[e2]);
        __syncthreads();
    }
}

// Decode batches (T <= kDecTokens), one wave segments the routed pairs (ssel / sw: T * topk, LDS or global): its
// LDS operations complete in order, so it needs no barrier. Per-expert counts and 32-bit token masks by LDS atomics,
// the exclusive scans of the counts and job counts with lane l owning experts PER l .. PER l + PER - 1, then each
// pair's slot = the expert's offset + the number of earlier tokens on that expert. Same off / slots / jobs as
// moe_segment_kernel. cnt / pre / mark: LDS [64 PER], cnt and mark zeroed by the caller.
constexpr int kDecTokens = 32;
// decode job records (jdec [job][kJobInts]): expert, first slot, rows m, 0, the token of each row (4 slots), its
// routing weight (float bits; 4 slots), 4 unused: one 64-byte line that the decode kernels load first, in place of the
// dependent loads of jobs, off, slot_tok and slot_w (slots past m are not written: the kernels use row 0 there)
constexpr int kJobInts = 16, kJobRows = 4;
template <int PER>
__device__ void seg_one_wave(const int32_t* ssel, const float* sw, int T, int E, int topk, int chunk, int* cnt,
                             int* pre, unsigned* mark, int32_t* __restrict__ off, int32_t* __restrict__ slot_pair,
                             int32_t* __restrict__ slot_tok, float* __restrict__ slot_w, int32_t* __restrict__ inv,
                             int32_t* __restrict__ jobs, int32_t* __restrict__ njobs, int32_t* __restrict__ jdec) {
    const int lane = threadIdx.x & 63;
    const int P = T * topk;
    for (int p = lane; p < P; p += 64) {
        const int e = ssel[p];
        atomicAdd(&cnt[e], 1);
        atomicOr(&mark[e], 1u << (p / topk));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int c[PER], a = 0, jb = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane * PER + j;
        c[j] = e < E ? cnt[e] : 0;
        a += c[j];
        jb += (c[j] + chunk - 1) / chunk;
    }
    int ai = a, ji = jb;  // inclusive wave scans
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int a2 = __shfl_up(ai, o), j2 = __shfl_up(ji, o);
        ai += lane >= o ? a2 : 0;
        ji += lane >= o ? j2 : 0;
    }
    int run = ai - a, jrun = ji - jb;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane * PER + j;
        if (e < E) {
            pre[e] = run;
            off[e] = run;
            const int nj = (c[j] + chunk - 1) / chunk;
            for (int q = 0; q < nj; q++) {
                jobs[2 * (jrun + q)] = e;
                jobs[2 * (jrun + q) + 1] = q * chunk;
                int32_t* jd = jdec + (size_t)kJobInts * (jrun + q);  // tokens and weights: the pair loop below
                jd[0] = e;
                jd[1] = run + q * chunk;
                jd[2] = min(chunk, c[j] - q * chunk);
                jd[3] = 0;
            }
            cnt[e] = jrun;  // the expert's first job (its count is no longer read)
            run += c[j];
            jrun += nj;
        }
    }
    if (lane == 63) {
        off[E] = ai;
        *njobs = ji;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int p = lane; p < P; p += 64) {
        const int e = ssel[p], t = p / topk;
        const int i = __popc(mark[e] & ((1u << t) - 1u)), slot = pre[e] + i;
        slot_pair[slot] = p;
        slot_tok[slot] = t;
        slot_w[slot] = sw[p];
        inv[p] = slot;
        int32_t* jd = jdec + (size_t)kJobInts * (cnt[e] + i / chunk);
        jd[4 + i % chunk] = t;
        const float wp = sw[p];
        jd[8 + i % chunk] = __builtin_bit_cast(int32_t, wp);
    }
}

// T <= kDecRouteSeg: route and segment in one block of T waves (routing into LDS, one barrier, wave 0 segments;
// the routing is also stored to sel / w, which the fused decode down + combine kernel reads). Measured against
// routing over CUs then a one-wave segmentation (C4 layer, graph replay, same box): T = 5 / 8 32.1 / 41.4 -> 31.6 /
// 40.7 us, T = 12 the same, T = 16 62.3 -> 63.1 us (16 routing waves on one CU), so up to 8 tokens
constexpr int kDecRouteFused = 4;  // routing inside the gate_up blocks (below)
constexpr int kDecRouteSeg = 8;
template <int PER>
__global__ void __launch_bounds__(64 * kDecRouteSeg) moe_route_segment_kernel(
    const float* __restrict__ logits, int T, int E, int topk, int chunk, int32_t* __restrict__ sel,
    float* __restrict__ w, int32_t* __restrict__ off,
    int32_t* __restrict__ slot_pair, int32_t* __restrict__ slot_tok, float* __restrict__ slot_w,
    int32_t* __restrict__ inv, int32_t* __restrict__ jobs, int32_t* __restrict__ njobs, int32_t* __restrict__ jdec) {
    __shared__ int32_t ssel[kDecRouteSeg * 16];
    __shared__ float sw[kDecRouteSeg * 16];
    __shared__ int cnt[64 * PER], pre[64 * PER];
    __shared__ unsigned mark[64 * PER];
    const int tid = threadIdx.x, wv = tid >> 6;
    for (int e = tid; e < E; e += blockDim.x) {
        cnt[e] = 0;
        mark[e] = 0u;
    }
    if (wv < T) route_token<PER>(logits, wv, E, topk, ssel + wv * topk, sw + wv * topk);
    __syncthreads();
    for (int p = tid; p < T * topk; p += blockDim.x) {
        sel[p] = ssel[p];
        w[p] = sw[p];
    }
    if (wv != 0) return;
    seg_one_wave<PER>(ssel, sw, T, E, topk, chunk, cnt, pre, mark, off, slot_pair, slot_tok, slot_w, inv, jobs, njobs,
                      jdec);
}

// kDecRouteSeg < T <= kDecTokens: routed by moe_route_kernel (tokens over CUs: one CU routing 16+ tokens is
// issue-bound), then this one-wave kernel segments sel / w
template <int PER>
__global__ void __launch_bounds__(64) moe_dec_segment_kernel(const int32_t* __restrict__ sel,
                                                             const float* __restrict__ w, int T, int E, int topk,
                                                             int chunk, int32_t* __restrict__ off,
                                                             int32_t* __restrict__ slot_pair,
                                                             int32_t* __restrict__ slot_tok, float* __restrict__ slot_w,
                                                             int32_t* __restrict__ inv, int32_t* __restrict__ jobs,
                                                             int32_t* __restrict__ njobs,
                                                             int32_t* __restrict__ jdec) {
    __shared__ int32_t ssel[kDecTokens * 16];
    __shared__ float sw[kDecTokens * 16];
    __shared__ int cnt[64 * PER], pre[64 * PER];
    __shared__ unsigned mark[64 * PER];
    const int lane = threadIdx.x;
    for (int e = lane; e < E; e += 64) {
        cnt[e] = 0;
        mark[e] = 0u;
    }
    for (int p = lane; p < T * topk; p += 64) {
        ssel[p] = sel[p];
        sw[p] = w[p];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    seg_one_wave<PER>(ssel, sw, T, E, topk, chunk, cnt, pre, mark, off, slot_pair, slot_tok, slot_w, inv, jobs, njobs,
                      jdec);
}

void launch_route_segment(const float* logits, int T, int E, int topk, int chunk, int32_t* sel, float* w, int32_t* off,
                          int32_t* slot_pair, int32_t* slot_tok, float* slot_w, int32_t* inv, int32_t* jobs,
                          int32_t* njobs, int32_t* jdec, hipStream_t st) {
    const int per = (E + 63) / 64;
    if (T > kDecRouteSeg) launch_route(logits, T, E, topk, sel, w, st);
#define QE_RS(PER_)                                                                                                 \
    do {                                                                                                            \
        if (T <= kDecRouteSeg)                                                                                      \
            moe_route_segment_kernel<PER_><<<1, 64 * T, 0, st>>>(logits, T, E, topk, chunk, sel, w, off, slot_pair,   \
                                                                 slot_tok, slot_w, inv, jobs, njobs, jdec);         \
        else                                                                                                        \
            moe_dec_segment_kernel<PER_><<<1, 64, 0, st>>>(sel, w, T, E, topk, chunk, off, slot_pair, slot_tok,      \
                                                           slot_w, inv, jobs, njobs, jdec);                         \
    } while (0)
    if (per <= 1) QE_RS(1);
    else if (per <= 2) QE_RS(2);
    else if (per <= 4) QE_RS(4);
    else if (per <= 8) QE_RS(8);
    else QE_RS(16);
#undef QE_RS
    HIP_CHECK(hipGetLastError());
}

// above this many tokens the layer segments with the three-kernel path below (one block walks the chunks in turn)
constexpr int kSegOneBlockTokens = 256;

// Many tokens: the chunks in parallel. (1) counts per (chunk, expert) -> cntb [B][E]; (2) one block: per expert the
// exclusive scan over the chunks (cntb becomes each chunk's offset inside the expert), the expert offsets and the
// jobs; (3) per chunk: the pairs placed at off[e] + cntb[b][e] + rank. Same slots as the one-block kernel.
__global__ void __launch_bounds__(kSegThreads) moe_seg_count_kernel(const int32_t* __restrict__ sel, int T, int E,
                                                                    int topk, int32_t* __restrict__ cntb) {
    __shared__ int cnt[kMaxExperts];
    const int tid = threadIdx.x, b = blockIdx.x;
    for (int e = tid; e < E; e += kSegThreads) cnt[e] = 0;
    __syncthreads();
    const int p0 = b * kSegChunk * topk, p1 = min(T, (b + 1) * kSegChunk) * topk;
    for (int p = p0 + tid; p < p1; p += kSegThreads) atomicAdd(&cnt[sel[p]], 1);
    __syncthreads();
    for (int e = tid; e < E; e += kSegThreads) cntb[(size_t)b * E + e] = cnt[e];
}

__global__ void __launch_bounds__(kSegThreads) moe_seg_scan_kernel(int nchunk, int E, int chunk,
                                                                   int32_t* __restrict__ cntb,
                                                                   int32_t* __restrict__ off,
                                                                   int32_t* __restrict__ jobs,
                                                                   int32_t* __restrict__ njobs) {
    __shared__ int cnt[kMaxExperts], pre[kMaxExperts + 1];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kSegThreads) {
        int run = 0;
        for (int b0 = 0; b0 < nchunk; b0 += 16) {  // 16 loads in flight, then the running sums
            int v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = b0 + j < nchunk ? cntb[(size_t)(b0 + j) * E + e] : 0;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (b0 + j < nchunk) cntb[(size_t)(b0 + j) * E + e] = run;
                run += v[j];
            }
        }
        cnt[e] = run;
    }
    __syncthreads();
    seg_scan_jobs(cnt, pre, E, chunk, off, jobs, njobs);
}

__global__ void __launch_bounds__(kSegThreads) moe_seg_place_kernel(const int32_t* __restrict__ sel,
                                                                    const float* __restrict__ w, int T, int E,
                                                                    int topk, const int32_t* __restrict__ off,
                                                                    const int32_t* __restrict__ cntb,
                                                                    int32_t* __restrict__ slot_pair,
                                                                    int32_t* __restrict__ slot_tok,
                                                                    float* __restrict__ slot_w,
                                                                    int32_t* __restrict__ inv) {
    __shared__ int base[kMaxExperts];
    __shared__ unsigned long long mark[kMaxExperts];
    const int tid = threadIdx.x, b = blockIdx.x;
    for (int e = tid; e < E; e += kSegThreads) base[e] = off[e] + cntb[(size_t)b * E + e];
    __syncthreads();
    seg_place_chunk(sel, w, T, E, topk, b * kSegChunk, base, mark, slot_pair, slot_tok, slot_w, inv);
}

// ------------------------------------------------------------------ decode grouped GEMVs (gemv_tile)
constexpr int kDecRows = 2;  // rows per decode job

// Matrix-core decode tile (W4, fp16 scales, slices of NG <= 8 groups, MT <= 4 gathered activation rows) behind
// gemv_tile's interface. Lane 16 q + i holds A row i of the 16-row tile (its half of the records (g = i % 8, t = q):
// t = (w >> 4 (i / 8)) & 0x0F0F0F0F) and B column i = activation row i (class-major staged activations, one
// ds_read_b128 per MFMA). The A values are the weight operand bf16_rn((u - 8) s) (gate_up, bf16 activations) or, with
// F16, fp16_rn((u - 8) s) (down, on the fp16 activation), s the row's group scale (the prefill GEMMs' operands too, so
// a token gets the same weights at every T), accumulated across the groups by the MFMAs in fp32. Activations, scales
// and every group's records are loaded before any wait. Returns red in gemv_tile's layout [S][2][MT][16] (half 1
// zero) for rsum().
template <int MT, int NG, bool F16 = false>
__device__ __forceinline__ float* mfma_dec_tile(uint32_t* lds, const uint4* __restrict__ qp,
                                               const uint16_t* __restrict__ sp, const uint32_t* const* xw, int m,
                                               size_t qgs, size_t sgs) {
    static_assert(NG >= 1 && NG <= 8 && MT <= 4, "mfma_dec_tile");
    constexpr int XS = 68;                       // staged activation rows XS dwords apart (disjoint bank groups)
    constexpr int WSZ = NG * MT * XS + NG * 8;   // dwords per wave: xl [NG][MT][XS], scales [NG][16] half
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6, L = threadIdx.x & 63;
    uint32_t* xl = lds + (size_t)w * WSZ;
    uint32_t* sl = xl + NG * MT * XS;
    const uint16_t* sl16 = reinterpret_cast<const uint16_t*>(sl);
    float* red = reinterpret_cast<float*>(lds + (size_t)S * WSZ);  // [S][2][MT][16]
    const int qg = L >> 4, i = L & 15, g = i & 7, sh = 4 * (i >> 3);

    // 1. loads: activation pieces p = L + 64 r (row p / (16 NG), group (p / 16) % NG, 16-byte chunk p % 16; rows
    //    past m re-read row m - 1), the scale dword L (group L / 8), then the records of every group
    constexpr int XL = MT * NG * 16, XR = (XL + 63) / 64;
    u32x4_v xv[XR];
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int p = L + 64 * r < XL ? L + 64 * r : XL - 1;
        const int row = p / (16 * NG), gi = (p >> 4) % NG, ch = p & 15;
        xv[r] = reinterpret_cast<const u32x4_v*>(xw[row < m ? row : m - 1] + gi * 64)[ch];
    }
    const int ls = L < NG * 8 ? L : NG * 8 - 1;
    const uint32_t sraw = reinterpret_cast<const uint32_t*>(sp)[(size_t)(ls >> 3) * sgs + (ls & 7)];
    u32x4_v wv[NG][2];
#pragma unroll
    for (int ii = 0; ii < NG; ii++)
#pragma unroll
        for (int c = 0; c < 2; c++) wv[ii][c] = ld_stream(qp + (size_t)ii * qgs + 32 * c + 4 * g + qg);
    __builtin_amdgcn_sched_barrier(0);

    // 2. staging: scales, activations class-major (x_slot)
    if (L < NG * 8) sl[L] = sraw;
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int p = L + 64 * r;
        if (p < XL) {
            const int row = p / (16 * NG), gi = (p >> 4) % NG, ch = p & 15;
#pragma unroll
            for (int c = 0; c < 4; c++) xl[(gi * MT + row) * XS + x_slot<kFmtW4>(4 * ch + c)] = xv[r][c];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 3. per group: the row's scale, 4 k steps of one MFMA on the dequantized weights (pairs of bytes 0 / 2 and 1 / 3
    //    of the nibble words: k, k + 1 and k + 8, k + 9 of the record's byte order; qe_tile::dq_pair /
    //    dq_f16_pair). bf16: rows g + 8 (lanes i >= 8) keep their high nibbles in place (v = 16 u) and take s / 16;
    //    fp16: those lanes shift their nibbles down. B columns i >= MT read row 0 again (never stored).
    const uint32_t lmask = sh ? 0xF0F0F0F0u : qe_tile::nib_mask();
    f32x4_v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ii = 0; ii < NG; ii++) {
        const uint16_t s_bits = sl16[ii * 16 + i];
        const float s_row = scale_to_f32<kScaleF16>(s_bits);
        const float sv = sh ? s_row * 0.0625f : s_row, bv = sh ? -72.f * s_row : -1032.f * s_row;
        const _Float16 s_h = __builtin_bit_cast(_Float16, s_bits);
        const f16x2_v s2 = {s_h, s_h};
#pragma unroll
        for (int mm = 0; mm < 4; mm++) {
            const u32x4_v b = *reinterpret_cast<const u32x4_v*>(
                &xl[(ii * MT + (i < MT ? i : 0)) * XS + (4 * (mm >> 1) + qg) * 8 + 4 * (mm & 1)]);
            const u32x4_v rec = wv[ii][mm >> 1];
            const int j0 = 2 * (mm & 1);
            u32x4_v a;
            if constexpr (F16) {
                const uint32_t t0 = (rec[j0] >> sh) & qe_tile::nib_mask(), t1 = (rec[j0 + 1] >> sh) & qe_tile::nib_mask();
                a = u32x4_v{qe_tile::dq_f16_pair(qe_tile::magic_f16<qe_tile::kSel02>(t0), s2), qe_tile::dq_f16_pair(qe_tile::magic_f16<qe_tile::kSel13>(t0), s2),
                            qe_tile::dq_f16_pair(qe_tile::magic_f16<qe_tile::kSel02>(t1), s2), qe_tile::dq_f16_pair(qe_tile::magic_f16<qe_tile::kSel13>(t1), s2)};
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_v, a), __builtin_bit_cast(f16x8_v, b),
                                                             acc, 0, 0, 0);
            } else {
                const uint32_t t0 = rec[j0] & lmask, t1 = rec[j0 + 1] & lmask;
                a = u32x4_v{qe_tile::dq_pair(qe_tile::magic_f16<qe_tile::kSel02>(t0), sv, bv), qe_tile::dq_pair(qe_tile::magic_f16<qe_tile::kSel13>(t0), sv, bv),
                            qe_tile::dq_pair(qe_tile::magic_f16<qe_tile::kSel02>(t1), sv, bv), qe_tile::dq_pair(qe_tile::magic_f16<qe_tile::kSel13>(t1), sv, bv)};
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, a), __builtin_bit_cast(bf16x8_v, b),
                                                              acc, 0, 0, 0);
            }
        }
    }
    // 4. lane (q, i < MT) holds rows 4 q .. 4 q + 3 of activation row i
    if (i < MT) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            red[((w * 2) * MT + i) * 16 + 4 * qg + j] = acc[j];
            red[((w * 2 + 1) * MT + i) * 16 + 4 * qg + j] = 0.f;
        }
    }
    __syncthreads();
    return red;
}

// gate_up: block (job, record g * 16 + 16-row tile); S = G / NG waves over K = H
template <int MT, int NG>
__global__ void __launch_bounds__(64 * kMaxWaves) moe_dec_gate_up_kernel(
    const char* __restrict__ recs, MoeShape sh, const uint16_t* __restrict__ x, const int32_t* __restrict__ jdec,
    const int32_t* __restrict__ njobs, uint16_t* __restrict__ act) {
    static_assert(MT <= kJobRows, "moe decode job rows");
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int job = blockIdx.x;
    if (job >= *njobs) return;
    const int4* jr = reinterpret_cast<const int4*>(jdec + (size_t)kJobInts * job);
    const int4 j0 = jr[0], jt = jr[1], jw = jr[2];  // (e, slot0, m, -), tokens, weights
    const int e = j0.x, slot0 = j0.y, m = j0.z;
    const int tok[4] = {jt.x, jt.y, jt.z, jt.w};
    const int wbits[4] = {jw.x, jw.y, jw.z, jw.w};
    const int g = blockIdx.y >> 4, tile = blockIdx.y & 15;
    const int S = blockDim.x >> 6, w = threadIdx.x >> 6;
    const int G = sh.H >> 7, gb = w * NG;
    const char* rp = rec_ptr(recs, sh, e, g);
    const uint4* qp = reinterpret_cast<const uint4*>(rp) + ((size_t)tile * (sh.H >> 6) + 2 * gb) * 32;
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(rp + sh.gg_q) + ((size_t)tile * G + gb) * 16;
    const uint32_t* xw[MT];
#pragma unroll
    for (int r = 0; r < MT; r++)
        xw[r] = reinterpret_cast<const uint32_t*>(x + (size_t)tok[r < m ? r : 0] * sh.H) + gb * 64;
    const float* red = mfma_dec_tile<MT, NG>(lds, qp, sp, xw, m, 64, 8);
    for (int idx = threadIdx.x; idx < m * 8; idx += blockDim.x) {
        const int r = idx >> 3, gg = idx & 7;
        const int wb = wbits[r & 3];
        const float v = silu_f32(rsum<MT>(red, S, r, gg)) * rsum<MT>(red, S, r, gg + 8) * __builtin_bit_cast(float, wb);
        act[(size_t)(slot0 + r) * sh.I + g * 128 + tile * 8 + gg] = f32_to_f16(v * kMoeF16Scale);
    }
}

// T <= kDecRouteFused, T * topk <= 64 (followed by the fused down + combine): routing and gate_up in one launch.
// Every block routes the T tokens itself (route_token into LDS, one token per wave), so no launch waits for a routing
// kernel and nothing is segmented: block (pair p = t * topk + k, record g * 16 + tile) multiplies expert sel[p]'s
// tile by token t's row into act slot p. Block (0, 0) stores sel, w and inv (inv[p] = p) for the down + combine.
// Same arithmetic as moe_dec_gate_up_kernel with one row per job.
template <int PER, int NG>
__global__ void __launch_bounds__(64 * kMaxWaves) moe_dec_route_gate_up_kernel(
    const float* __restrict__ logits, int T, int E, int topk, const char* __restrict__ recs, MoeShape sh,
    const uint16_t* __restrict__ x, int32_t* __restrict__ sel, float* __restrict__ w, int32_t* __restrict__ inv,
    uint16_t* __restrict__ act) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    __shared__ int32_t ssel[kDecRouteFused * 16];
    __shared__ float sw[kDecRouteFused * 16];
    const int S = blockDim.x >> 6, wv = threadIdx.x >> 6;
    for (int tt = wv; tt < T; tt += S) route_token<PER>(logits, tt, E, topk, ssel + tt * topk, sw + tt * topk);
    __syncthreads();
    const int p = blockIdx.x, t = p / topk;
    if (blockIdx.x == 0 && blockIdx.y == 0) {
        for (int q = threadIdx.x; q < T * topk; q += blockDim.x) {
            sel[q] = ssel[q];
            w[q] = sw[q];
            inv[q] = q;
        }
    }
    const int e = ssel[p];
    const int g = blockIdx.y >> 4, tile = blockIdx.y & 15;
    const int G = sh.H >> 7, gb = wv * NG;
    const char* rp = rec_ptr(recs, sh, e, g);
    const uint4* qp = reinterpret_cast<const uint4*>(rp) + ((size_t)tile * (sh.H >> 6) + 2 * gb) * 32;
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(rp + sh.gg_q) + ((size_t)tile * G + gb) * 16;
    const uint32_t* xw[1] = {reinterpret_cast<const uint32_t*>(x + (size_t)t * sh.H) + gb * 64};
    const float* red = mfma_dec_tile<1, NG>(lds, qp, sp, xw, 1, 64, 8);
    if (threadIdx.x < 8) {
        const int gg = threadIdx.x;
        const float v = silu_f32(rsum<1>(red, S, 0, gg)) * rsum<1>(red, S, 0, gg + 8) * sw[p];
        act[(size_t)p * sh.I + g * 128 + tile * 8 + gg] = f32_to_f16(v * kMoeF16Scale);
    }
}

// down: block = one wave = (job, 16-row tile of H), all NGRP records of the expert (K = I = 128 per record): the
// wave streams NGRP KB and no K slice is reduced across waves
template <int MT, int NGRP>
__global__ void __launch_bounds__(64) moe_dec_down_kernel(
    const char* __restrict__ recs, MoeShape sh, const uint16_t* __restrict__ act, const int32_t* __restrict__ jdec,
    const int32_t* __restrict__ njobs, uint16_t* __restrict__ slot_out) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int job = blockIdx.x;
    if (job >= *njobs) return;
    const int4 j0 = *reinterpret_cast<const int4*>(jdec + (size_t)kJobInts * job);  // (e, slot0, m, -)
    const int e = j0.x, slot0 = j0.y, m = j0.z;
    const int tile = blockIdx.y;
    const char* rp = rec_ptr(recs, sh, e, 0);
    const uint4* qp = reinterpret_cast<const uint4*>(rp + sh.gg_q + sh.gg_s) + (size_t)tile * 2 * 32;
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(rp + sh.gg_q + sh.gg_s + sh.gd_q) + (size_t)tile * 16;
    const uint32_t* xw[MT];
#pragma unroll
    for (int r = 0; r < MT; r++)
        xw[r] = reinterpret_cast<const uint32_t*>(act + (size_t)(slot0 + (r < m ? r : 0)) * sh.I);
    // NGRP = 16 (I = 2048): two tiles of 8 groups, each thread keeping its sums of the first (m * 16 <= 64 outputs,
    // one per thread) before the second reuses the LDS
    constexpr int NH = NGRP <= 8 ? NGRP : 8;
    static_assert(NGRP <= 8 || NGRP == 16, "moe decode down: I / 128 in 1..8 or 16");
    const int idx = threadIdx.x, r = idx >> 4, rr = idx & 15;
    const float* red = mfma_dec_tile<MT, NH, true>(lds, qp, sp, xw, m, sh.rec / 16, sh.rec / 4);
    float v = idx < m * 16 ? rsum<MT>(red, 1, r, rr) : 0.f;
    if constexpr (NGRP == 16) {
        __syncthreads();
        const uint32_t* xw2[MT];
#pragma unroll
        for (int q = 0; q < MT; q++) xw2[q] = xw[q] + 8 * 64;  // activations of groups 8..15
        red = mfma_dec_tile<MT, 8, true>(lds, qp + 8 * (sh.rec / 16), sp + 8 * (sh.rec / 2), xw2, m, sh.rec / 16,
                                         sh.rec / 4);
        v += idx < m * 16 ? rsum<MT>(red, 1, r, rr) : 0.f;
    }
    // the activation is act / 16, so v is the slot / 16: stored as is (fp16)
    if (idx < m * 16) slot_out[(size_t)(slot0 + r) * sh.H + tile * 16 + rr] = f32_to_f16(v);
}

// T * topk <= 64 (decode, few pairs), I / 128 <= 8: the down GEMV and the combine in one launch. Block (16-row tile
// of H, token t) of topk waves; wave k multiplies expert sel[t, k]'s tile by act slot inv[t, k] over the whole K = I
// (the tile of moe_dec_down_kernel with one activation row), and 16 lanes sum the waves' fp16-rounded slots (x 16) in
// k order in fp32: the values moe_dec_down_kernel + moe_combine_kernel produce, without the slot_out round trip.
template <int NGRP>
__global__ void __launch_bounds__(64 * 16) moe_dec_down_combine_kernel(
    const char* __restrict__ recs, MoeShape sh, const uint16_t* __restrict__ act, const int32_t* __restrict__ sel,
    const int32_t* __restrict__ inv, int topk, void* __restrict__ out, int out_bf16) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int tile = blockIdx.x, t = blockIdx.y, k = threadIdx.x >> 6;
    const int e = sel[t * topk + k], slot = inv[t * topk + k];
    const char* rp = rec_ptr(recs, sh, e, 0);
    const uint4* qp = reinterpret_cast<const uint4*>(rp + sh.gg_q + sh.gg_s) + (size_t)tile * 2 * 32;
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(rp + sh.gg_q + sh.gg_s + sh.gd_q) + (size_t)tile * 16;
    const uint32_t* xw[1] = {reinterpret_cast<const uint32_t*>(act + (size_t)slot * sh.I)};
    const float* red = mfma_dec_tile<1, NGRP, true>(lds, qp, sp, xw, 1, sh.rec / 16, sh.rec / 4);
    if (threadIdx.x < 16) {
        const int rr = threadIdx.x;
        float a = 0.f;
        for (int kk = 0; kk < topk; kk++) a += 16.f * f16_round(rsum<1>(red + kk * 2 * 16, 1, 0, rr));
        const size_t o = (size_t)t * sh.H + tile * 16 + rr;
        if (out_bf16) reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16(a);
        else reinterpret_cast<float*>(out)[o] = a;
    }
}

// ------------------------------------------------------------------ prefill grouped GEMMs
// (expert, 128-row) jobs: moe_pf_gemm in moe_pf.hip

// ------------------------------------------------------------------ combine: out[t] = sum_k slot_out[inv[t, k]]
// block t, H / 8 threads: each thread's 8 columns of every slot of the token are one 16-byte load, all issued
// before the sums (in k order, fp32)
__global__ void moe_combine_kernel(const uint16_t* __restrict__ slot_out, const int32_t* __restrict__ inv, int topk,
                                   int H, void* __restrict__ out, int out_bf16) {
    const int t = blockIdx.x, c = threadIdx.x * 8;
    int sl[16];
#pragma unroll
    for (int k = 0; k < 16; k++) sl[k] = k < topk ? inv[t * topk + k] : 0;
    u32x4_v v[16];
#pragma unroll
    for (int k = 0; k < 16; k++)
        if (k < topk) v[k] = *reinterpret_cast<const u32x4_v*>(slot_out + (size_t)sl[k] * H + c);
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        if (k < topk) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                a[2 * j] += 16.f * f16_to_f32((uint16_t)v[k][j]);
                a[2 * j + 1] += 16.f * f16_to_f32((uint16_t)(v[k][j] >> 16));
            }
        }
    }
    if (out_bf16) {
        *reinterpret_cast<u32x4_v*>(reinterpret_cast<uint16_t*>(out) + (size_t)t * H + c) =
            u32x4_v{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(a[4], a[5]), pack_bf16x2(a[6], a[7])};
    } else {
        f32x4_v* o = reinterpret_cast<f32x4_v*>(reinterpret_cast<float*>(out) + (size_t)t * H + c);
        o[0] = f32x4_v{a[0], a[1], a[2], a[3]};
        o[1] = f32x4_v{a[4], a[5], a[6], a[7]};
    }
}

// ------------------------------------------------------------------ record packer (load time)
// One thread per 32-bit word of the records (expert-major, record e * NGRP + g). A record is four parts:
//   gq: the group's 256 gate/up rows (record row dr of 16-row tile dr / 16: rows 0..7 of the tile are gate row
//       128 g + 8 tile + j, rows 8..15 the matching up rows I + 128 g + 8 tile + j - 8) in the W4 fragment layout
//       (u32 idx: k-step idx % 4, lane (idx / 4) % 32, chunk idx / 128 = tile * (H / 64) + 64-k chunk; nibble slot
//       s = rowhalf + 2 khalf + 4 odd holds (row 16 tile + lane / 4 + 8 rowhalf, k = 64 c + 16 j + 2 (lane % 4) +
//       8 khalf + odd)), the same map as repack_w4 after the GLU interleave;
//   gs: their fp16 scales [16][H / 128][16];
//   dq: the expert's H down rows restricted to columns 128 g .. 128 g + 127, W4 fragment layout (K = 128);
//   ds: their scales [H / 16][16] (one group).
__device__ __forceinline__ uint32_t pack_nibbles(const int32_t* __restrict__ src, size_t wpr, int row, int k0) {
    // slots: (row, k0) (row + 8, k0) (row, k0 + 8) (row + 8, k0 + 8) (row, k0 + 1) ... ; k0 even, so k0 / k0 + 1
    // share a source word and k0 + 8 / k0 + 9 the next one
    const int w0 = k0 >> 3, sh = 4 * (k0 & 7);
    const uint32_t a0 = (uint32_t)src[(size_t)row * wpr + w0], a1 = (uint32_t)src[(size_t)row * wpr + w0 + 1];
    const uint32_t b0 = (uint32_t)src[(size_t)(row + 8) * wpr + w0], b1 = (uint32_t)src[(size_t)(row + 8) * wpr + w0 + 1];
    uint32_t word = 0;
    const uint32_t ra[2] = {a0, a1}, rb[2] = {b0, b1};
#pragma unroll
    for (int sl = 0; sl < 8; sl++) {
        const int rowhalf = sl & 1, khalf = (sl >> 1) & 1, odd = sl >> 2;
        const uint32_t v = ((rowhalf ? rb[khalf] : ra[khalf]) >> (sh + 4 * odd)) & 15u;
        word |= v << (4 * sl);
    }
    return word;
}

// the gq part with the GLU interleave: source row of record row dr (rows of the expert's [2I] gate/up matrix)
__device__ __forceinline__ int glu_src_row(int dr, int g, int I) {
    const int tile = dr >> 4, j = dr & 15;
    return j < 8 ? 128 * g + 8 * tile + j : I + 128 * g + 8 * tile + (j - 8);
}

__global__ void __launch_bounds__(256) moe_pack_kernel(const int32_t* __restrict__ gu_q, const uint16_t* __restrict__ gu_s,
                                                       const int32_t* __restrict__ dn_q,
                                                       const uint16_t* __restrict__ dn_s, MoeShape sh,
                                                       uint32_t* __restrict__ out) {
    const size_t rw = sh.rec / 4;  // words per record
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)sh.E * sh.ngrp * rw) return;
    const size_t recn = idx / rw;
    const int e = (int)(recn / sh.ngrp), g = (int)(recn % sh.ngrp);
    size_t wi = idx - recn * rw;  // word inside the record
    const int H = sh.H, I = sh.I, GH = H / 128;
    const size_t gq_w = sh.gg_q / 4, gs_w = sh.gg_s / 4, dq_w = sh.gd_q / 4;
    uint32_t word;
    if (wi < gq_w) {
        const int j = (int)(wi & 3), lane = (int)((wi >> 2) & 31);
        const size_t chunk = wi >> 7;
        const int chunks = H >> 6;
        const int r = (int)(chunk / chunks), c = (int)(chunk % chunks);
        const int dr = 16 * r + (lane >> 2);  // record row (rows dr and dr + 8 of the tile)
        const int k0 = 64 * c + 16 * j + 2 * (lane & 3);
        // rows dr and dr + 8 of a tile map to gate row 8 tile + j and up row 8 tile + j: both read their own source
        const int sa = glu_src_row(dr, g, I), sb = glu_src_row(dr + 8, g, I);
        const int32_t* src = gu_q + (size_t)e * 2 * I * (H / 8);
        const size_t wpr = H / 8;
        const int w0 = k0 >> 3, shf = 4 * (k0 & 7);
        const uint32_t ra[2] = {(uint32_t)src[(size_t)sa * wpr + w0], (uint32_t)src[(size_t)sa * wpr + w0 + 1]};
        const uint32_t rb[2] = {(uint32_t)src[(size_t)sb * wpr + w0], (uint32_t)src[(size_t)sb * wpr + w0 + 1]};
        word = 0;
#pragma unroll
        for (int sl = 0; sl < 8; sl++) {
            const int rowhalf = sl & 1, khalf = (sl >> 1) & 1, odd = sl >> 2;
            word |= (((rowhalf ? rb[khalf] : ra[khalf]) >> (shf + 4 * odd)) & 15u) << (4 * sl);
        }
    } else if ((wi -= gq_w) < gs_w) {
        // two consecutive 16-bit scales [tile][gi][i], i even
        const size_t h0 = 2 * wi;
        const int i = (int)(h0 & 15), gi = (int)((h0 >> 4) % GH), r = (int)((h0 >> 4) / GH);
        const uint16_t* ss = gu_s + (size_t)e * 2 * I * GH;
        const uint32_t v0 = ss[(size_t)glu_src_row(16 * r + i, g, I) * GH + gi];
        const uint32_t v1 = ss[(size_t)glu_src_row(16 * r + i + 1, g, I) * GH + gi];
        word = v0 | (v1 << 16);
    } else if ((wi -= gs_w) < dq_w) {
        // down rows, the group's 128 columns: K = 128 (two 64-k chunks per tile)
        const int j = (int)(wi & 3), lane = (int)((wi >> 2) & 31);
        const size_t chunk = wi >> 7;
        const int r = (int)(chunk >> 1), c = (int)(chunk & 1);
        const int row = 16 * r + (lane >> 2);
        const int k0 = 128 * g + 64 * c + 16 * j + 2 * (lane & 3);  // column of the expert's [H][I] down matrix
        word = pack_nibbles(dn_q + (size_t)e * H * (I / 8), I / 8, row, k0);
    } else {
        wi -= dq_w;
        const size_t h0 = 2 * wi;  // scale [tile][i] of rows 16 tile + i, i + 1: column group g
        const int GI = I / 128;
        const uint16_t* ss = dn_s + (size_t)e * H * GI;
        word = (uint32_t)ss[h0 * GI + g] | ((uint32_t)ss[(h0 + 1) * GI + g] << 16);
    }
    out[idx] = word;
}

// ------------------------------------------------------------------ workspace layout
struct MoeWs {
    int32_t *sel, *off, *slot_pair, *slot_tok, *inv, *jobs, *njobs, *cntb, *jdec;
    float *w, *slot_w;
    uint16_t *act, *slot_out;
    size_t bytes;
};

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int max_jobs(int T, int E, int topk, int chunk) { return (T * topk + chunk - 1) / chunk + (E < T * topk ? E : T * topk); }

MoeWs moe_ws(void* base, int T, int E, int topk, int H, int I) {
    MoeWs ws;
    char* p = reinterpret_cast<char*>(base);
    size_t o = 0;
    auto take = [&](size_t b) {
        char* r = p ? p + o : nullptr;
        o += align256(b);
        return r;
    };
    const size_t P = (size_t)T * topk;
    const int mj = max_jobs(T, E, topk, T <= kDecTokens ? kDecRows : kMoePfRows);
    ws.sel = reinterpret_cast<int32_t*>(take(P * 4));
    ws.w = reinterpret_cast<float*>(take(P * 4));
    ws.off = reinterpret_cast<int32_t*>(take((size_t)(E + 1) * 4));
    ws.slot_pair = reinterpret_cast<int32_t*>(take(P * 4));
    ws.slot_tok = reinterpret_cast<int32_t*>(take(P * 4));
    ws.slot_w = reinterpret_cast<float*>(take(P * 4));
    ws.inv = reinterpret_cast<int32_t*>(take(P * 4));
    ws.jobs = reinterpret_cast<int32_t*>(take((size_t)mj * 8));
    ws.njobs = reinterpret_cast<int32_t*>(take(4));
    ws.jdec = reinterpret_cast<int32_t*>(take(T <= kDecTokens ? (size_t)mj * kJobInts * 4 : 0));
    ws.cntb = reinterpret_cast<int32_t*>(take((size_t)((T + kSegChunk - 1) / kSegChunk) * E * 4));
    ws.act = reinterpret_cast<uint16_t*>(take(P * I * 2));
    ws.slot_out = reinterpret_cast<uint16_t*>(take(P * H * 2));
    ws.bytes = o;
    return ws;
}

void moe_check(int T, int E, int topk, int H, int I) {
    CHECK(T >= 1 && E >= 1 && E <= kMaxExperts && topk >= 1 && topk <= 16 && topk <= E, "moe T %d E %d topk %d", T, E,
          topk);
    CHECK(H % 512 == 0 && H / 128 <= 4 * kMaxWaves && I % 128 == 0 && (I / 128 <= 8 || I / 128 == 16), "moe H %d I %d",
          H, I);
}

}  // namespace

extern "C" {

void qe_moe_route(const float* logits, int T, int E, int topk, int32_t* sel, float* w, void* stream) {
    CHECK(T >= 1 && E >= 1 && E <= kMaxExperts && topk >= 1 && topk <= 32 && topk <= E, "moe_route T %d E %d topk %d",
          T, E, topk);
    launch_route(logits, T, E, topk, sel, w, reinterpret_cast<hipStream_t>(stream));
}

void qe_moe_segment(const int32_t* sel, const float* w, int T, int E, int topk, int chunk, int32_t* off,
                    int32_t* slot_pair, int32_t* slot_tok, float* slot_w, int32_t* inv, int32_t* jobs, int32_t* njobs,
                    void* stream) {
    CHECK(T >= 1 && E >= 1 && E <= kMaxExperts && topk >= 1 && topk <= 16 && chunk >= 1, "moe_segment T %d E %d", T, E);
    moe_segment_kernel<<<1, kSegThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        sel, w, T, E, topk, chunk, off, slot_pair, slot_tok, slot_w, inv, jobs, njobs);
    HIP_CHECK(hipGetLastError());
}

size_t qe_moe_workspace_bytes(int T, int E, int topk, int H, int I) {
    moe_check(T, E, topk, H, I);
    return moe_ws(nullptr, T, E, topk, H, I).bytes;
}

size_t qe_moe_record_bytes(int H, int I) { return moe_shape(1, 1, H, I).rec * (size_t)(I / 128); }

}  // extern "C"

namespace {

// the fused decode down + combine (T * topk <= 64, I / 128 <= 8)
void launch_down_combine(const char* recs, const MoeShape& sh, const uint16_t* act, const int32_t* sel,
                         const int32_t* inv, int T, int topk, int H, void* out, int flags, hipStream_t st) {
#define QE_DOWN_COMBINE(NGRP_)                                                                                 \
    moe_dec_down_combine_kernel<NGRP_><<<dim3(H / 16, T), 64 * topk, gemv_lds_bytes<1, NGRP_, true>(topk), st>>>( \
        recs, sh, act, sel, inv, topk, out, (flags & QE_OUT_BF16) ? 1 : 0)
    switch (sh.ngrp) {
        case 1: QE_DOWN_COMBINE(1); break;
        case 2: QE_DOWN_COMBINE(2); break;
        case 3: QE_DOWN_COMBINE(3); break;
        case 4: QE_DOWN_COMBINE(4); break;
        case 5: QE_DOWN_COMBINE(5); break;
        case 6: QE_DOWN_COMBINE(6); break;
        case 7: QE_DOWN_COMBINE(7); break;
        default: QE_DOWN_COMBINE(8); break;
    }
#undef QE_DOWN_COMBINE
    HIP_CHECK(hipGetLastError());
}

// the layer on a workspace of moe_ws(T, ...).bytes at `workspace` (checked by the callers)
void moe_run(const float* logits, const uint16_t* x, const void* records, int T, int E, int topk, int H, int I,
             void* out, int flags, void* workspace, hipStream_t st) {
    const MoeShape sh = moe_shape(E, topk, H, I);
    const MoeWs ws = moe_ws(workspace, T, E, topk, H, I);
    CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)workspace & 255) == 0,
          "moe x / out 16-byte, workspace 256-byte alignment");
    const char* recs = reinterpret_cast<const char*>(records);
    const bool decode = T <= kDecTokens;
    const int chunk = decode ? kDecRows : kMoePfRows;
    const int mj = max_jobs(T, E, topk, chunk);

    // a few decode tokens: routing + gate_up in one launch, then the fused down + combine (two launches in all)
    if (T <= kDecRouteFused && T * topk <= 64 && sh.ngrp <= 8) {
        const int G = H / 128, per = (E + 63) / 64;
        const int ng = (G % 2 == 0 && G / 2 <= kMaxWaves) ? 2 : (G % 4 == 0 && G / 4 <= kMaxWaves) ? 4 : 8;
        CHECK(G % ng == 0 && G / ng <= kMaxWaves, "moe decode H %d", H);
        const size_t lds = ng == 2 ? gemv_lds_bytes<1, 2, true>(G / 2)
                           : ng == 4 ? gemv_lds_bytes<1, 4, true>(G / 4)
                                     : gemv_lds_bytes<1, 8, true>(G / 8);
        const dim3 grid((unsigned)(T * topk), (unsigned)(sh.ngrp * 16)), block((unsigned)(64 * (G / ng)));
#define QE_RGU(PER_, NG_)                                                                                     \
    moe_dec_route_gate_up_kernel<PER_, NG_><<<grid, block, lds, st>>>(logits, T, E, topk, recs, sh, x, ws.sel, ws.w, \
                                                                       ws.inv, ws.act)
#define QE_RGU_NG(PER_)                      \
    do {                                     \
        if (ng == 2) QE_RGU(PER_, 2);        \
        else if (ng == 4) QE_RGU(PER_, 4);   \
        else QE_RGU(PER_, 8);                \
    } while (0)
        if (per <= 1) QE_RGU_NG(1);
        else if (per <= 2) QE_RGU_NG(2);
        else if (per <= 4) QE_RGU_NG(4);
        else if (per <= 8) QE_RGU_NG(8);
        else QE_RGU_NG(16);
#undef QE_RGU_NG
#undef QE_RGU
        HIP_CHECK(hipGetLastError());
        launch_down_combine(recs, sh, ws.act, ws.sel, ws.inv, T, topk, H, out, flags, st);
        return;
    }
    if (T > kDecTokens) launch_route(logits, T, E, topk, ws.sel, ws.w, st);
    if (T <= kDecTokens) {
        launch_route_segment(logits, T, E, topk, chunk, ws.sel, ws.w, ws.off, ws.slot_pair, ws.slot_tok, ws.slot_w,
                             ws.inv, ws.jobs, ws.njobs, ws.jdec, st);
    } else if (T > kSegOneBlockTokens) {
        const int nchunk = (T + kSegChunk - 1) / kSegChunk;
        moe_seg_count_kernel<<<nchunk, kSegThreads, 0, st>>>(ws.sel, T, E, topk, ws.cntb);
        HIP_CHECK(hipGetLastError());
        moe_seg_scan_kernel<<<1, kSegThreads, 0, st>>>(nchunk, E, chunk, ws.cntb, ws.off, ws.jobs, ws.njobs);
        HIP_CHECK(hipGetLastError());
        moe_seg_place_kernel<<<nchunk, kSegThreads, 0, st>>>(ws.sel, ws.w, T, E, topk, ws.off, ws.cntb, ws.slot_pair,
                                                             ws.slot_tok, ws.slot_w, ws.inv);
    } else {
        moe_segment_kernel<<<1, kSegThreads, 0, st>>>(ws.sel, ws.w, T, E, topk, chunk, ws.off, ws.slot_pair,
                                                      ws.slot_tok, ws.slot_w, ws.inv, ws.jobs, ws.njobs);
    }
    HIP_CHECK(hipGetLastError());
    if (decode) {
        const int G = H / 128;
        // gate_up K slices: 2-group slices (more, shorter waves) while the pairs are few (<= 64: a latency-bound
        // launch), else 4 (measured, H = 2048: T = 1 21.0 -> 19.6 us at 2 groups, T = 16 58.4 -> 64.5 us)
        const bool few = T * topk <= 64;
        const int ng = (few && G % 2 == 0 && G / 2 <= kMaxWaves) ? 2 : (G % 4 == 0 && G / 4 <= kMaxWaves) ? 4 : 8;
        CHECK(G % ng == 0 && G / ng <= kMaxWaves, "moe decode H %d", H);
        const size_t lds_gu = ng == 2   ? gemv_lds_bytes<kDecRows, 2, true>(G / 2)
                              : ng == 4 ? gemv_lds_bytes<kDecRows, 4, true>(G / 4)
                                        : gemv_lds_bytes<kDecRows, 8, true>(G / 8);
        if (ng == 2)
            moe_dec_gate_up_kernel<kDecRows, 2><<<dim3(mj, sh.ngrp * 16), 64 * (G / 2), lds_gu, st>>>(
                recs, sh, x, ws.jdec, ws.njobs, ws.act);
        else if (ng == 4)
            moe_dec_gate_up_kernel<kDecRows, 4><<<dim3(mj, sh.ngrp * 16), 64 * (G / 4), lds_gu, st>>>(
                recs, sh, x, ws.jdec, ws.njobs, ws.act);
        else
            moe_dec_gate_up_kernel<kDecRows, 8><<<dim3(mj, sh.ngrp * 16), 64 * (G / 8), lds_gu, st>>>(
                recs, sh, x, ws.jdec, ws.njobs, ws.act);
        HIP_CHECK(hipGetLastError());
        if (few && sh.ngrp <= 8) {
            launch_down_combine(recs, sh, ws.act, ws.sel, ws.inv, T, topk, H, out, flags, st);
            return;
        }
#define QE_DOWN(NGRP_)                                                                                         \
    moe_dec_down_kernel<kDecRows, NGRP_><<<dim3(mj, H / 16), 64, gemv_lds_bytes<kDecRows, NGRP_, true>(1), st>>>( \
        recs, sh, ws.act, ws.jdec, ws.njobs, ws.slot_out)
        switch (sh.ngrp) {
            case 1: QE_DOWN(1); break;
            case 2: QE_DOWN(2); break;
            case 3: QE_DOWN(3); break;
            case 4: QE_DOWN(4); break;
            case 5: QE_DOWN(5); break;
            case 6: QE_DOWN(6); break;
            case 7: QE_DOWN(7); break;
            case 8: QE_DOWN(8); break;
            case 16: QE_DOWN(16); break;
            default: CHECK(false, "moe decode: I = %d (I / 128 in 1..8 or 16)", I);
        }
#undef QE_DOWN
        HIP_CHECK(hipGetLastError());
    } else {
        MoePfArgs pa;
        pa.recs = recs;
        pa.rec = sh.rec;
        pa.gg_q = sh.gg_q;
        pa.gg_s = sh.gg_s;
        pa.gd_q = sh.gd_q;
        pa.ngrp = sh.ngrp;
        pa.H = H;
        pa.I = I;
        pa.off = ws.off;
        pa.slot_tok = ws.slot_tok;
        pa.slot_w = ws.slot_w;
        pa.jobs = ws.jobs;
        pa.njobs = ws.njobs;
        pa.max_jobs = mj;
        pa.a = x;
        pa.out = ws.act;
        moe_pf_gemm(1, pa, st);
        pa.a = ws.act;
        pa.out = ws.slot_out;
        moe_pf_gemm(2, pa, st);
    }
    moe_combine_kernel<<<T, H / 8, 0, st>>>(ws.slot_out, ws.inv, topk, H, out, (flags & QE_OUT_BF16) ? 1 : 0);
    HIP_CHECK(hipGetLastError());
}

// ---- the allocation-free variant's workspace: one file-scope device array per GPU (each device that loads the
// library holds its own copy until the process ends). Host code never uses the array's name as a device address:
// its address on each device comes from hipGetSymbolAddress, taken once per device with that device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[QE_MOE_SCRATCH_BYTES];

// address of `scratch` on the current device (resolved and kept on the device's first use)
void* moe_scratch_ptr() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    CHECK(dev >= 0 && dev < kMaxDevices, "device %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        CHECK(p != nullptr && ((uintptr_t)p & 255) == 0, "scratch address");
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

extern "C" {

void qe_moe_w4(const float* logits, const uint16_t* x, const void* records, int T, int E, int topk, int H, int I,
               void* out, int flags, void* workspace, size_t ws_bytes, void* stream) {
    moe_check(T, E, topk, H, I);
    const size_t need = moe_ws(nullptr, T, E, topk, H, I).bytes;
    CHECK(workspace && ws_bytes >= need, "moe workspace %zu < %zu bytes", ws_bytes, need);
    moe_run(logits, x, records, T, E, topk, H, I, out, flags, workspace, reinterpret_cast<hipStream_t>(stream));
}

void qe_moe_w4_noalloc(const float* logits, const uint16_t* x, const void* records, int T, int E, int topk, int H,
                       int I, void* out, int flags, void* stream) {
    moe_check(T, E, topk, H, I);
    const size_t need = moe_ws(nullptr, T, E, topk, H, I).bytes;
    CHECK(need <= (size_t)QE_MOE_SCRATCH_BYTES,
          "qe_moe_w4_noalloc: T %d E %d topk %d H %d I %d needs %zu bytes of workspace, above the %d-byte scratch",
          T, E, topk, H, I, need, QE_MOE_SCRATCH_BYTES);
    moe_run(logits, x, records, T, E, topk, H, I, out, flags, moe_scratch_ptr(), reinterpret_cast<hipStream_t>(stream));
}

// compressed-tensors experts -> group records. gate_up: int32 [E][2I][H/8] (rows gate 0..I then up 0..I), fp16
// scales [E][2I][H/128]; down: int32 [E][H][I/8], fp16 scales [E][H][I/128]. The reference's loader does the same
// per group (flash.cu:1555-1611): gather the group's gate/up rows, GLU-interleave, repack; gather the group's down
// columns, repack. Here one kernel writes every 32-bit word of every record straight from the source tensors
// (moe_pack_kernel): no staging copies, no allocation, no host synchronization (stream-ordered like any kernel).
void qe_moe_pack_w4(const int32_t* gu_q, const uint16_t* gu_s, const int32_t* dn_q, const uint16_t* dn_s, int E, int H,
                    int I, void* records, void* stream) {
    moe_check(1, E, 1, H, I);
    const MoeShape sh = moe_shape(E, 1, H, I);
    const size_t words = (size_t)E * sh.ngrp * (sh.rec / 4);
    const unsigned blocks = (unsigned)((words + 255) / 256);
    CHECK(sh.rec % 4 == 0 && blocks > 0, "moe_pack: record of %zu bytes", sh.rec);
    moe_pack_kernel<<<blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(gu_q, gu_s, dn_q, dn_s, sh,
                                                                               reinterpret_cast<uint32_t*>(records));
    HIP_CHECK(hipGetLastError());
}

}  // extern "C"
