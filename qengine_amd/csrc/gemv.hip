// Decode GEMV / skinny GEMM host side: K slicing policy, CU count, workspace init (kernels: gemv_impl.hpp,
// instantiated in gemv_w4.hip and gemv_w8.hip).
#include "gemv_impl.hpp"

#include <algorithm>
#include <atomic>

namespace {
// CU count per device index (devices may differ, e.g. under compute partitioning); 0 = not queried yet
constexpr int kMaxCuDev = 64;
std::atomic<int> g_cus[kMaxCuDev];
QeConfig g_cfg;
}

const QeConfig& qe_config() { return g_cfg; }
void qe_config_set(const QeConfig& c) {
    CHECK(c.skinny_min_m >= 1 && c.skinny_min_m <= kMaxGemvRows + 1 && c.w8_mfma_min_m >= 0 &&
              c.w8_mfma_min_m <= kMaxGemvRows + 1 && (c.batch_invariant == 0 || c.batch_invariant == 1) &&
              (c.gemm_tune == 0 || c.gemm_tune == 1) && (c.gemm_h16 == 0 || c.gemm_h16 == 1),
          "config skinny_min_m %d w8_mfma_min_m %d batch_invariant %d gemm_tune %d gemm_h16 %d", c.skinny_min_m,
          c.w8_mfma_min_m, c.batch_invariant, c.gemm_tune, c.gemm_h16);
    g_cfg = c;
}

// the current device's CU count (every grid-sizing decision uses it)
int qe_num_cus() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    CHECK(dev >= 0 && dev < kMaxCuDev, "device %d", dev);
    int c = g_cus[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        HIP_CHECK(hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev));
        c = c > 0 ? c : 256;
        g_cus[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

// The decode GEMV keeps no device workspace (its K slices are reduced in LDS); the entry point stays for the
// reference's calling convention (gemv_workspace_init once per device before any graph capture).
void gemv_workspace_init() { qe_num_cus(); }

namespace qe_gemv {

// Aim for about 20 resident waves per CU (1 KB loads in flight per wave and group), with slices of 8, 4 or 2
// groups that divide K evenly and at most 8 waves per block; otherwise uneven slices of <= 16 groups.
Slicing gemv_slicing(int n, int k) {
    const int tiles = n / 16, G = k / 128;
    const int s_target = std::max(1, (20 * qe_num_cus() + tiles - 1) / tiles);
    int best = 0;
    for (int ng : {8, 4, 2}) {
        if (G % ng || G / ng > kMaxWaves) continue;
        if (best == 0) best = ng;                     // fewest waves that fit
        if (G / ng >= s_target) { best = ng; break; }  // largest slice reaching the target
        best = ng;                                     // else keep the one with the most waves
    }
    if (best > 0) return {best, G / best};
    // uneven: up to 12 waves toward the target (skinny kernel, K = 17408, 136 groups: N = 5120 m = 2 / 8 16.2 / 24.5 ->
    // 15.6 / 21.7 us at 12 slices instead of 9; N = 2048 12.8 -> 10.8 us at m = 2), 16 where the tiles fit one round
    // of CUs (N = 2048, K = 17408, m = 1 (batch_invariant) / 2 / 4 / 8 / 16: 10.7 / 10.9 / 10.9 / 11.7 / 15.9 -> 9.7 /
    // 9.8 / 9.8 / 11.6 / 16.0 us; N = 3072 and 4096 alike, m = 8 up to 5 % slower; the VALU GEMV 2-8 % faster)
    const int cap = tiles <= qe_num_cus() ? 16 : 12;
    int S = std::max((G + kGenericNG - 1) / kGenericNG, std::min(s_target, std::min(G, cap)));
    CHECK(S <= kMaxWavesGeneric, "gemv: k = %d above the supported 32768", k);
    return {0, S};
}

// K slicing of the matrix-core decode kernels (m = 1 and the skinny GEMM): groups per wave NG in {2, 4, 5, 8, 10}
// dividing K / 128 with at most 8 waves per block; the smallest NG whose grid stays within ~34 waves per CU (about
// what can be resident at 8 waves per SIMD): more, shorter waves hide the per-group latencies best, as long as they
// need not wait for a second round of wave slots. 0 when none divides. Depends on (n, k) only.
int decode_groups(int n, int k) {
    const int tiles = n / 16, G = k / 128;
    int pick = 0;
    for (int ng : {10, 8, 5, 4, 2}) {
        if (G % ng || G / ng > kMaxWaves) continue;
        if (pick != 0 && (long)tiles * (G / ng) > 34L * qe_num_cus()) break;
        pick = ng;
    }
    return pick;
}

}  // namespace qe_gemv
