// Exposes the reference's Q8 layout header (src/kernels/q8_layout.h, compiled as it lies under /root/reference) to
// the tests through a C ABI, to check the oracle's restatement (or_q8_pos) against it. Test infrastructure only.
#include "kernels/q8_layout.h"

extern "C" size_t ref_q8_pos(int row, int k, int K) { return q8_pos(row, k, K); }
extern "C" int ref_q8_koff(int i) { return q8_koff(i); }
