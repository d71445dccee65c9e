// Prefill GEMM choices: the measured (tile configuration, split) per matrix shape and token bucket, per device, in
// memory and optionally in a file (the reference's persisted tuner, src/kernels/gemm.cu:4116-4348: a tuned choice
// changes the rounding of everything downstream, so a later process reads the stored choice instead of timing).
#pragma once
#include "qe_api.hpp"

struct GemmChoice {
    int cfg = 0;  // 0: 256 x 256 tiles, 1: 256 x 128
    int ks = 1;   // K ranges of the last partial round's tiles (1: no split)
};
struct GemmKey {
    int fmt, n, k, bucket, glu;
    bool operator<(const GemmKey& o) const {
        if (fmt != o.fmt) return fmt < o.fmt;
        if (n != o.n) return n < o.n;
        if (k != o.k) return k < o.k;
        if (bucket != o.bucket) return bucket < o.bucket;
        return glu < o.glu;
    }
};
// power of two >= t (at least 64): token counts of one bucket share a choice
int gemm_bucket(int t);
// the current device's table
bool gemm_table_find(const GemmKey& key, GemmChoice& ch);
void gemm_table_add(const GemmKey& key, const GemmChoice& ch);
void gemm_table_clear();
size_t gemm_table_size();
// persist the table at `path` (nullptr or "": in memory only): entries of this device and build already in the file
// are loaded, every new choice rewrites the file (a temporary file renamed over it). A file written by another
// build or for other candidates is ignored and replaced.
void gemm_tune_file(const char* path);
