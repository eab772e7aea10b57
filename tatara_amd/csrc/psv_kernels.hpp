// Host launchers of the PSV decode / feature extraction kernels (see psv_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tatara {

constexpr int kPsvThreads = 64;  // records per workgroup

// FeatureSetSpec of the five public feature sets
// (crates/shogi-features/src/feature_set.rs:103-185).
struct FeatureSetShape {
    int32_t king_buckets, piece_inputs, max_active;
    int32_t emit_king, fold_enemy, mirror;
    uint32_t feature_hash;
};
int32_t feature_set_shape(int32_t feature_set, FeatureSetShape& s);

struct PsvArgs {
    const uint8_t* psv;  // [n][40]
    uint32_t n;
    int32_t piece_inputs, max_active, emit_king, fold_enemy, mirror;
    int32_t bucket_mode;  // 0 none (bucket 0), 1 kingrank9, 2 KP-absolute progress
    int32_t num_buckets;
    const float* weights;  // [81 * 1548] progress weights (mode 2)
    int32_t* stm;          // [n][max_active], -1 past nnz
    int32_t* nstm;
    int32_t* nnz;
    int32_t* bucket;       // optional
    float* score;
    float* wdl;
    float* progress;       // optional, mode 2
};

int32_t launch_psv_to_batch(const PsvArgs& a, hipStream_t stream);
// expf evaluated as the reference's CPU path does (glibc's method).
int32_t launch_expf(const float* x, float* y, uint64_t n, hipStream_t stream);

}  // namespace tatara
