// Host launchers of the FT kernels (see ft_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "optim.hpp"

namespace tatara {

struct FtForwardArgs {
    int mode;  // 0 raw sum, 1 LayerStack pairwise post, 2 Simple concat post
    const float* W;
    const int32_t* idx_stm;
    const int32_t* idx_nstm;
    const int32_t* nnz;
    const int32_t* schedule;  // [n_persp][batch] or null (identity order)
    const float* bias;
    float* out_stm;
    float* out_nstm;
    float* combined;
    uint32_t batch, ft_out, cols, max_active, n_persp;
    float scale;
};

struct OccurrenceSortArgs {
    const int32_t* idx_stm;
    const int32_t* idx_nstm;
    const int32_t* nnz;
    uint32_t batch, max_active, cols;
    uint32_t* keys_in;   // [2*batch*max_active]
    uint32_t* vals_in;
    uint32_t* keys_out;
    uint32_t* vals_out;  // sorted dft row ids
    uint32_t* offsets;   // [2*cols + 2]; key k occupies [offsets[k], offsets[k+1])
    void* temp;
    size_t temp_bytes;
};

struct FtGradArgs {
    // dft rows: element (row r, column c) lives at
    // dft[r * dft_row_stride + (c / 256) * dft_chunk_stride + c % 256], r = persp*batch + pos.
    // Row-major [2][batch][ft_out]: (ft_out, 256); chunk-major
    // [ceil(ft_out/256)][2*batch][256]: (256, 2*batch*256).
    const float* dft;
    uint64_t dft_row_stride, dft_chunk_stride;
    const uint32_t* occ_vals;  // sorted dft row ids
    const uint32_t* occ_off;   // offsets by key 2*f+p
    float *w, *m, *v, *slow;
    float* grad;               // gradient per row (required with a factorizer)
    uint32_t ft_out;
    uint32_t rows;             // real FT rows (ft_in)
    int32_t apply_update;      // 0: only write gradients
    OptScalars opt;
};

// Columns per dft chunk in the chunk-major layout (one wave of float4 lanes).
constexpr uint32_t kDftChunk = 256;

int32_t launch_ft_forward(const FtForwardArgs& a, hipStream_t stream);
int32_t launch_king_block_keys(const int32_t* idx_stm, const int32_t* idx_nstm, const int32_t* nnz,
                               uint8_t* keys, uint32_t batch, uint32_t max_active, uint32_t cols,
                               uint32_t piece_inputs, uint32_t n_bins, hipStream_t stream);
uint32_t occurrence_key_bits(uint32_t cols);
size_t occurrence_sort_temp_bytes(uint64_t n_items, uint32_t cols);
int32_t launch_occurrence_sort(const OccurrenceSortArgs& a, hipStream_t stream);
int32_t launch_ft_grad_update(const FtGradArgs& a, hipStream_t stream);
int32_t launch_ft_virtual_fold(const FtGradArgs& a, uint32_t piece_inputs, float* comb,
                               hipStream_t stream);
int32_t launch_ft_fold(const float* w, float* comb, uint32_t ft_in, uint32_t ft_out,
                       uint32_t piece_inputs, hipStream_t stream);
int32_t launch_ft_reduce(float* grad, uint32_t ft_in, uint32_t ft_out, uint32_t piece_inputs,
                         hipStream_t stream);
int32_t launch_radam(float* w, float* m, float* v, float* g, float* slow, uint64_t n,
                     const OptScalars& s, hipStream_t stream);
int32_t launch_lerp(float* w, float* slow, uint64_t n, float alpha, hipStream_t stream);

}  // namespace tatara
