// Host launchers of the FT kernels (see ft_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "optim.hpp"

namespace tatara {

// 16-bit tables and activations are IEEE binary16 values held as uint16_t
// (the --ft-fp16 / --ft-fp16-out / --fp16-opt-state modes of the reference,
// bins/nnue_train/src/trainer_common.rs:49-61).

// Layout of a forward table (the factorizer's folded table): row-major
// [rows][ft_out], or slice-major for the pairwise block-resident gather:
// [king block][slice][feature][64 bytes], a slice being the columns one
// ft_forward_block_kernel workgroup holds (2 x QC columns of each half;
// QC = 4 for f32, 8 for f16), so a workgroup stages its slice as one
// contiguous run.
enum FtTableLayout : int { kTableRows = 0, kTablePairSlices = 1 };

struct FtForwardArgs {
    int mode;  // 0 raw sum, 1 LayerStack pairwise post, 2 Simple concat post
    const float* W;
    const uint16_t* W16;  // f16 forward table, read instead of W when non-null
    const int32_t* idx_stm;
    const int32_t* idx_nstm;
    const int32_t* nnz;
    const int32_t* schedule;  // [n_persp][batch] or null (identity order)
    const float* bias;
    float* out_stm;
    float* out_nstm;
    uint16_t* out_stm16;  // pairwise mode: f16 raw sums, written instead of out_* when non-null
    uint16_t* out_nstm16;
    float* combined;
    uint16_t* combined16;  // pairwise mode: `combined` rounded to f16, written instead when non-null
    uint32_t batch, ft_out, cols, max_active, n_persp;
    float scale;
    // Optional king-block statement of the schedule: bins [2*n_blocks + 1]
    // (perspective-major, as FtBlockScan::sched_start) and the block width.
    // When set (and the shape fits), the gather holds each block's table
    // slice in LDS (ft_forward_block_kernel) instead of reading rows through
    // the vector memory path.
    const uint32_t* sched_start;
    uint32_t n_blocks, piece_inputs;
    // ... with the per-slot LDS offsets and out-of-block row flags of
    // launch_king_block_keys (both required for the LDS-resident gather)
    const uint32_t* slot_off;
    const uint8_t* row_bad;
    int w_layout;  // FtTableLayout of W / W16 (slice-major only with the LDS-resident gather)
};

// Whether the LDS-resident forward serves this shape (mode, table type,
// ft_out, piece_inputs, max_active); otherwise the row gather runs.
bool ft_forward_block_ok(int mode, bool f16_table, uint32_t ft_out, uint32_t piece_inputs, uint32_t max_active);
// Slots per row of FtForwardArgs::slot_off (max_active rounded up to 40 or 48;
// the padding holds the zero row's offset).
uint32_t ft_block_slot_stride(uint32_t max_active);

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
    // The sort is stable LSD passes of 8 bits (the bin-sort kernels) with
    // scratch radix_hist [256 * binsort_tiles(2*batch*max_active)] and
    // radix_count [256], or, when those are null, temp
    // (occurrence_sort_temp_bytes).
    void* temp;
    size_t temp_bytes;
    // Device gate: when set, the sort runs only if *run_if != 0, so a step
    // can queue it without the host learning whether it is needed.
    const uint32_t* run_if;
    uint32_t* radix_hist;
    uint32_t* radix_count;
};

struct FtGradArgs {
    // dft rows: element (row r, column c) lives at
    // dft[r * dft_row_stride + (c / 256) * dft_chunk_stride + c % 256], r = persp*batch + pos.
    // Row-major [2][batch][ft_out]: (ft_out, 256); chunk-major
    // [ceil(ft_out/256)][2*batch][256]: (256, 2*batch*256).
    const float* dft;
    const uint16_t* dft16;     // f16 dft (values scaled by 1 / dft_inv_scale), read instead of dft
    float dft_inv_scale;
    uint64_t dft_row_stride, dft_chunk_stride;
    const uint32_t* occ_vals;  // sorted dft row ids
    const uint32_t* occ_off;   // offsets by key 2*f+p
    float *w, *m, *v, *slow;
    uint16_t *m16, *v16;       // f16 moments stored x m_scale / x v_scale, used instead of m / v
    float m_scale, v_scale;
    uint16_t* mirror16;        // f16 copy of every updated real row (unfactorized f16 forward), or null
    float* grad;               // gradient per row (required with a factorizer)
    uint32_t ft_out;
    uint32_t rows;             // real FT rows (ft_in)
    int32_t apply_update;      // 0: only write gradients
    OptScalars opt;
    const uint32_t* run_if;    // when non-null the kernel does nothing unless *run_if != 0
};

// The block-scan FT backward (ft_grad_scan_kernel): the forward's king-block
// schedule, per-row hit masks and the flag that hands a step to the
// occurrence-list kernel.
struct FtBlockScan {
    const int32_t* idx_stm;
    const int32_t* idx_nstm;
    const int32_t* nnz;
    const int32_t* schedule;      // [2*batch] positions grouped by (perspective, block), ascending
    const uint32_t* sched_start;  // [2*n_blocks + 1] first entry of each (perspective, block) bin
    uint32_t* multi;              // [1] set when a row has features of two blocks, or one twice
    // per-stage tables of the block scan (ft_scan_max_stages stages)
    uint32_t* stage_rows;         // [stages][32] dft row of each stage slot
    uint32_t* stage_masks;        // [stages][mask words][16] per-feature slot masks
    uint32_t batch, max_active, cols, piece_inputs, n_blocks;
    // optional: also set (and never cleared by the kernels) with *multi, for
    // a batch whose caller said its rows are king-blocked
    uint32_t* multi_sticky;
    // the tables deal a feature group to the block scan's waves round-robin
    // (feature i of a group to wave i % 8) instead of in runs of 16; the
    // matrix-core form needs the runs
    uint32_t dealt;
};

// Columns per dft chunk in the chunk-major layout (one wave of float4 lanes).
constexpr uint32_t kDftChunk = 256;


int32_t launch_ft_forward(const FtForwardArgs& a, hipStream_t stream);
// Schedule keys; with slot_off [2*batch*ft_block_slot_stride(max_active)] and row_bad [2*batch]
// also the block-resident forward's LDS slot offsets and out-of-block row
// flags (FtForwardArgs::slot_off, row_bad).
int32_t launch_king_block_keys(const int32_t* idx_stm, const int32_t* idx_nstm, const int32_t* nnz,
                               uint8_t* keys, uint32_t batch, uint32_t max_active, uint32_t cols,
                               uint32_t piece_inputs, uint32_t n_bins, hipStream_t stream,
                               uint32_t* slot_off = nullptr, uint8_t* row_bad = nullptr);
uint32_t occurrence_key_bits(uint32_t cols);
size_t occurrence_sort_temp_bytes(uint64_t n_items, uint32_t cols);
int32_t launch_occurrence_sort(const OccurrenceSortArgs& a, hipStream_t stream);
int32_t launch_ft_grad_update(const FtGradArgs& a, hipStream_t stream);
// Mask words per schedule entry (0 when the block scan cannot serve piece_inputs).
uint32_t ft_scan_mask_words(uint32_t piece_inputs);
// Stages of 32 rows the block scan's tables hold at most for a batch.
uint64_t ft_scan_max_stages(uint32_t batch, uint32_t n_blocks);
// The block scan's stage tables and the multi flag of a batch (after its
// schedule).
int32_t launch_ft_scan_tables(const FtBlockScan& s, hipStream_t stream);
// FT gradient + update by block scan (chunk-major dft, f32 or f16); the kernel does
// nothing when *s.multi is set.  With fallback, the occurrence-list kernel
// (its lists already sorted) is queued behind it and runs only in that case.
int32_t launch_ft_grad_scan(const FtGradArgs& a, const FtBlockScan& s, hipStream_t stream, bool fallback = true);
// The same gradient and update from an f16 dft as a GEMM of the hit masks
// and the dft rows on the matrix cores (f32 sums in the matrix core's order).
int32_t launch_ft_grad_mfma(const FtGradArgs& a, const FtBlockScan& s, hipStream_t stream, bool fallback = true);
// comb or comb16 (f16) receives the rewritten forward rows; both may be null.
int32_t launch_ft_virtual_fold(const FtGradArgs& a, uint32_t piece_inputs, float* comb, uint16_t* comb16,
                               hipStream_t stream, int layout = kTableRows);
// comb = w + w_virtual (f32), or comb16 = f16(w + w_virtual) when comb is null.
int32_t launch_ft_fold(const float* w, float* comb, uint16_t* comb16, uint32_t ft_in, uint32_t ft_out,
                       uint32_t piece_inputs, hipStream_t stream, int layout = kTableRows);
// dst[i] = f16(src[i]), round to nearest even (cast_f32_to_f16).
int32_t launch_cast_f16(const float* src, uint16_t* dst, uint64_t n, hipStream_t stream);
int32_t launch_ft_reduce(float* grad, uint32_t ft_in, uint32_t ft_out, uint32_t piece_inputs,
                         hipStream_t stream);
int32_t launch_radam(float* w, float* m, float* v, float* g, float* slow, uint64_t n,
                     const OptScalars& s, hipStream_t stream);
int32_t launch_lerp(float* w, float* slow, uint64_t n, float alpha, hipStream_t stream);

}  // namespace tatara
